// hipGraph capture / replay of one decode step, and error names.
//
// Reference: engine/engine.py:1029-1065 (_capture / _decode_step, a CUDA graph
// captured after warm steps and replayed once per token).  Capture records
// every launch enqueued on `stream` between q3_graph_begin and q3_graph_end;
// the launchers in this library neither allocate nor synchronise, so a whole
// decode step records cleanly.  Thread-local capture mode keeps launches from
// other host threads out of the graph.
#include "q3_common.hpp"
#include "q3.h"

extern "C" const char* q3_error_string(int code) {
    return hipGetErrorString(static_cast<hipError_t>(code));
}

extern "C" int q3_graph_begin(hipStream_t stream) {
    return (int)hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
}

extern "C" int q3_graph_end(hipStream_t stream, void** exec_out) {
    if (!exec_out) return (int)hipErrorInvalidValue;
    hipGraph_t graph = nullptr;
    hipError_t rc = hipStreamEndCapture(stream, &graph);
    if (rc != hipSuccess) return (int)rc;
    hipGraphExec_t exec = nullptr;
    rc = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (rc != hipSuccess) return (int)rc;
    *exec_out = exec;
    return 0;
}

extern "C" int q3_graph_launch(void* exec, hipStream_t stream) {
    if (!exec) return (int)hipErrorInvalidValue;
    return (int)hipGraphLaunch(static_cast<hipGraphExec_t>(exec), stream);
}

extern "C" int q3_graph_destroy(void* exec) {
    if (!exec) return 0;
    return (int)hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec));
}
