// Plain BF16 projections of the prompt pass through hipBLASLt, and the SwiGLU
// row kernel that follows the gate/up projection there.
//
// Reference: engine/engine.py:431-450,803 (F.linear -> cuBLAS for the prompt
// pass).  y[M, N] = bf16(x[M, K] . W[N, K]^T) with FP32 accumulation and one
// rounding, as the reference's cuBLAS call and this library's own MFMA GEMM
// compute it; only the order of the K sum differs.  The epilogues the decode
// kernels fuse (residual join, SwiGLU) run as row kernels on the rounded
// output, at the same rounding points: residual = bf16(r + bf16(acc)) in
// q3_add_rmsnorm, act = bf16(bf16(silu(bf16 g)) * bf16 u) here.
//
// The library handle is created once per device on first use (it allocates),
// so the first call must not be inside a stream capture; the prompt pass is
// never captured.
#include <hipblaslt/hipblaslt.h>

#include "q3_common.hpp"
#include "q3.h"

namespace {

constexpr int MAX_DEV = 64;

hipblasLtHandle_t lt_handle() {
    static hipblasLtHandle_t handles[MAX_DEV];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return nullptr;
    if (!handles[dev] && hipblasLtCreate(&handles[dev]) != HIPBLAS_STATUS_SUCCESS) handles[dev] = nullptr;
    return handles[dev];
}

// Owns the descriptors of one call.
struct LtCall {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulPreference_t pref = nullptr;
    ~LtCall() {
        if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        if (d) hipblasLtMatrixLayoutDestroy(d);
        if (b) hipblasLtMatrixLayoutDestroy(b);
        if (a) hipblasLtMatrixLayoutDestroy(a);
        if (desc) hipblasLtMatmulDescDestroy(desc);
    }
};

// out[r, j] = bf16(bf16(silu(g)) * u) with (g, u) = gu[r, 2j], gu[r, 2j + 1]
// (gate/up rows interleaved, as the decode epilogue reads them).  Eight
// outputs per thread: two 16-byte loads, one 16-byte store.
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const bf16_t* __restrict__ gu, bf16_t* __restrict__ out,
                                                          int64_t chunks, int ichunks) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const int64_t r = c / ichunks, j = c % ichunks;
    const bf16_t* src = gu + (r * ichunks + j) * 16;
    const uint4 p0 = *reinterpret_cast<const uint4*>(src);
    const uint4 p1 = *reinterpret_cast<const uint4*>(src + 8);
    const uint32_t w[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t lo = f2bf(silu_bf16(bflo(w[2 * k])) * bfhi(w[2 * k]));
        const uint32_t hi = f2bf(silu_bf16(bflo(w[2 * k + 1])) * bfhi(w[2 * k + 1]));
        o[k] = pack2(lo, hi);
    }
    *reinterpret_cast<uint4*>(out + (r * ichunks + j) * 8) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace

extern "C" int q3_gemm_lt(const bf16_t* x, int ldx, const bf16_t* w, int M, int N, int K, bf16_t* y, int ldy,
                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (M < 1 || N < 1 || K < 1 || ldx < K || ldy < N || !x || !w || !y || (workspace_bytes && !workspace))
        return (int)hipErrorInvalidValue;
    hipblasLtHandle_t h = lt_handle();
    if (!h) return (int)hipErrorNotInitialized;
    // Column-major view: D[N, M] (ld ldy) = op_T(A = W, stored K x N, ld K) * (B = x, stored K x M, ld ldx).
    LtCall c;
    const hipblasOperation_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
    const uint64_t ws = workspace_bytes;
    hipblasLtMatmulHeuristicResult_t best;
    int found = 0;
    const bool ok =
        hipblasLtMatmulDescCreate(&c.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulDescSetAttribute(c.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulDescSetAttribute(c.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatrixLayoutCreate(&c.a, HIP_R_16BF, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatrixLayoutCreate(&c.b, HIP_R_16BF, K, M, ldx) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatrixLayoutCreate(&c.d, HIP_R_16BF, N, M, ldy) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulPreferenceCreate(&c.pref) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulPreferenceSetAttribute(c.pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulAlgoGetHeuristic(h, c.desc, c.a, c.b, c.d, c.d, c.pref, 1, &best, &found) ==
            HIPBLAS_STATUS_SUCCESS;
    if (!ok || found < 1 || best.workspaceSize > workspace_bytes) return (int)hipErrorNotSupported;
    const float alpha = 1.f, beta = 0.f;
    if (hipblasLtMatmul(h, c.desc, &alpha, w, c.a, x, c.b, &beta, y, c.d, y, c.d, &best.algo, workspace,
                        workspace_bytes, stream) != HIPBLAS_STATUS_SUCCESS)
        return (int)hipErrorLaunchFailure;
    return 0;
}

extern "C" int q3_swiglu_rows(const bf16_t* gu, bf16_t* out, int rows, int I, hipStream_t stream) {
    if (rows < 1 || I < 8 || I % 8 || !gu || !out ||
        ((reinterpret_cast<uintptr_t>(gu) | reinterpret_cast<uintptr_t>(out)) & 15))
        return (int)hipErrorInvalidValue;
    const int64_t chunks = (int64_t)rows * (I / 8);
    Q3_LAUNCH(swiglu_rows_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, gu, out, chunks,
              I / 8);
    Q3_CHECK_LAUNCH();
}
