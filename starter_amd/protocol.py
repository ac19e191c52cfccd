"""The contest's streaming protocol: an engine in a child process, timed by a client through a pipe.

Reference ``QWEN_ENGINE_CONTRACT.md`` "What is measured" and "Gates and failure",
``AGENTS.md`` "The gates": for each workload the judge starts the engine in a
fresh process, lets it load and warm up on a prompt of the workload's shape,
then writes each sample's prompt ids to it and reads the token stream back; a
separate trusted process holds the clock.  Time to first token is when the
first step arrives, time per output token is the rest of the stream over the
remaining steps, total time is the whole stream; tokens/s is
``batch * output tokens / total``.  Native Qwen is timed by the same clock
through the same pipe.  A workload fails on a token outside the tie margin,
TTFT or TPOT above 1.10x native's (medians), peak GPU memory above 90% of the
device, more than 25% spread across the samples, load plus warmup above 300 s,
a sample above 300 s, or the wrong number of steps or tokens.

Wire format (one JSON object per line, both directions):
  child -> client  {"ready": true, "load_s": s, "warmup_s": s}   after load + warmup
  client -> child  {"ids": [[...], ...], "new": N}                one sample
  child -> client  {"step": [id, ...]}                            N times, flushed each
  child -> client  {"done": true, "peak_bytes": b, "reserved_bytes": b, "used_bytes": b,
                   "device_bytes": b}
  client -> child  {"quit": true}
Anything the engine prints goes to stderr; stdout carries only these lines.

``serve`` is the child side for any object with ``generate(ids, new)``;
``python -m starter_amd.protocol MODEL_PATH BATCH PROMPT NEW`` serves this
package's ``Engine``.  ``run_workload`` is the client side; ``gates`` applies the
contest's limits to what it measured.
"""

from __future__ import annotations

import json
import queue
import statistics
import subprocess
import sys
import threading
import time
from dataclasses import dataclass, field

#: Reference QWEN_ENGINE_CONTRACT.md "Gates and failure" / AGENTS.md "The gates".
LATENCY_RATIO_LIMIT = 1.10
MEMORY_FRACTION_LIMIT = 0.90
SPREAD_LIMIT = 0.25
LOAD_BUDGET_S = 300.0
SAMPLE_BUDGET_S = 300.0


def _emit(out, obj) -> None:
    out.write(json.dumps(obj) + "\n")
    out.flush()


def _memory() -> tuple[int, int, int]:
    """(bytes torch's caching allocator has reserved at its peak, bytes in use on
    the whole device now, device bytes); 0s without a GPU.  The device figure
    (``hipMemGetInfo``: total - free) also holds what the allocator does not see
    -- the HIP context, code objects, graph memory, a library's static device
    arrays -- and anything else on the device."""
    try:
        import torch
        if torch.cuda.is_available():
            free, total = torch.cuda.mem_get_info(0)
            return torch.cuda.max_memory_reserved(), total - free, total
    except Exception:  # noqa: BLE001 - a server without torch / GPU reports no memory
        pass
    return 0, 0, 0


def serve(engine, warmup_ids: list[list[int]], warmup_new: int, inp=None, out=None,
          load_s: float = 0.0) -> None:
    """Child side: warm up on a prompt of the workload's shape, announce
    readiness, then answer samples until told to quit (or stdin closes).

    Each sample's ``done`` line reports ``peak_bytes``: the larger of the
    allocator's reserved peak and the device's used bytes, read after the
    warmup and after every sample so far (``_memory``)."""
    inp = inp if inp is not None else sys.stdin
    out = out if out is not None else sys.stdout
    t0 = time.perf_counter()
    for _ in engine.generate(warmup_ids, warmup_new):
        pass
    _, used_peak, _ = _memory()
    _emit(out, {"ready": True, "load_s": round(load_s, 3), "warmup_s": round(time.perf_counter() - t0, 3)})
    for line in inp:
        msg = json.loads(line)
        if msg.get("quit"):
            break
        for step in engine.generate(msg["ids"], msg["new"]):
            _emit(out, {"step": [int(t) for t in step]})
        reserved, used, device = _memory()
        used_peak = max(used_peak, used)
        _emit(out, {"done": True, "peak_bytes": max(reserved, used_peak), "reserved_bytes": reserved,
                    "used_bytes": used_peak, "device_bytes": device})


@dataclass
class SampleTiming:
    steps: list[list[int]]
    arrivals: list[float]       # seconds from the prompt write to each step line
    peak_bytes: int
    device_bytes: int

    @property
    def ttft(self) -> float:
        return self.arrivals[0]

    @property
    def total(self) -> float:
        return self.arrivals[-1]

    @property
    def tpot(self) -> float:
        n = len(self.arrivals)
        return (self.total - self.ttft) / (n - 1) if n > 1 else 0.0


@dataclass
class WorkloadRun:
    batch: int
    new_tokens: int
    load_s: float
    warmup_s: float
    samples: list[SampleTiming] = field(default_factory=list)

    def summary(self) -> dict:
        totals = [s.total for s in self.samples]
        med = statistics.median(totals)
        return {
            "samples": len(self.samples),
            "total_s_median": med,
            "ttft_s_median": statistics.median(s.ttft for s in self.samples),
            "tpot_s_median": statistics.median(s.tpot for s in self.samples),
            "tokens_per_s": self.batch * self.new_tokens / med,
            "spread": (max(totals) - min(totals)) / med if med > 0 else 0.0,
            "peak_bytes": max(s.peak_bytes for s in self.samples),
            "device_bytes": max(s.device_bytes for s in self.samples),
            "load_s": self.load_s,
            "warmup_s": self.warmup_s,
        }


class ProtocolError(RuntimeError):
    pass


class _Lines:
    """The child's stdout lines, read by a daemon thread into a queue, so that
    the client can wait for the next one with a deadline (a child that hangs
    or stops writing must not block the clock's owner)."""

    def __init__(self, stream):
        self.q: queue.Queue = queue.Queue()
        threading.Thread(target=self._pump, args=(stream,), daemon=True).start()

    def _pump(self, stream) -> None:
        try:
            for line in stream:
                self.q.put(line)
        finally:
            self.q.put(None)

    def get(self, proc, deadline: float, what: str) -> dict:
        remaining = deadline - time.perf_counter()
        try:
            line = self.q.get(timeout=max(remaining, 0.0))
        except queue.Empty:
            raise ProtocolError(f"the engine process exceeded its time budget ({what})") from None
        if line is None:
            raise ProtocolError(f"the engine process ended (exit {proc.poll()}) before answering ({what})")
        if time.perf_counter() > deadline:
            raise ProtocolError(f"the engine process exceeded its time budget ({what})")
        return json.loads(line)


def run_workload(cmd: list[str], prompts: list[list[list[int]]], new_tokens: int, env=None,
                 cwd=None, load_budget_s: float = LOAD_BUDGET_S,
                 sample_budget_s: float = SAMPLE_BUDGET_S) -> WorkloadRun:
    """Client side: start ``cmd`` (a child that speaks this protocol), wait for
    it to load and warm up, then time each prompt's stream.  The clock is this
    process's; the child's own claims are used only for its memory figures.
    A child that misses the load or a sample budget is killed and the run
    raises ``ProtocolError``."""
    batch = len(prompts[0])
    proc = subprocess.Popen(cmd, stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True, bufsize=1,
                            env=env, cwd=cwd)
    lines = _Lines(proc.stdout)
    try:
        t0 = time.perf_counter()
        hello = lines.get(proc, t0 + load_budget_s, "load and warmup")
        if not hello.get("ready"):
            raise ProtocolError(f"expected the ready line, got {hello}")
        run = WorkloadRun(batch, new_tokens, hello.get("load_s", 0.0), hello.get("warmup_s", 0.0))
        for ids in prompts:
            if len(ids) != batch:
                raise ProtocolError("every sample of a workload has the same batch")
            start = time.perf_counter()
            proc.stdin.write(json.dumps({"ids": ids, "new": new_tokens}) + "\n")
            proc.stdin.flush()
            steps, arrivals = [], []
            while True:
                msg = lines.get(proc, start + sample_budget_s, f"sample {len(run.samples)}")
                if "step" in msg:
                    arrivals.append(time.perf_counter() - start)
                    steps.append(msg["step"])
                    continue
                if msg.get("done"):
                    break
                raise ProtocolError(f"unexpected line {msg}")
            if len(steps) != new_tokens or any(len(s) != batch for s in steps):
                raise ProtocolError(f"wrong stream shape: {len(steps)} steps of "
                                    f"{sorted({len(s) for s in steps})} ids, wanted {new_tokens} of {batch}")
            run.samples.append(SampleTiming(steps, arrivals, int(msg.get("peak_bytes", 0)),
                                            int(msg.get("device_bytes", 0))))
        proc.stdin.write(json.dumps({"quit": True}) + "\n")
        proc.stdin.flush()
        proc.wait(timeout=60)
        return run
    finally:
        if proc.poll() is None:
            proc.kill()
            proc.wait()


def gates(candidate: dict, native: dict, failing_tokens: int = 0) -> dict:
    """The contest's per-workload gates on two ``WorkloadRun.summary()`` dicts
    (the candidate's and native's, timed by the same client).  Returns each
    gate's measured ratio or value, its limit, and whether it passed."""
    checks = {
        "tokens": {"value": failing_tokens, "limit": 0, "ok": failing_tokens == 0},
        "ttft": {"value": candidate["ttft_s_median"] / native["ttft_s_median"], "limit": LATENCY_RATIO_LIMIT},
        "tpot": {"value": candidate["tpot_s_median"] / native["tpot_s_median"] if native["tpot_s_median"] else 0.0,
                 "limit": LATENCY_RATIO_LIMIT},
        "memory": {"value": candidate["peak_bytes"] / candidate["device_bytes"] if candidate["device_bytes"] else 0.0,
                   "limit": MEMORY_FRACTION_LIMIT},
        "spread": {"value": candidate["spread"], "limit": SPREAD_LIMIT},
        "load": {"value": candidate["load_s"] + candidate["warmup_s"], "limit": LOAD_BUDGET_S},
    }
    for name in ("ttft", "tpot", "memory", "spread", "load"):
        checks[name]["ok"] = checks[name]["value"] <= checks[name]["limit"]
    checks["passed"] = all(c["ok"] for c in checks.values() if isinstance(c, dict))
    return checks


def main(argv: list[str]) -> int:
    """Child process for this package's engine: load MODEL_PATH, warm up on a
    BATCH x PROMPT prompt with NEW tokens, then serve samples on stdin/stdout."""
    if len(argv) != 4:
        print("usage: python -m starter_amd.protocol MODEL_PATH BATCH PROMPT NEW", file=sys.stderr)
        return 2
    model_path, batch, prompt, new = argv[0], int(argv[1]), int(argv[2]), int(argv[3])
    real_stdout = sys.stdout
    sys.stdout = sys.stderr  # the engine's own prints must not reach the pipe
    t0 = time.perf_counter()
    from .engine import Engine
    engine = Engine(model_path)
    load_s = time.perf_counter() - t0
    warm = [[(7 * r + 13 * t) % engine.VOCAB for t in range(prompt)] for r in range(batch)]
    serve(engine, warm, new, out=real_stdout, load_s=load_s)
    return 0


if __name__ == "__main__":
    raise SystemExit(main(sys.argv[1:]))
