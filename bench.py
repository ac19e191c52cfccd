"""Decode throughput of the MI355X Qwen3-4B engine on one GPU.

    python bench.py [--steps K] [--warmup W] [--config 2] [--gpus 1]

A step is one decode step of the whole batch (one token per sequence): one
replay of the captured hipGraph.  The workload is BASELINE config 2 by default
(seeded Qwen3-4B BF16, batch 1, prompt 1024, 512 new tokens): the prompt is
prefilled (untimed), W steps warm up, then exactly K steps are timed with HIP
events on the engine's stream, bracketed by device synchronisation.  Inputs
(weights, KV cache, token buffers) are resident in HBM throughout.

Printed: one JSON line with decode tokens/s (value), ms/step, the whole-step
HBM roofline fraction (weights + KV bytes per step over 8 TB/s), the dominant
kernel's roofline (the gate/up GEMV, timed live over the same weights), and
the CPU baseline: the CPU oracle (a PyTorch restatement of the reference's
eager path) timed on this host's cores on a bounded sample of the workload.
Beside them, ``prefill``: the prompt's forward (warm, second call) timed with
HIP events, as tokens/s and as a fraction of dense BF16 MFMA peak.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import pathlib
import sys
import time

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense BF16
KV_BYTES_PER_TOKEN = 36 * 2 * 8 * 128 * 2  # K and V, all layers, one position


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def weight_bytes(eng) -> int:
    total = eng.embed.numel() * 2 + eng.final_norm.numel() * 2
    for L in eng.layers:
        total += sum(t.numel() * 2 for t in L.values())
    return total


def prefill_figures(B: int, P: int, ms: float) -> dict:
    """Prefill of B prompts of P tokens in `ms`: algorithmic flop are the
    projections (2 flop per weight per token, LM head at the last position
    only) plus causal attention (QK^T and PV: 4*D flop per (query, key <=
    query) pair per query head), against 2.5 PFLOP/s dense BF16 MFMA."""
    L, H, I, Hq, Hkv, D, V = 36, 2560, 9728, 32, 8, 128, 151936
    per_layer = (Hq + 2 * Hkv) * D * H + H * Hq * D + 2 * I * H + H * I
    gemm = 2.0 * B * P * L * per_layer + 2.0 * B * V * H
    attn = 4.0 * D * B * Hq * L * P * (P + 1) / 2
    tflops = (gemm + attn) / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 3), "tokens_per_s": round(B * P / (ms * 1e-3), 1), "bound": "mfma",
            "achieved": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_PEAK_TFLOPS, 4), "flop": int(gemm + attn)}


def dominant_kernel_roofline(eng, config: int, reps: int = 20) -> dict:
    """Average duration of the gate/up GEMV (norm prologue + SwiGLU epilogue)
    over all 36 layers' weights, captured as one graph and replayed.

    Bytes per launch (algorithmic): the [2I, H] BF16 weight, plus B rows of the
    residual in, B rows of I activations out, and the [H] gain.
    """
    import torch
    from starter_amd import _lib
    from starter_amd._lib import call

    B, H, I = eng.batch, eng.HIDDEN, eng.INTER
    s = eng.stream.cuda_stream
    if not eng.small:
        return {}
    call("q3_graph_begin", s)
    for L in eng.layers:
        call("q3_gemv", _lib.X_NORM, eng.resid.data_ptr(), H, None, L["post_ln"].data_ptr(), eng.EPS, None,
             L["gate_up"].data_ptr(), B, 2 * I, H, _lib.EPI_SWIGLU, eng.act.data_ptr(), I, None, None,
             None, None, None, s)
    ex = ctypes.c_void_p()
    call("q3_graph_end", s, ctypes.byref(ex))
    try:
        call("q3_graph_launch", ex.value, s)
        eng.stream.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(eng.stream)
        for _ in range(reps):
            call("q3_graph_launch", ex.value, s)
        stop.record(eng.stream)
        stop.synchronize()
        ms = start.elapsed_time(stop) / (reps * len(eng.layers))
    finally:
        call("q3_graph_destroy", ex.value)
    nbytes = 2 * I * H * 2 + B * H * 2 + B * I * 2 + H * 2
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "kernel": "gemv_dot2 gate_up (norm prologue, SwiGLU epilogue)",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(f"gemv_gate_up_config{config}_b{B}_traffic.txt"),
            "bytes_per_launch": nbytes, "us_per_launch": round(ms * 1e3, 2)}


def measured_traffic(name: str):
    """HBM bytes per launch from a committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary
    (``profiles/<name>``, counters scaled by a plain copy of known size), or None
    when no such measurement exists for this kernel and workload."""
    path = pathlib.Path(__file__).resolve().parent / "profiles" / name
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def cpu_baseline(wl, ckpt, budget_s: float = 20.0) -> dict:
    """The CPU oracle's decode steps at this workload's cache shape (pre-filled cache)."""
    import torch
    from oracle.qwen3_cpu import Qwen3Oracle
    from starter_amd.checkpoint import load_checkpoint

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cfg, tensors = load_checkpoint(ckpt)
    orc = Qwen3Oracle(cfg, tensors, torch.bfloat16)
    del tensors
    B, P = wl.batch, wl.prompt
    orc.reset(B, P + wl.new_tokens)
    g = torch.Generator().manual_seed(0)
    for ck, cv in zip(orc.cache_k, orc.cache_v):  # decode cost does not depend on the values
        ck[:, :, :P].copy_(torch.randn(ck[:, :, :P].shape, generator=g))
        cv[:, :, :P].copy_(torch.randn(cv[:, :, :P].shape, generator=g))
    tok = torch.tensor(wl.prompt_ids(), dtype=torch.int64)[:, -1:]
    orc.forward(tok, P)  # warm
    steps, t0 = 0, time.perf_counter()
    while True:
        orc.forward(tok, P + 1 + steps)
        steps += 1
        if time.perf_counter() - t0 > budget_s or P + 2 + steps >= P + wl.new_tokens:
            break
    dt = time.perf_counter() - t0
    return {"value": round(B * steps / dt, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "ms_per_step": round(dt / steps * 1e3, 1),
            "sample": f"{steps} decode steps of {wl.name} (B={B}) at context {P + 1}..{P + steps} "
                      f"on a pre-filled cache; CPU oracle (PyTorch BF16, oracle/qwen3_cpu.py)"}


def copy_probe(nbytes: int = 1 << 30) -> int:
    """A plain copy of ``nbytes`` (reads nbytes, writes nbytes), three times.

    Under ``rocprofv3 --pmc FETCH_SIZE`` (or WRITE_SIZE) its per-dispatch
    reading against the known 1 GiB gives the counter's scale on this device.
    """
    import torch

    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy probe: 3 copies of {nbytes} bytes")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--ckpt-dir", default=os.environ.get("Q3_CKPT_DIR", "/tmp/q3_seeded_qwen3_4b"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (3 times): the known-size "
                         "kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(one MI355X per box); run with --gpus 1", file=sys.stderr)
        return 2
    if args.copy_probe:
        return copy_probe()

    sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))
    import torch
    from starter_amd.checkpoint import ensure_seeded_checkpoint
    from starter_amd.engine import Engine
    from starter_amd.workloads import MODEL, MODEL_SEED, WORKLOADS

    wl = WORKLOADS[args.config]
    B, P, N = wl.batch, wl.prompt, wl.new_tokens
    K, W = args.steps, args.warmup
    if W + K > N - 1:
        K = max(1, N - 1 - W)
        log(f"steps clamped to {K}: {wl.name} has {N - 1} decode steps")

    t0 = time.time()
    ckpt = ensure_seeded_checkpoint(args.ckpt_dir, MODEL, MODEL_SEED)
    log(f"checkpoint ready in {time.time() - t0:.1f}s")
    eng = Engine(str(ckpt))
    ids = torch.tensor(wl.prompt_ids(), dtype=torch.int64, device="cuda:0")
    eng._ensure_shape(B, P, N)
    t0 = time.time()
    eng._forward_prefill(ids, P)
    eng.stream.synchronize()
    log(f"prefill {B}x{P} (first call) in {time.time() - t0:.2f}s")
    # The prompt again, warm and timed on the engine's stream (the time to the
    # first token's logits); it rewrites the same cache rows.
    p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    p0.record(eng.stream)
    logits = eng._forward_prefill(ids, P)
    p1.record(eng.stream)
    p1.synchronize()
    prefill = prefill_figures(B, P, p0.elapsed_time(p1))
    log(f"prefill {B}x{P}: {prefill['ms']} ms, {prefill['tokens_per_s']} tok/s, "
        f"{prefill['achieved']} TFLOP/s ({prefill['frac']:.1%} of dense BF16 MFMA)")
    eng._begin_decode(logits, P)
    eng.stream.synchronize()

    for _ in range(W):
        eng._decode_step()
    torch.cuda.synchronize()
    # One event between consecutive replays: the mean over the K steps is the
    # headline, the median of the per-step durations is reported beside it.
    events = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    events[0].record(eng.stream)
    for k in range(K):
        eng._decode_step()
        events[k + 1].record(eng.stream)
    torch.cuda.synchronize()
    eng._check_step()
    ms_step = events[0].elapsed_time(events[K]) / K
    per_step = sorted(events[k].elapsed_time(events[k + 1]) for k in range(K))
    ms_median = per_step[K // 2] if K % 2 else 0.5 * (per_step[K // 2 - 1] + per_step[K // 2])
    value = B * K / (ms_step * K / 1e3)

    wbytes = weight_bytes(eng)
    # Decode step d (0-based) attends over context P + d + 1 and appends one position.
    ctx_mean = P + W + (K + 1) / 2
    step_bytes = wbytes + B * ctx_mean * KV_BYTES_PER_TOKEN + B * KV_BYTES_PER_TOKEN
    step_gbs = step_bytes / (ms_step * 1e-3) / 1e9
    roof = dominant_kernel_roofline(eng, args.config)
    log(f"{ms_step:.3f} ms/step, {value:.1f} tok/s, step HBM {step_gbs:.0f} GB/s "
        f"({step_gbs / HBM_PEAK_GBS:.1%}); gate_up GEMV {roof.get('achieved')} GB/s")

    cpu = None
    if not args.no_cpu_baseline:
        del eng
        torch.cuda.empty_cache()
        cpu = cpu_baseline(wl, ckpt)
        log(f"cpu baseline {cpu}")

    line = {
        "metric": "decode tokens/s (Qwen3-4B bf16 greedy, seeded random init)",
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_median": round(ms_median, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) BF16 weights of the Qwen3-4B shapes, uniform random prompt ids)",
        "config": {"workload": wl.name, "batch": B, "prompt": P, "new_tokens": N},
        "step_roofline": {"bound": "hbm", "bytes_per_step": int(step_bytes),
                          "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "prefill": prefill,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
