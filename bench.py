"""Decode throughput of the MI355X Qwen3-4B engine on one GPU.

    python bench.py [--steps K] [--warmup W] [--config 2] [--extra-configs 1,3,4,5] [--gpus 1]
    python bench.py --kernel {gemm_gate_up,gemm_qkv,gemm_o,gemm_down,attn_prefill} --config N [--launches L]

A step is one decode step of the whole batch (one token per sequence): one
replay of the captured hipGraph.  The headline workload is BASELINE config 2
(seeded Qwen3-4B BF16, batch 1, prompt 1024, 512 new tokens): the prompt is
prefilled (untimed), W steps warm up, then exactly K steps are timed with HIP
events on the engine's stream, bracketed by device synchronisation.  Inputs
(weights, KV cache, token buffers) are resident in HBM throughout.  The timed
steps are decode steps W .. W+K-1 of the workload (contexts P+W+1 ..
P+W+K), and the step's bytes are counted at those contexts; a workload with
fewer than W+K decode steps clamps K.

Printed: one JSON line with decode tokens/s (value), ms/step, the whole-step
HBM roofline fraction (weights + KV bytes per step over 8 TB/s), the dominant
kernel's roofline (timed live, HIP events on the engine's stream, over a
graph of its 36 layer launches at the workload's shapes), and the CPU
baseline: the reference engine's eager CPU decode step
(oracle/ref_cpu_path.py) timed on this host's cores on a bounded sample of the
workload (at least 8 decode steps at the workload's real cache shape; every
decode step of config 1).  Beside them, ``prefill``: the prompt's forward
(warm, second call) timed with HIP events, as tokens/s and as a fraction of
dense BF16 MFMA peak; and ``workloads``: the same figures for the other
BASELINE configs (1, 3, 4 and 5 by default), each timed over the same
decode steps W .. W+K-1 of its own run.
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


def _graph_ms(eng, enqueue, reps: int) -> float:
    """Mean device time (ms) of one replay of the graph that ``enqueue()``
    captures on the engine's stream, replayed ``reps`` times between two HIP
    events on that stream."""
    import torch
    from starter_amd._lib import call

    s = eng.stream.cuda_stream
    call("q3_graph_begin", s)
    try:
        with torch.cuda.stream(eng.stream):
            enqueue()
    finally:
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
        return start.elapsed_time(stop) / reps
    finally:
        call("q3_graph_destroy", ex.value)


def time_layer_graph(eng, enqueue_layer, reps: int = 20, clear_exchange: bool = False) -> float:
    """Mean device time (ms) of one launch: ``enqueue_layer(i, L)`` for every
    layer captured as one graph, timed over ``reps`` replays.  With
    ``clear_exchange`` each replay first zeroes the fused launches' exchange
    words, so that no launch finds words a previous replay left at the same
    (position, layer) and every wait in it is a real one; the fill kernels' own
    time, taken from a graph of the fills alone, is subtracted."""
    def layers():
        if clear_exchange:
            eng._clear_exchange()
        for i, L in enumerate(eng.layers):
            enqueue_layer(i, L)

    ms = _graph_ms(eng, layers, reps)
    if clear_exchange:
        ms -= _graph_ms(eng, eng._clear_exchange, reps)
    return ms / len(eng.layers)


def kernel_line(name: str, nbytes: int, ms: float, traffic_file: str) -> dict:
    achieved = nbytes / (ms * 1e-3) / 1e9
    line = {"bound": "hbm", "kernel": name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(traffic_file),
            "bytes_per_launch": int(nbytes), "us_per_launch": round(ms * 1e3, 2)}
    note = measured_traffic(traffic_file, "traffic_note")
    if note:
        line["traffic_note"] = note
    return line


def kernel_rooflines(eng, wl) -> list[dict]:
    """The step's heaviest kernels, each timed live at the workload's shapes.

    B <= 4: the gate/up GEMV (norm prologue, SwiGLU epilogue); bytes per launch
    are the [2I, H] BF16 weight, B rows of the residual in, B rows of I
    activations out and the [H] gain.  At one row also the fused launch of
    q|k|v projection, attention, split merge and o projection + residual join:
    the q|k|v and o weights, K+V of every cached key at the current position,
    the residual read and written, the gains and the appended key and value
    (the gate/up rows it warms into L2 are not counted); where that launch
    also runs the previous layer's down projection (every layer but the
    first), its weights and input row too, averaged over the layers.  B = 5..64: decode attention at the
    current position (K+V of every cached key of every (sequence, KV head),
    the q|k|v rows in, the output rows out, the appended key and value) and
    the MFMA gate/up projection (weight, input rows, activations out).
    Sorted by time per launch, heaviest first.
    """
    from starter_amd import _lib
    from starter_amd._lib import call

    B, H, I = eng.batch, eng.HIDDEN, eng.INTER
    s = eng.stream.cuda_stream
    # Counter summaries: the projections' launches depend only on the batch
    # (same weights and shapes at every config), attention's on the context too.
    tag = f"config{wl.number}_b{B}"
    out = []
    gate_up = 2 * I * H * 2 + B * H * 2 + B * I * 2
    if eng.small:
        ms = time_layer_graph(eng, lambda i, L: call(
            "q3_gemv", _lib.X_NORM, eng.resid.data_ptr(), H, None, L["post_ln"].data_ptr(), eng.EPS, None,
            L["gate_up"].data_ptr(), B, 2 * I, H, _lib.EPI_SWIGLU, eng.act.data_ptr(), I, None, None, None, None,
            None, 0, s))
        out.append(kernel_line("gemv_dot2 gate_up (norm prologue, SwiGLU epilogue)", gate_up + H * 2, ms,
                               f"gemv_gate_up_b{B}_traffic.txt"))
        if eng.qkv_attn_o:
            ctx = int(eng.g_pos.item()) + 1
            Hkv, Hq, D = eng.KV_HEADS, eng.HEADS, eng.HEAD_DIM
            fused = (eng.qkv_size * H * 2 + H * Hq * D * 2 + B * Hkv * ctx * D * 2 * 2 + 2 * B * H * 2
                     + (H + 2 * D) * 2 + B * Hkv * D * 2 * 2)
            name = f"q|k|v GEMV + attention + {eng.splits}-split merge + o GEMV + residual"
            if eng.down_attn:
                # Layers 1..L-1 also stream the previous layer's down weights
                # and its input row: the mean over the timed layers.
                L_ = len(eng.layers)
                fused += (L_ - 1) * (H * I * 2 + B * I * 2) // L_
                name = f"down GEMV + residual (layers 1-{L_ - 1}) + " + name
            ms = time_layer_graph(eng, eng._qkv_attn_layer, clear_exchange=True)
            out.append(kernel_line(f"qkv_attn ({name}, one launch, context {ctx})", fused, ms,
                                   f"qkv_attn_{tag}_traffic.txt"))
    elif eng.skinny:
        T = lambda w: eng.tiled[id(w)].data_ptr()  # noqa: E731
        ms = time_layer_graph(eng, lambda i, L: call(
            "q3_skinny_tiled", eng.nbuf.data_ptr(), H, T(L["gate_up"]), B, 2 * I, H, _lib.EPI_SWIGLU,
            eng.act.data_ptr(), I, eng.skinny_ws.data_ptr(), s))
        line = kernel_line("skinny MFMA gate_up (SwiGLU epilogue)", gate_up, ms, f"skinny_gate_up_b{B}_traffic.txt")
        line["mfma_tflops"] = round(2.0 * B * 2 * I * H / (ms * 1e-3) / 1e12, 1)
        out.append(line)
        ctx = int(eng.g_pos.item()) + 1
        s_qkv = call("q3_skinny_splits", B, eng.qkv_size, H)
        layer_stride = eng.cache_k[0].numel() * 2
        kc0, vc0 = eng.cache_k.data_ptr(), eng.cache_v.data_ptr()
        ms = time_layer_graph(eng, lambda i, L: eng._attention(
            i, L, (None, eng.qkv_size, eng.skinny_ws.data_ptr(), s_qkv), kc0 + i * layer_stride,
            vc0 + i * layer_stride), clear_exchange=eng.attn_fused)
        Hkv, Hq, D = eng.KV_HEADS, eng.HEADS, eng.HEAD_DIM
        attn = B * Hkv * ctx * D * 2 * 2 + B * eng.qkv_size * 2 + B * Hq * D * 2 + B * Hkv * D * 2 * 2
        out.append(kernel_line(f"attn_decode (split-K GQA, {eng.splits} split(s), context {ctx})", attn, ms,
                               f"attn_decode_{tag}_traffic.txt"))
    return sorted(out, key=lambda k: -k["us_per_launch"])


def measured_traffic(name: str, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch from a committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary
    (``profiles/<name>``, counters scaled by a plain copy of known size), or None
    when no such measurement exists for this kernel and workload.  With
    ``key="traffic_note"``: the summary's one-line reading of that figure, if any."""
    path = pathlib.Path(__file__).resolve().parent / "profiles" / name
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(key + ":"):
            value = line.split(":", 1)[1].strip()
            return int(value) if key == "traffic_bytes_per_launch" else value
    return None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(ref, wl, budget_s: float, min_steps: int = 8) -> dict:
    """The reference engine's eager CPU decode step (``ref``, an
    oracle.ref_cpu_path.RefCpuDecode) at this workload's cache shape: one warm
    step, then steps until ``budget_s`` is spent and at least ``min_steps``
    ran, or every decode step of the workload.  The cache's prompt positions
    are zero except the first few: a decode step's cost does not depend on the
    cache's values."""
    import torch

    B, P, N = wl.batch, wl.prompt, wl.new_tokens
    ref.reset(B, P + N)
    g = torch.Generator().manual_seed(0)
    head = min(P, 64)
    for ck, cv in zip(ref.cache_k, ref.cache_v):
        ck[:, :, :head].copy_(torch.randn(ck[:, :, :head].shape, generator=g))
        cv[:, :, :head].copy_(torch.randn(cv[:, :, :head].shape, generator=g))
    tok = torch.tensor(wl.prompt_ids(), dtype=torch.int64)[:, -1:]
    tok = ref.step(tok, P)  # warm: decode step 0
    available = N - 2  # decode steps 1 .. N-2 (step k attends over P + k + 1 keys)
    steps, t0 = 0, time.perf_counter()
    while steps < available:
        tok = ref.step(tok, P + 1 + steps)
        steps += 1
        if time.perf_counter() - t0 > budget_s and steps >= min(min_steps, available):
            break
    dt = time.perf_counter() - t0
    ref.cache_k = ref.cache_v = None
    cores = torch.get_num_threads()
    whole = "every further decode step" if steps == available else f"{steps} decode steps"
    return {"value": round(B * steps / dt, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu": cpu_model(), "ms_per_step": round(dt / steps * 1e3, 1),
            "sample": f"{whole} of {wl.name} (B={B}) at context {P + 2}..{P + 1 + steps} after one "
                      f"warm step, on a pre-filled cache at the workload's real shape; the reference engine's "
                      f"eager CPU path restated in PyTorch BF16 (oracle/ref_cpu_path.py: fused qkv and gate/up "
                      f"GEMMs, repeat-KV SDPA over the full capacity with an additive mask), {cores} threads"}


def run_workload(eng, wl, K: int, W: int) -> dict:
    """Prefill (first call untimed, second timed), W warm steps, K timed steps."""
    import torch

    B, P, N = wl.batch, wl.prompt, wl.new_tokens
    if W + K > N - 1:
        K = max(1, N - 1 - W)
        log(f"{wl.name}: steps clamped to {K} ({N - 1} decode steps)")
    ids = torch.tensor(wl.prompt_ids(), dtype=torch.int64, device="cuda:0")
    eng._ensure_shape(B, P, N)
    t0 = time.time()
    eng._forward_prefill(ids, P)
    eng.stream.synchronize()
    log(f"{wl.name}: prefill (first call) in {time.time() - t0:.2f}s")
    # The prompt again, warm and timed on the engine's stream (the time to the
    # first token's logits); it rewrites the same cache rows.
    p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    p0.record(eng.stream)
    logits = eng._forward_prefill(ids, P)
    p1.record(eng.stream)
    p1.synchronize()
    prefill = prefill_figures(B, P, p0.elapsed_time(p1))
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
    kernels = kernel_rooflines(eng, wl)
    log(f"{wl.name}: {ms_step:.3f} ms/step, {value:.1f} tok/s, step HBM {step_gbs:.0f} GB/s "
        f"({step_gbs / HBM_PEAK_GBS:.1%}); " + "; ".join(f"{k['kernel']} {k['achieved']} GB/s" for k in kernels)
        + f"; prefill {prefill['ms']} ms ({prefill['frac']:.1%} of dense BF16 MFMA)")
    return {
        "value": round(value, 2), "unit": "tokens/s", "steps": K, "warmup": W,
        "ms_per_step": round(ms_step, 4), "ms_per_step_median": round(ms_median, 4),
        "config": {"workload": wl.name, "batch": B, "prompt": P, "new_tokens": N},
        "step_roofline": {"bound": "hbm", "bytes_per_step": int(step_bytes), "achieved": round(step_gbs, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "roofline": kernels[0] if kernels else None,
        "kernels": kernels,
        "prefill": prefill,
    }


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


#: The prompt-pass kernels ``--kernel`` runs alone at a config's shape, for
#: rocprofv3 counter passes: the four projections (q3_gemm_ws with their
#: epilogues) and the causal attention.  Synthetic operands (N(0,1)
#: activations, N(0,0.02) weights); the config gives the token count.
KERNELS = ("gemm_gate_up", "gemm_qkv", "gemm_o", "gemm_down", "attn_prefill")


def kernel_probe(name: str, config: int, launches: int) -> int:
    """Run one prompt-pass kernel at config ``config``'s shape: one untimed
    launch, then ``launches`` launches timed with HIP events (each printed).
    ``rocprofv3 --pmc ... -- python3 bench.py --kernel NAME --config N``
    then reads the kernel's counters per dispatch."""
    import torch

    sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))
    from starter_amd import _lib
    from starter_amd._lib import call
    from starter_amd.workloads import MODEL, WORKLOADS

    wl = WORKLOADS[config]
    B, T = wl.batch, wl.prompt
    M, H, I = B * T, MODEL.hidden_size, MODEL.intermediate_size
    Hq, Hkv, D = MODEL.num_attention_heads, MODEL.num_key_value_heads, MODEL.head_dim
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(config)
    stream = torch.cuda.current_stream().cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731
    if name.startswith("gemm_"):
        N, K, epi = {"gemm_gate_up": (2 * I, H, _lib.EPI_SWIGLU), "gemm_qkv": ((Hq + 2 * Hkv) * D, H, _lib.EPI_STORE),
                     "gemm_o": (H, Hq * D, _lib.EPI_RESID), "gemm_down": (H, I, _lib.EPI_RESID)}[name]
        x = torch.randn(M, K, device=dev, generator=g).bfloat16()
        w = (0.02 * torch.randn(N, K, device=dev, generator=g)).bfloat16()
        cols = N // 2 if epi == _lib.EPI_SWIGLU else N
        y = torch.randn(M, cols, device=dev, generator=g).bfloat16()
        ws = torch.empty(max(call("q3_gemm_ws_floats", M, N, K), 4), dtype=torch.float32, device=dev)
        flop = 2.0 * M * N * K
        run = lambda: call("q3_gemm_ws", P(x), K, P(w), M, N, K, epi, P(y), cols, P(ws), stream)  # noqa: E731
        what = f"q3_gemm_ws M={M} N={N} K={K} epi={epi}"
    elif name == "attn_prefill":
        q = torch.randn(B, T, Hq, D, device=dev, generator=g).bfloat16()
        k = torch.randn(B, Hkv, T, D, device=dev, generator=g).bfloat16()
        v = torch.randn(B, Hkv, T, D, device=dev, generator=g).bfloat16()
        out = torch.empty_like(q)
        flop = 4.0 * D * Hq * B * T * (T + 1) / 2
        run = lambda: call("q3_attn_prefill", P(q), P(k), P(v), P(out), B, T, 0, Hq, Hkv, T,  # noqa: E731
                           D ** -0.5, stream)
        what = f"q3_attn_prefill B={B} T={T} start=0"
    else:
        raise SystemExit(f"--kernel must be one of {', '.join(KERNELS)}")
    run()
    torch.cuda.synchronize()
    for i in range(launches):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        log(f"{what}: launch {i}: {ms:.3f} ms, {flop / ms / 1e9:.0f} TFLOP/s")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--extra-configs", default="1,3,4,5",
                    help="comma-separated BASELINE configs reported beside the headline (empty: none)")
    ap.add_argument("--ckpt-dir", default=os.environ.get("Q3_CKPT_DIR", "/tmp/q3_seeded_qwen3_4b"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (3 times): the known-size "
                         "kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--kernel", choices=KERNELS,
                    help="only run one prompt-pass kernel at --config's shape (an untimed launch, then "
                         "--launches timed ones): the program rocprofv3's counter passes profile")
    ap.add_argument("--launches", type=int, default=1)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(one MI355X per box); run with --gpus 1", file=sys.stderr)
        return 2
    if args.copy_probe:
        return copy_probe()
    if args.kernel:
        return kernel_probe(args.kernel, args.config, args.launches)

    sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))
    import torch
    from starter_amd.checkpoint import ensure_seeded_checkpoint, load_checkpoint
    from starter_amd.engine import Engine
    from starter_amd.workloads import MODEL, MODEL_SEED, WORKLOADS

    head = WORKLOADS[args.config]
    extras = [WORKLOADS[int(c)] for c in args.extra_configs.split(",") if c.strip() and int(c) != args.config]

    t0 = time.time()
    ckpt = ensure_seeded_checkpoint(args.ckpt_dir, MODEL, MODEL_SEED)
    log(f"checkpoint ready in {time.time() - t0:.1f}s")
    eng = Engine(str(ckpt))
    results = {wl.number: run_workload(eng, wl, args.steps, args.warmup) for wl in [head] + extras}

    if not args.no_cpu_baseline:
        del eng
        torch.cuda.empty_cache()
        from oracle.ref_cpu_path import RefCpuDecode

        torch.set_num_threads(len(os.sched_getaffinity(0)))
        cfg, tensors = load_checkpoint(ckpt)
        ref = RefCpuDecode(cfg, tensors)
        del tensors
        for wl in [head] + extras:
            results[wl.number]["cpu_baseline"] = cpu_baseline(ref, wl, 20.0 if wl is head else 6.0)
            log(f"{wl.name}: cpu baseline {results[wl.number]['cpu_baseline']}")

    r = results[head.number]
    line = {
        "metric": "decode tokens/s (Qwen3-4B bf16 greedy, seeded random init)",
        "value": r["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": r["warmup"],
        "ms_per_step": r["ms_per_step"],
        "ms_per_step_median": r["ms_per_step_median"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) BF16 weights of the Qwen3-4B shapes, uniform random prompt ids)",
        "config": r["config"],
        "step_roofline": r["step_roofline"],
        "roofline": r["roofline"],
        "kernels": r["kernels"],
        "cpu_baseline": r.get("cpu_baseline"),
        "prefill": r["prefill"],
        "workloads": {WORKLOADS[n].name: results[n] for n in results if n != head.number},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
