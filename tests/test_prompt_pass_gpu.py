"""The prompt pass at the benchmark's own sizes, on the GPU.

BASELINE configs 4 and 5 prefill 131,072 prompt tokens in one chunk
(``PREFILL_CHUNK_TOKENS`` = 131072): every projection is a q3_gemm_ws call
with M = 131,072 (the down projection's input, [131072, 9728] BF16, is
2.55 GB, past 2^31 bytes), and prefill attention walks causal ranges of up to
16,384 keys.  These tests run exactly those launches and check them:

  * the projections on sampled token rows (first, last, the rows either side
    of the 2^31-byte offset, random) against float64 dot products of the same
    BF16 operands, each epilogue (store, residual join, SwiGLU) included;
  * prefill attention on sampled query rows (first, either side of the
    64-key block edges, the last, random) against float64 softmax attention,
    with a bound derived from the one rounding the kernel adds (P to BF16
    before P.V, as reference fused.py:699-701 does);
  * the whole prompt pass end to end on a 2-layer model at Qwen3-4B's real
    dimensions, B = 1 and P = 16,384 tokens, in one chunk and in chunks of
    4,096 (later chunks attend over a cached prefix), against the CPU oracle:
    the last position's logits over the whole vocabulary, both layers' K/V
    cache rows at every prompt position, and decode steps read from that
    cache -- bounded by twice what a legal reordering of the oracle's own
    arithmetic moves (its projections summed by torch's FP32 GEMM), measured
    beside it on the same inputs.

Reference: engine/engine.py:738-803 (the chunked prompt pass),
tests/test_equivalence.py:145-171 (the prefill logit delta).
"""

import dataclasses

import numpy as np
import pytest
import torch

from oracle import qwen3_cpu as oc
from starter_amd import _lib
from starter_amd import engine as engine_mod
from starter_amd._lib import call
from starter_amd.checkpoint import QWEN3_4B, load_checkpoint, write_seeded_checkpoint

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
M_FULL = 131072                 # configs 4 and 5: 64 x 2048 and 8 x 16384 prompt tokens, one chunk
FLOOR_FACTOR = 2.0


def S():
    return torch.cuda.current_stream().cuda_stream


def P(t):
    return None if t is None else t.data_ptr()


def device_normal(shape, scale, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV, dtype=torch.float32) * scale).to(torch.bfloat16)


def check_projection(got, x, w, frac=0.03):
    """``got`` (BF16) vs the float64 dot products of the same BF16 operands:
    within one BF16 ulp of the exact value plus 2^-17 * sum|x*w| (FP32
    accumulation in two orders), and most elements rounded exactly like it."""
    x64 = x.float().numpy().astype(np.float64)
    w64 = w.float().numpy().astype(np.float64)
    exact = x64 @ w64.T
    s_abs = np.abs(x64) @ np.abs(w64).T
    g = got.cpu().float().numpy().astype(np.float64)
    spacing = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 2.0 ** -126))) - 7)
    err = np.abs(g - exact)
    assert np.all(err <= spacing + 2.0 ** -17 * s_abs), f"max excess {(err - spacing - 2.0**-17 * s_abs).max():.3e}"
    assert (g != oc.bf16_round(exact)).mean() <= frac, f"{(g != oc.bf16_round(exact)).mean():.3f} differ"


def sample_rows(M, row_bytes, n, seed):
    """First and last rows, the two rows either side of the 2^31-byte offset of
    an operand whose rows are ``row_bytes`` long (when it has one), and random
    rows; sorted, unique."""
    g = torch.Generator().manual_seed(seed)
    rows = [0, M - 1]
    edge = (1 << 31) // row_bytes
    if edge < M - 1:
        rows += [edge, edge + 1]
    rows += torch.randint(0, M, (n,), generator=g).tolist()
    return torch.tensor(sorted(set(rows)), dtype=torch.int64)


# (name, N, K, epilogue): the four prompt-pass projections of Qwen3-4B.
PROJECTIONS = [("qkv", 6144, 2560, _lib.EPI_STORE), ("o", 2560, 4096, _lib.EPI_RESID),
               ("gate_up", 19456, 2560, _lib.EPI_SWIGLU), ("down", 2560, 9728, _lib.EPI_RESID)]


@pytest.mark.parametrize("name,N,K,epi", PROJECTIONS, ids=[p[0] for p in PROJECTIONS])
def test_gemm_ws_full_prompt(name, N, K, epi):
    """q3_gemm_ws at M = 131,072, as the engine calls it for one chunk of
    configs 4 and 5.  The store epilogue against float64 on ~200 sampled rows;
    the residual and SwiGLU epilogues on the same rows against the plain
    projection of those rows (itself checked against float64), the residual
    bit-exact up to the one rounding its FP32 sum order may move, SwiGLU
    within 2 ulps as in the smaller-shape tests."""
    M = M_FULL
    x = device_normal((M, K), 1.0, 11 + K)
    w = device_normal((N, K), 0.02, 13 + N)
    wc = w.cpu()
    floats = call("q3_gemm_ws_floats", M, N, K)
    ws = torch.empty(max(floats, 1), dtype=torch.float32, device=DEV)
    cols = N // 2 if epi == _lib.EPI_SWIGLU else N
    rows = sample_rows(M, max(K, cols) * 2, 200, N + K)
    rows_d = rows.to(DEV)
    xs = x[rows_d].cpu()
    if epi == _lib.EPI_RESID:
        out = device_normal((M, cols), 1.0, 17)
        res = out[rows_d].cpu()
    else:
        out = torch.empty(M, cols, dtype=torch.bfloat16, device=DEV)
    print(f"{name}: M={M} N={N} K={K} epi={epi}, x {x.numel() * 2 / 2**30:.2f} GiB, "
          f"split-tail floats {floats}", flush=True)
    call("q3_gemm_ws", P(x), K, P(w), M, N, K, epi, P(out), cols, P(ws), S())
    torch.cuda.synchronize()
    got = out[rows_d].cpu()
    del x, out
    if epi == _lib.EPI_STORE:
        check_projection(got, xs, wc)
        return
    # The plain projection of the sampled rows through the narrow tiling,
    # checked against float64, then the fused epilogue against it.
    y = torch.empty(len(rows), N, dtype=torch.bfloat16, device=DEV)
    call("q3_gemm", P(xs.to(DEV)), K, P(w), len(rows), N, K, _lib.EPI_STORE, P(y), N, S())
    torch.cuda.synchronize()
    yc = y.cpu()
    check_projection(yc, xs, wc)
    if epi == _lib.EPI_RESID:
        want = (res.float() + yc.float()).bfloat16()
        diff = (got.float() - want.float()).abs()
        assert (diff > 0).float().mean() <= 0.03
        assert torch.all(diff <= 2.0 ** -7 * (want.float().abs() + yc.float().abs()) + 1e-6)
    else:
        want = oc.swiglu(yc[:, 0::2], yc[:, 1::2])
        u = np.abs(got.float().numpy().astype(np.float64) - want.float().numpy().astype(np.float64))
        spacing = np.exp2(np.floor(np.log2(np.maximum(np.abs(want.float().numpy()), 2.0 ** -126))) - 7)
        assert (u / spacing).max() <= 2 and (u > 0).mean() <= 0.06


def attention_rows_f64(q, k, v, scale):
    """float64 softmax attention of query rows q [n, D] over k, v [L, D];
    returns (out [n, D], the rounding scale sqrt(sum p^2 v^2) / sum p [n, D])."""
    s = (q.astype(np.float64) @ k.astype(np.float64).T) * scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    l = p.sum(axis=1, keepdims=True)
    v64 = v.astype(np.float64)
    out = (p @ v64) / l
    spread = np.sqrt((p * p) @ (v64 * v64)) / l
    return out, spread


# (B, T, start, capacity): config 5's and config 4's prompt passes in one chunk,
# and the last chunk of config 5 under the reference's 16,384-token chunking
# (16384 // 8 = 2048 tokens per sequence, over a 14,336-key cached prefix).
ATTN_SHAPES = [(1, 16384, 0, 16512), (64, 2048, 0, 2176), (8, 2048, 14336, 16512)]


@pytest.mark.parametrize("B,T,start,C", ATTN_SHAPES, ids=["b1_t16384", "b64_t2048", "b8_t2048_start14336"])
def test_attn_prefill_full_prompt(B, T, start, C):
    """q3_attn_prefill at the benchmark's causal ranges, on sampled query rows
    of every head against float64.

    The bound: the kernel rounds each probability to BF16 before P.V (relative
    error <= 2^-9, unbiased), so its output differs from the exact one by a sum
    of independent terms of standard deviation <= 2^-9 sqrt(sum p^2 v^2) / sum p;
    8 of those, plus one BF16 ulp of the exact value for the output's own
    rounding.  At 16K keys that is ~2e-4 against outputs of ~1e-2, so a causal
    range off by one 64-key block (a change of ~5e-4) fails it."""
    Hq, Hkv, D = 32, 8, 128
    scale = D ** -0.5
    q = device_normal((B * T, Hq, D), 1.0, 21 + T)
    ck = device_normal((B, Hkv, C, D), 1.0, 22 + T)
    cv = device_normal((B, Hkv, C, D), 1.0, 23 + T)
    out = torch.empty(B * T, Hq * D, dtype=torch.bfloat16, device=DEV)
    print(f"attn_prefill B={B} T={T} start={start} C={C}", flush=True)
    call("q3_attn_prefill", P(q), P(ck), P(cv), P(out), B, T, start, Hq, Hkv, C, scale, S())
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(B * T + start)
    ts = {0, 1, 63, 64, 65, 127, 128, T - 2, T - 1} | set(torch.randint(0, T, (8,), generator=g).tolist())
    bs = sorted({0, B - 1} | set(torch.randint(0, B, (2,), generator=g).tolist()))
    worst = 0.0
    for b in bs:
        kb, vb = ck[b].cpu().float().numpy(), cv[b].cpu().float().numpy()
        for t in sorted(ts):
            r = b * T + t
            qr = q[r].cpu().float().numpy()                   # [Hq, D]
            got = out[r].cpu().float().numpy().reshape(Hq, D)
            L = start + t + 1
            for h in range(Hkv):
                heads = slice(4 * h, 4 * h + 4)
                want, spread = attention_rows_f64(qr[heads], kb[h, :L], vb[h, :L], scale)
                spacing = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
                err = np.abs(got[heads] - want)
                bound = spacing + 8 * 2.0 ** -9 * spread + 1e-6
                worst = max(worst, float((err / bound).max()))
                assert np.all(err <= bound), (b, t, h, float((err - bound).max()))
    print(f"attn_prefill B={B} T={T} start={start}: worst error / bound {worst:.3f}", flush=True)


# ------------------------------------------------------------------ end to end

DECODE_STEPS = 4
LAYER0_DIFF_FRACTION = 1e-3
LAYER0_ROW_REL = 2.0 ** -4


@pytest.fixture(scope="module")
def two_layer_ckpt(tmp_path_factory):
    """Qwen3-4B's dimensions with two layers (1.2 GB), seeded like the benchmark model."""
    cfg = dataclasses.replace(QWEN3_4B, num_hidden_layers=2)
    path = tmp_path_factory.mktemp("q3_2layer")
    write_seeded_checkpoint(path, cfg, 0)
    return path


_ORACLE_RUNS = {}


def oracle_run(ckpt, B, prompt):
    """The CPU oracle's prompt pass (one chunk) and its teacher-forced decode
    steps, and the same with FP32-GEMM projections (the reordering floor):
    (ids, the oracle's greedy stream [steps][B], {label: logits, cache})."""
    key = (B, prompt)
    if key in _ORACLE_RUNS:
        return _ORACLE_RUNS[key]
    cfg, tensors = load_checkpoint(ckpt)
    orc = oc.Qwen3Oracle(cfg, tensors, torch.bfloat16)
    ids = torch.tensor(np.random.Generator(np.random.PCG64(prompt + B)).integers(0, 151643, (B, prompt)))
    runs, stream = {}, None
    for label, lin in (("oracle", oc.linear), ("floor", oc.f32_linear())):
        orc.linear = lin
        orc.reset(B, prompt + DECODE_STEPS)
        first = orc.prefill(ids).float()
        cache = [(k[:, :, :prompt].clone(), v[:, :, :prompt].clone()) for k, v in zip(orc.cache_k, orc.cache_v)]
        if stream is None:  # the oracle's own greedy stream, fed to every run
            stream = [oc.argmax_first(first).tolist()]
        logits = [first]
        for k in range(DECODE_STEPS - 1):
            lg = orc.forward(torch.tensor(stream[k]).view(B, 1), prompt + k).float()
            logits.append(lg)
            if len(stream) < DECODE_STEPS:
                stream.append(oc.argmax_first(lg).tolist())
        runs[label] = {"logits": torch.stack(logits), "cache": cache}
    orc.cache_k = orc.cache_v = None
    _ORACLE_RUNS[key] = (ids, stream, runs)
    return _ORACLE_RUNS[key]


@pytest.fixture(scope="module")
def two_layer_engine(two_layer_ckpt):
    eng = engine_mod.Engine(str(two_layer_ckpt))
    yield eng
    eng.graph_key_reset()


def _stats(a, want):
    """(max-abs, mean-abs, fraction of elements not identical, max |a - want|
    over the RMS of want's 128-element row)."""
    a, w = a.float(), want.float()
    d = (a - w).abs()
    rms = w.pow(2).mean(dim=-1, keepdim=True).sqrt().clamp_min(1e-30)
    return float(d.max()), float(d.mean()), float((d > 0).float().mean()), float((d / rms).max())


def _fmt(t):
    return f"{t[0]:.4f}/{t[1]:.6f}/{t[2]:.2e}/{t[3]:.4f}"


@pytest.mark.parametrize("B,prompt,chunk", [(1, 16384, 0), (1, 16384, 4096), (8, 2048, 0)],
                         ids=["b1_p16384_one_chunk", "b1_p16384_chunks_of_4096", "b8_p2048_one_chunk"])
def test_prompt_pass_matches_oracle(two_layer_engine, two_layer_ckpt, B, prompt, chunk):
    """The engine's prompt pass at full width, then DECODE_STEPS - 1 decode
    steps (graph replays reading the cache the pass wrote), teacher-forced on
    the oracle's stream.  B = 1, P = 16,384 in one chunk (every projection at
    M = 16,384, attention over the whole causal range) and in chunks of 4,096
    (three later chunks over cached prefixes of 4K-12K keys); B = 8, P = 2,048
    (config 5's chunk under the reference's chunking: eight sequences in one
    16,384-row pass, decoded on the MFMA path).  Checked against the oracle's
    one-chunk pass:
      * the logits of every step over the whole vocabulary, and layer 1's K and
        V cache rows at every prompt position (each a function of layer 0's
        whole output at that position): max-abs and mean-abs within
        FLOOR_FACTOR x the FP32-GEMM floor's;
      * layer 0's K and V rows, which see one projection's rounding and no
        propagated difference (the floor matches them in all but ~1e-5 of the
        elements): at most LAYER0_DIFF_FRACTION of the elements differ, each
        by at most LAYER0_ROW_REL of its row's RMS (two BF16 ulps at four
        times the RMS; RoPE's sums cancel, so an ulp of the element itself
        says nothing near zero).
    An argmax may differ from the oracle's only where the oracle's own gap is
    within what the logit bound allows."""
    ids, stream, runs = oracle_run(two_layer_ckpt, B, prompt)
    eng = two_layer_engine
    saved = engine_mod.PREFILL_CHUNK_TOKENS
    if chunk:
        engine_mod.PREFILL_CHUNK_TOKENS = chunk
    try:
        steps, logits = eng.trace_logits(ids.tolist(), DECODE_STEPS, forced=stream)
        cache = [(eng.cache_k[i, :, :, :prompt].cpu(), eng.cache_v[i, :, :, :prompt].cpu())
                 for i in range(eng.LAYERS)]
    finally:
        engine_mod.PREFILL_CHUNK_TOKENS = saved
    want, floor = runs["oracle"], runs["floor"]
    lg = logits.float()
    e, f = _stats(lg, want["logits"]), _stats(floor["logits"], want["logits"])
    report = [f"logits engine {_fmt(e)} floor {_fmt(f)}"]
    bounded = [("logits", e, f)]
    for i in range(eng.LAYERS):
        for j, kv in enumerate("KV"):
            e = _stats(cache[i][j], want["cache"][i][j])
            f = _stats(floor["cache"][i][j], want["cache"][i][j])
            report.append(f"layer {i} {kv} engine {_fmt(e)} floor {_fmt(f)}")
            if i == 0:
                assert e[2] <= LAYER0_DIFF_FRACTION and e[3] <= LAYER0_ROW_REL, (i, kv, e)
            else:
                bounded.append((f"layer {i} {kv}", e, f))
    print(f"B={B} P={prompt} chunk={chunk or prompt} (max-abs/mean-abs/differing/max over row RMS): "
          + "; ".join(report), flush=True)
    for name, e, f in bounded:
        assert e[0] <= FLOOR_FACTOR * f[0] and e[1] <= FLOOR_FACTOR * f[1], (name, e, f)
    f_max = _stats(floor["logits"], want["logits"])[0]
    top = want["logits"].max(dim=-1).values
    for k in range(DECODE_STEPS):
        for b in range(B):
            if steps[k][b] != stream[k][b]:
                assert float(top[k, b] - want["logits"][k, b, steps[k][b]]) <= 2 * FLOOR_FACTOR * f_max, (k, b)
