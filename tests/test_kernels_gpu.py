"""Kernel parity on the GPU, each launch through the C ABI (libq3.so).

Each kernel is compared with the CPU oracle's function for the same op
(oracle/qwen3_cpu.py, itself pinned by tests/test_oracle.py) or, for the
projections, a float32 reference of the same dot products.  Tolerances, written
per test:
  * element-wise ops (norm, RoPE, residual add, SwiGLU, KV append): bit-exact
    except where an FP32 reduction (the RMS of a row) sums in another order,
    which may move one element by one BF16 ulp -- at most 1e-3 of elements;
  * projections: |gpu - exact| <= 1 BF16 ulp + 2^-17 sum|x*w| against the
    float64 dot product, >= 97% of elements rounding exactly like it (only the
    summation order differs); the fused prologues and epilogues are checked
    bit-exactly against the unfused kernels they replace;
  * attention: max |gpu - oracle| <= 1e-2 + 1e-2 |oracle| (P rounds to BF16
    before P.V, as in reference fused.py:699-701).
"""

import numpy as np
import pytest
import torch

from oracle import qwen3_cpu as oc
from starter_amd import _lib
from starter_amd._lib import call

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def P(t):
    return None if t is None else t.data_ptr()


_KEEP = []


def dv(t):
    """Device copy that stays alive for the rest of the test.

    A pointer taken from a temporary (``P(x.to(DEV))``) would dangle: the
    caching allocator hands the freed block to the next temporary.
    """
    d = t.to(DEV)
    _KEEP.append(d)
    return d


@pytest.fixture(autouse=True)
def _release_device_copies():
    yield
    torch.cuda.synchronize()
    _KEEP.clear()


def S():
    return torch.cuda.current_stream().cuda_stream


def rnd(shape, scale=1.0, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def ulps(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    """|a - b| in units of b's BF16 spacing."""
    a64, b64 = a.float().numpy().astype(np.float64), b.float().numpy().astype(np.float64)
    spacing = np.exp2(np.floor(np.log2(np.maximum(np.abs(b64), 2.0 ** -126))) - 7)
    return np.abs(a64 - b64) / spacing


def assert_nearly_exact(got, want, frac=1e-3, max_ulp=1):
    u = ulps(got.cpu(), want.cpu())
    assert u.max() <= max_ulp, f"max {u.max()} ulp"
    assert (u > 0).mean() <= frac, f"{(u > 0).mean():.2e} of elements differ"


# ------------------------------------------------------------------ norms


@pytest.mark.parametrize("rows,cols", [(1, 128), (37, 320), (5, 2560), (3, 4096)])
def test_rmsnorm(rows, cols):
    x = rnd((rows, cols), 2.0, 1)
    w = (1 + rnd((cols,), 0.2, 2).float()).to(torch.bfloat16)
    y = torch.empty(rows, cols, dtype=torch.bfloat16, device=DEV)
    call("q3_rmsnorm", P(dv(x)), cols, P(dv(w)), P(y), cols, rows, cols, 1e-6, S())
    torch.cuda.synchronize()
    assert_nearly_exact(y, oc.rms_norm(x, w, 1e-6))


def test_add_rmsnorm_and_embed():
    rows, cols = 9, 2560
    r, d = rnd((rows, cols), 1.0, 3), rnd((rows, cols), 1.0, 4)
    w = (1 + rnd((cols,), 0.2, 5).float()).to(torch.bfloat16)
    rd, dd, wd = r.to(DEV), d.to(DEV), w.to(DEV)
    s = torch.empty_like(rd)
    y = torch.empty_like(rd)
    call("q3_add_rmsnorm", P(rd), P(dd), P(s), P(y), P(wd), rows, cols, 1e-6, S())
    torch.cuda.synchronize()
    want_s = r + d
    assert torch.equal(s.cpu(), want_s)  # the residual sum rounds exactly like a BF16 add
    assert_nearly_exact(y, oc.rms_norm(want_s, w, 1e-6))
    # In place (sum_out == res).
    call("q3_add_rmsnorm", P(rd), P(dd), P(rd), P(y), P(wd), rows, cols, 1e-6, S())
    torch.cuda.synchronize()
    assert torch.equal(rd.cpu(), want_s)

    table = rnd((50, cols), 1.0, 6)
    ids = torch.tensor([3, 49, 0, 3], dtype=torch.int64)
    resid = torch.empty(4, cols, dtype=torch.bfloat16, device=DEV)
    y = torch.empty_like(resid)
    call("q3_embed_rmsnorm", P(dv(ids)), P(dv(table)), P(resid), P(y), P(wd), 4, cols, 1e-6, S())
    torch.cuda.synchronize()
    assert torch.equal(resid.cpu(), table[ids])
    assert_nearly_exact(y, oc.rms_norm(table[ids], w, 1e-6))


# ------------------------------------------------------- qk norm + rope + kv


@pytest.mark.parametrize("B,T,start", [(1, 1, 0), (2, 5, 3), (3, 17, 40)])
def test_qk_norm_rope_kv(B, T, start):
    Hq, Hkv, D, C = 8, 2, 128, 64
    width = (Hq + 2 * Hkv) * D
    qkv = rnd((B * T, width), 1.5, 7)
    qw = (1 + rnd((D,), 0.2, 8).float()).to(torch.bfloat16)
    kw = (1 + rnd((D,), 0.2, 9).float()).to(torch.bfloat16)
    cos, sin = oc.rope_tables(5e6, D, 4096)
    ck = torch.zeros(B, Hkv, C, D, dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    q_out = torch.empty(B * T, Hq, D, dtype=torch.bfloat16, device=DEV)
    call("q3_qk_norm_rope_kv", P(dv(qkv)), width, P(dv(qw)), P(dv(kw)), P(dv(cos)),
         P(dv(sin)), None, start, P(q_out), P(ck), P(cv), B, T, Hq, Hkv, D, C, 1e-6, S())
    torch.cuda.synchronize()
    x = qkv.view(B, T, Hq + 2 * Hkv, D)
    c = cos[start:start + T].view(1, T, 1, D)
    s_ = sin[start:start + T].view(1, T, 1, D)
    want_q = oc.apply_rope(oc.rms_norm(x[:, :, :Hq], qw, 1e-6), c, s_)
    want_k = oc.apply_rope(oc.rms_norm(x[:, :, Hq:Hq + Hkv], kw, 1e-6), c, s_)
    assert_nearly_exact(q_out.view(B, T, Hq, D), want_q, frac=2e-3, max_ulp=2)
    got_k = ck.cpu()
    assert_nearly_exact(got_k[:, :, start:start + T].transpose(1, 2), want_k, frac=2e-3, max_ulp=2)
    assert torch.equal(cv.cpu()[:, :, start:start + T].transpose(1, 2), x[:, :, Hq + Hkv:])
    # Nothing outside the written slots.
    mask = torch.ones(C, dtype=torch.bool)
    mask[start:start + T] = False
    assert torch.all(got_k[:, :, mask] == 0) and torch.all(cv.cpu()[:, :, mask] == 0)


# ------------------------------------------------------------ projections


def check_projection(got, x, w, frac=0.03):
    """``got`` vs the float64 dot products of the same BF16 operands.

    Allowed error: one BF16 ulp of the exact value (the final rounding, plus
    one rounding boundary crossed by summation error) and 2^-17 * sum|x*w|
    (FP32 accumulation error of both orders, which dominates near zero).
    Most elements must round exactly like the float64 sum.
    """
    x64 = x.float().numpy().astype(np.float64)
    w64 = w.float().numpy().astype(np.float64)
    exact = x64 @ w64.T
    s_abs = np.abs(x64) @ np.abs(w64).T
    g = got.cpu().float().numpy().astype(np.float64)
    spacing = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 2.0 ** -126))) - 7)
    err = np.abs(g - exact)
    assert np.all(err <= spacing + 2.0 ** -17 * s_abs), f"max excess {(err - spacing - 2.0**-17 * s_abs).max():.3e}"
    assert (g != oc.bf16_round(exact)).mean() <= frac, f"{(g != oc.bf16_round(exact)).mean():.3f} differ"


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("N,K", [(1536, 320), (320, 1024), (2560, 2560), (2560, 9728), (330, 1024), (2570, 4096)])
def test_gemv_plain_store(M, N, K):
    """N = 330 and 2570 leave waves past the last row in the last workgroup:
    they load clamped rows and store nothing."""
    x, w = rnd((M, K), 1.0, M), rnd((N, K), 0.02, N + K)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    call("q3_gemv", _lib.X_PLAIN, P(dv(x)), K, None, None, 0.0, None, P(dv(w)), M, N, K,
         _lib.EPI_STORE, P(y), N, None, None, None, None, None, 0, S())
    torch.cuda.synchronize()
    check_projection(y, x, w)


def gemv(x_mode, x, ldx, w, M, N, K, epi, y, ldy, ids=None, norm_w=None, resid_out=None, pv=None, pi=None,
         pos=None, feed=None, rec=None):
    call("q3_gemv", x_mode, P(x), ldx, P(ids), P(norm_w), 1e-6, P(resid_out), P(w), M, N, K, epi, P(y), ldy,
         P(pv), P(pi), P(pos), P(feed), P(rec), 0 if rec is None else rec.shape[0], S())


def finish(pv, pi, nparts, M, tok, pos=None, counter=None, feed=None, rec=None, stream=None):
    call("q3_argmax_finish", P(pv), P(pi), nparts, M, P(tok), P(pos), P(counter), P(feed), P(rec),
         0 if rec is None else rec.shape[0], stream if stream is not None else S())


@pytest.mark.parametrize("M", [1, 3, 8])
def test_gemv_epilogues_and_norm_prologue(M):
    """Each fused prologue/epilogue equals the unfused kernels it replaces, bit for bit."""
    K, N, I = 2560, 1024, 512
    src = dv(rnd((M, K), 1.0, 11))
    g = dv((1 + rnd((K,), 0.2, 12).float()).to(torch.bfloat16))
    w = dv(rnd((N, K), 0.02, 13))
    # NORM prologue == q3_rmsnorm then a plain GEMV (same reduction order).
    n = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
    call("q3_rmsnorm", P(src), K, P(g), P(n), K, M, K, 1e-6, S())
    y_ref = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    gemv(_lib.X_PLAIN, n, K, w, M, N, K, _lib.EPI_STORE, y_ref, N)
    y = torch.empty_like(y_ref)
    gemv(_lib.X_NORM, src, K, w, M, N, K, _lib.EPI_STORE, y, N, norm_w=g)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    assert_nearly_exact(n, oc.rms_norm(src.cpu(), g.cpu(), 1e-6))
    # RESID epilogue == bf16(res + bf16(acc)), in place.
    res = rnd((M, N), 1.0, 14)
    resd = dv(res)
    gemv(_lib.X_NORM, src, K, w, M, N, K, _lib.EPI_RESID, resd, N, norm_w=g)
    torch.cuda.synchronize()
    assert torch.equal(resd.cpu(), res + y.cpu())
    # SWIGLU epilogue on interleaved (gate, up) rows == swiglu of the stored projections.
    wgu = dv(torch.stack([rnd((I, K), 0.02, 15), rnd((I, K), 0.02, 16)], 1).reshape(2 * I, K))
    gu = torch.empty(M, 2 * I, dtype=torch.bfloat16, device=DEV)
    gemv(_lib.X_NORM, src, K, wgu, M, 2 * I, K, _lib.EPI_STORE, gu, 2 * I, norm_w=g)
    act = torch.empty(M, I, dtype=torch.bfloat16, device=DEV)
    gemv(_lib.X_NORM, src, K, wgu, M, 2 * I, K, _lib.EPI_SWIGLU, act, I, norm_w=g)
    torch.cuda.synchronize()
    gu = gu.cpu()
    assert_nearly_exact(act, oc.swiglu(gu[:, 0::2], gu[:, 1::2]), frac=5e-3)


@pytest.mark.parametrize("M", [1, 4])
def test_gemv_ragged_swiglu_and_argmax(M):
    """Row counts that leave idle waves in the last workgroup (SwiGLU: 4 rows per
    wave; argmax: 4 rows per wave) give the same bits as the unfused path."""
    K, I, V = 2560, 510, 4100
    src = dv(rnd((M, K), 1.0, 31))
    g = dv((1 + rnd((K,), 0.2, 32).float()).to(torch.bfloat16))
    wgu = dv(rnd((2 * I, K), 0.02, 33))
    gu = torch.empty(M, 2 * I, dtype=torch.bfloat16, device=DEV)
    gemv(_lib.X_NORM, src, K, wgu, M, 2 * I, K, _lib.EPI_STORE, gu, 2 * I, norm_w=g)
    act = torch.empty(M, I, dtype=torch.bfloat16, device=DEV)
    gemv(_lib.X_NORM, src, K, wgu, M, 2 * I, K, _lib.EPI_SWIGLU, act, I, norm_w=g)
    wv = dv(rnd((V, K), 0.02, 34))
    y = torch.empty(M, V, dtype=torch.bfloat16, device=DEV)
    gemv(_lib.X_NORM, src, K, wv, M, V, K, _lib.EPI_STORE, y, V, norm_w=g)
    nparts = call("q3_gemv_partials", M, V, _lib.EPI_ARGMAX)
    pv = torch.empty(nparts, M, dtype=torch.float32, device=DEV)
    pi = torch.empty(nparts, M, dtype=torch.int32, device=DEV)
    gemv(_lib.X_NORM, src, K, wv, M, V, K, _lib.EPI_ARGMAX, None, 0, norm_w=g, pv=pv, pi=pi)
    tok = torch.empty(M, dtype=torch.int64, device=DEV)
    finish(pv, pi, nparts, M, tok)
    torch.cuda.synchronize()
    gu = gu.cpu()
    assert_nearly_exact(act, oc.swiglu(gu[:, 0::2], gu[:, 1::2]), frac=5e-3)
    assert tok.cpu().tolist() == y.cpu().float().argmax(-1).tolist()


@pytest.mark.parametrize("M", [1, 4, 8])
def test_gemv_embed_norm_and_argmax(M):
    V, K = 4096, 2560
    table = rnd((V, K), 0.02, 21)
    g = dv((1 + rnd((K,), 0.2, 22).float()).to(torch.bfloat16))
    ids = torch.randint(0, V, (M,), generator=torch.Generator().manual_seed(M))
    td, idd = dv(table), dv(ids)
    resid = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
    y = torch.empty(M, V, dtype=torch.bfloat16, device=DEV)
    gemv(_lib.X_EMBED_NORM, td, K, td, M, V, K, _lib.EPI_STORE, y, V, ids=idd, norm_w=g, resid_out=resid)
    n = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
    call("q3_rmsnorm", P(resid), K, P(g), P(n), K, M, K, 1e-6, S())
    torch.cuda.synchronize()
    assert torch.equal(resid.cpu(), table[ids])
    check_projection(y, n.cpu(), table)
    # Fused argmax partials + finish == argmax of the stored logits (first index on ties).
    nparts = call("q3_gemv_partials", M, V, _lib.EPI_ARGMAX)
    pv = torch.empty(nparts, M, dtype=torch.float32, device=DEV)
    pi = torch.empty(nparts, M, dtype=torch.int32, device=DEV)
    y2 = torch.empty_like(y)
    gemv(_lib.X_NORM, resid, K, td, M, V, K, _lib.EPI_STORE_ARGMAX, y2, V, norm_w=g, pv=pv, pi=pi)
    tok = torch.empty(M, dtype=torch.int64, device=DEV)
    pos = torch.tensor([5], dtype=torch.int64, device=DEV)
    counter = torch.zeros(1, dtype=torch.int32, device=DEV)
    finish(pv, pi, nparts, M, tok, pos, counter)
    tok2 = torch.empty_like(tok)
    gemv(_lib.X_NORM, resid, K, td, M, V, K, _lib.EPI_ARGMAX, None, 0, norm_w=g, pv=pv, pi=pi)
    finish(pv, pi, nparts, M, tok2)
    torch.cuda.synchronize()
    assert torch.equal(y2.cpu(), y.cpu())
    assert tok.cpu().tolist() == y.cpu().argmax(-1).tolist() == tok2.cpu().tolist()
    assert pos.item() == 6 and counter.item() == 0
    # Step records at position 7 (the step's input at 6): rows 0.. fed chosen
    # tokens, the last row left to the greedy choice.
    npos = 10
    feed = torch.full((npos, M), -1, dtype=torch.int64)
    targets = torch.randint(0, V, (M,), generator=torch.Generator().manual_seed(40 + M))
    feed[7, :M - 1] = targets[:M - 1]
    feedd, rec = dv(feed), torch.zeros(npos, M, 4, dtype=torch.int32, device=DEV)
    tok3 = torch.empty_like(tok)
    gemv(_lib.X_NORM, resid, K, td, M, V, K, _lib.EPI_ARGMAX, None, 0, norm_w=g, pv=pv, pi=pi,
         pos=pos, feed=feedd, rec=rec)
    finish(pv, pi, nparts, M, tok3, pos, counter, feedd, rec)
    torch.cuda.synchronize()
    yc, r = y.cpu().float(), rec.cpu()
    greedy = yc.argmax(-1)
    fed = torch.where(feed[7] >= 0, feed[7], greedy)
    assert tok3.cpu().tolist() == fed.tolist()
    assert r[7, :, 0].tolist() == greedy.tolist() and r[7, :, 3].tolist() == fed.tolist()
    assert torch.equal(r[7, :, 1].view(torch.float32), yc.max(-1).values)
    assert torch.equal(r[7, :, 2].view(torch.float32), yc.gather(1, fed.view(M, 1))[:, 0])
    assert (r[:7] == 0).all() and (r[8:] == 0).all()  # only position 7 is written
    assert pos.item() == 7 and counter.item() == 0


def test_argmax_rows_ties():
    V = 5000
    x = torch.zeros(3, V, dtype=torch.bfloat16)
    x[0, [7, 4000]] = 3.0
    x[1, :] = -1.0
    x[2, [4999, 12, 13]] = 2.5
    tok = torch.empty(3, dtype=torch.int64, device=DEV)
    pos = torch.zeros(1, dtype=torch.int64, device=DEV)
    counter = torch.zeros(1, dtype=torch.int32, device=DEV)
    xd = dv(x)
    call("q3_argmax_rows", P(xd), V, 3, V, P(tok), P(pos), P(counter), None, None, 0, S())
    torch.cuda.synchronize()
    assert tok.cpu().tolist() == [7, 0, 12] and pos.item() == 1 and counter.item() == 0
    # With step records at position 2: row 1 fed token 9 (logit -1), the others greedy.
    feed = torch.full((4, 3), -1, dtype=torch.int64)
    feed[2, 1] = 9
    rec = torch.zeros(4, 3, 4, dtype=torch.int32, device=DEV)
    call("q3_argmax_rows", P(xd), V, 3, V, P(tok), P(pos), P(counter), P(dv(feed)), P(rec), 4, S())
    torch.cuda.synchronize()
    r = rec.cpu()
    assert tok.cpu().tolist() == [7, 9, 12] and pos.item() == 2
    assert r[2, :, 0].tolist() == [7, 0, 12] and r[2, :, 3].tolist() == [7, 9, 12]
    assert r[2, :, 1].view(torch.float32).tolist() == [3.0, -1.0, 2.5]
    assert r[2, :, 2].view(torch.float32).tolist() == [3.0, -1.0, 2.5]


@pytest.mark.parametrize("M", [1, 9, 16, 17, 40, 64, 100, 300])
@pytest.mark.parametrize("N,K", [(320, 1024), (1536, 320), (2560, 2560)])
def test_gemm(M, N, K):
    x, w = rnd((M, K), 1.0, M + 1), rnd((N, K), 0.02, N + K + 1)
    xd, wd = dv(x), dv(w)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    call("q3_gemm", P(xd), K, P(wd), M, N, K, _lib.EPI_STORE, P(y), N, S())
    torch.cuda.synchronize()
    check_projection(y, x, w)
    res = rnd((M, N), 1.0, 5)
    resd = dv(res)
    call("q3_gemm", P(xd), K, P(wd), M, N, K, _lib.EPI_RESID, P(resd), N, S())
    act = torch.empty(M, N // 2, dtype=torch.bfloat16, device=DEV)
    call("q3_gemm", P(xd), K, P(wd), M, N, K, _lib.EPI_SWIGLU, P(act), N // 2, S())
    torch.cuda.synchronize()
    yc = y.cpu()
    assert torch.equal(resd.cpu(), res + yc)
    assert_nearly_exact(act, oc.swiglu(yc[:, 0::2], yc[:, 1::2]), frac=5e-3)


@pytest.mark.parametrize("M,N,K,epi", [(4096, 6144, 2560, _lib.EPI_STORE), (4096, 2560, 4096, _lib.EPI_RESID),
                                       (2600, 19456, 2560, _lib.EPI_SWIGLU), (4096, 2560, 9728, _lib.EPI_RESID),
                                       (3000, 3800, 320, _lib.EPI_STORE), (40961, 4096, 64, _lib.EPI_STORE)])
def test_gemm_wide(M, N, K, epi):
    """The 256 x 256-tile path at the prompt pass's projection shapes, plus ragged
    token and weight tiles (M % 256, N % 256 != 0; an odd K step count; one K
    step): every epilogue checked on 96 sampled token rows (first, last, and
    random) against float64 dot products of the same BF16 operands, and the
    columns past N / rows past M of the output buffer untouched."""
    assert call("q3_gemm_tiles_wide", M, N) == 1
    g = torch.Generator().manual_seed(M + N + K)
    x, w = rnd((M, K), 1.0, M + 7), rnd((N, K), 0.02, N + K + 7)
    xd, wd = dv(x), dv(w)
    cols = N // 2 if epi == _lib.EPI_SWIGLU else N
    res = rnd((M, cols), 1.0, 9) if epi == _lib.EPI_RESID else torch.full((M, cols), 7.0, dtype=torch.bfloat16)
    pad = dv(torch.full((M + 1, cols + 4), 5.0, dtype=torch.bfloat16))
    pad[:M, :cols] = dv(res)
    call("q3_gemm", P(xd), K, P(wd), M, N, K, epi, P(pad), cols + 4, S())
    torch.cuda.synchronize()
    out = pad.cpu()
    assert torch.all(out[:, cols:] == 5.0) and torch.all(out[M] == 5.0)
    rows = torch.cat([torch.tensor([0, M - 1]), torch.randint(0, M, (94,), generator=g)])
    xs = x[rows]
    if epi == _lib.EPI_STORE:
        check_projection(out[rows, :N], xs, w)
        return
    # The fused epilogues against the unfused ones on the same rows: the plain
    # projection of those rows (checked above for its own bar) is recomputed
    # here through the narrow tiling, whose sums the wide path must match to
    # the same float64 bar.
    y = torch.empty(len(rows), N, dtype=torch.bfloat16, device=DEV)
    call("q3_gemm", P(dv(xs.contiguous())), K, P(wd), len(rows), N, K, _lib.EPI_STORE, P(y), N, S())
    torch.cuda.synchronize()
    yc = y.cpu()
    check_projection(yc, xs, w)
    if epi == _lib.EPI_RESID:
        want = (res[rows].float() + yc.float()).bfloat16()
        got = out[rows, :N]
        # Both round once from FP32 sums of different order: at most one BF16
        # ulp of the projection apart, on a small fraction of elements.
        diff = (got.float() - want.float()).abs()
        assert (diff > 0).float().mean() <= 0.03
        assert torch.all(diff <= 2.0 ** -7 * (want.float().abs() + yc.float().abs()) + 1e-6)
    else:
        want = oc.swiglu(yc[:, 0::2], yc[:, 1::2])
        assert_nearly_exact(out[rows, :cols], want, frac=0.06, max_ulp=2)


@pytest.mark.parametrize("M,N,K", [(4096, 6144, 2560), (2600, 19456, 2560), (3000, 3800, 320), (4100, 2576, 576)])
def test_gemm_wide_store_widths(M, N, K):
    """The wide tiling stores 16 bytes per lane (lanes regrouped by cross-row
    swaps) where the output rows allow it (ldy % 8 == 0, a 16-byte aligned
    base, N % 8, SwiGLU N % 16), else 8 (4 for SwiGLU): the same bits either
    way, every epilogue, with ragged token and weight tiles; nothing outside
    the output columns is written."""
    assert call("q3_gemm_tiles_wide", M, N) == 1
    x, w = rnd((M, K), 1.0, M + 3), rnd((N, K), 0.02, N + K + 3)
    xd, wd = dv(x), dv(w)
    for epi in (_lib.EPI_STORE, _lib.EPI_RESID, _lib.EPI_SWIGLU):
        cols = N // 2 if epi == _lib.EPI_SWIGLU else N
        res = rnd((M, cols), 1.0, 11)
        outs = []
        # ldy = cols (16-byte stores); cols + 4 (8-byte stores); ldy = cols + 8 with the rows
        # starting 8 bytes into the buffer (not 16-byte aligned: 8-byte stores).
        for pad, off in ((0, 0), (4, 0), (8, 4)):
            flat = dv(torch.full((M * (cols + pad) + off,), 5.0, dtype=torch.bfloat16))
            buf = flat[off:].view(M, cols + pad)
            buf[:, :cols] = dv(res)
            call("q3_gemm", P(xd), K, P(wd), M, N, K, epi, P(buf), cols + pad, S())
            torch.cuda.synchronize()
            out = flat.cpu()
            assert torch.all(out[:off] == 5.0)
            out = out[off:].view(M, cols + pad)
            assert torch.all(out[:, cols:] == 5.0)
            outs.append(out[:, :cols])
        assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2]), epi


@pytest.mark.parametrize("M,N,K", [(1024, 2560, 4096), (1024, 2560, 9728), (300, 2560, 4096),
                                   (2049, 2560, 640), (700, 3800, 576)])
def test_gemm_partials(M, N, K):
    """Split-K partials of the 256 x 256-tile path (prompts of 256-4095 tokens):
    at the split count q3_gemm_splits picks and at a ragged one (K steps not a
    multiple of the splits, some splits one step long), the partials summed in
    split order against float64 dot products on sampled rows (first, last,
    random), nothing written past splits * M * N floats, and
    q3_add_rmsnorm_partials on them: the residual bit-exact against the same
    split-order FP32 sum rounded on the CPU, the norm bit-exact against
    q3_rmsnorm of that residual and near the oracle's (an FP32 mean of squares
    summed in another order moves a row's scale by an ulp, and the gain's
    second rounding can double that to two BF16 ulps)."""
    steps = K // 64
    pick = call("q3_gemm_splits", M, N, K)
    assert pick >= 2
    g = torch.Generator().manual_seed(M + N + K + 1)
    x, w = rnd((M, K), 1.0, M + 31), rnd((N, K), 0.02, N + K + 31)
    res = rnd((M, N), 1.0, 33)
    gain = (1 + rnd((N,), 0.2, 34).float()).to(torch.bfloat16)
    xd, wd, gd = dv(x), dv(w), dv(gain)
    rows = torch.cat([torch.tensor([0, M - 1]), torch.randint(0, M, (62,), generator=g)])
    for splits in sorted({pick, min(7, steps)}):
        ws = dv(torch.full(((splits + 1) * M * N,), 123.0))
        call("q3_gemm_partials", P(xd), K, P(wd), M, N, K, P(ws), splits, S())
        torch.cuda.synchronize()
        part = ws.cpu()
        assert torch.all(part[splits * M * N:] == 123.0)
        part = part[:splits * M * N].view(splits, M, N)
        acc = part[0].clone()
        for s_ in range(1, splits):
            acc += part[s_]
        check_projection(acc[rows].bfloat16(), x[rows], w)
        rd = dv(res)
        y = dv(torch.empty(M, N, dtype=torch.bfloat16))
        call("q3_add_rmsnorm_partials", P(ws), splits, P(rd), P(gd), P(y), M, N, 1e-6, S())
        torch.cuda.synchronize()
        want = (res.float() + acc.bfloat16().float()).bfloat16()
        assert torch.equal(rd.cpu(), want), splits
        y_ref = dv(torch.empty(M, N, dtype=torch.bfloat16))
        call("q3_rmsnorm", P(dv(want)), N, P(gd), P(y_ref), N, M, N, 1e-6, S())
        torch.cuda.synchronize()
        assert torch.equal(y.cpu(), y_ref.cpu())
        assert_nearly_exact(y, oc.rms_norm(want, gain, 1e-6), max_ulp=2)


def wide_origin(t, tm, tn):
    """Tile t's (token, weight-row) origin in the 256 x 256 tiling's raster order."""
    per_group = 4 * tn
    grp = t // per_group
    first_m = 4 * grp
    gsz = min(4, tm - first_m)
    in_g = t - grp * per_group
    return (first_m + in_g % gsz) * 256, (in_g // gsz) * 256


@pytest.mark.parametrize("M,N,K", [(1024, 19456, 2560), (8192, 2560, 4096), (2600, 19456, 2560),
                                   (1000, 17008, 1024), (1024, 6144, 2560), (256, 19456, 2560)])
def test_gemm_ws_split_tail(M, N, K):
    """q3_gemm_ws: the tiles of the last, at most half-full round split along K
    (the last two shapes: every tile, below the 256 x 256 threshold).
    The whole tiles are q3_gemm's bits; each split tile against float64 dot
    products on sampled rows; RESID and SWIGLU on the split tiles bit-exact
    against the stored projection (the same split-order sums); nothing past N
    written (ragged M and N in the last case)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tm, tn = (M + 255) // 256, (N + 255) // 256
    tiles = tm * tn
    rem = tiles % cus
    assert 0 < rem and 2 * rem <= cus, "the shape must leave a split tail on this device"
    splits = min(cus // rem, 8, K // 64 // 4)
    assert call("q3_gemm_ws_floats", M, N, K) == rem * splits * 65536
    full = tiles - rem
    g = torch.Generator().manual_seed(M + N + K + 3)
    x, w = rnd((M, K), 1.0, M + 41), rnd((N, K), 0.02, N + K + 41)
    xd, wd = dv(x), dv(w)
    ws = dv(torch.empty(rem * splits * 65536, dtype=torch.float32))
    ref = dv(torch.empty(M, N, dtype=torch.bfloat16))
    call("q3_gemm", P(xd), K, P(wd), M, N, K, _lib.EPI_STORE, P(ref), N, S())
    pad = dv(torch.full((M, N + 4), 5.0, dtype=torch.bfloat16))
    call("q3_gemm_ws", P(xd), K, P(wd), M, N, K, _lib.EPI_STORE, P(pad), N + 4, P(ws), S())
    torch.cuda.synchronize()
    y, want = pad.cpu(), ref.cpu()
    assert torch.all(y[:, N:] == 5.0)
    y = y[:, :N].contiguous()
    split_mask = torch.zeros(M, N, dtype=torch.bool)
    for t in range(full, tiles):
        m0, n0 = wide_origin(t, tm, tn)
        split_mask[m0:m0 + 256, n0:n0 + 256] = True
        rows = torch.unique(torch.cat([torch.tensor([m0, min(m0 + 255, M - 1)]),
                                       torch.randint(m0, min(m0 + 256, M), (6,), generator=g)]))
        cols = slice(n0, min(n0 + 256, N))
        check_projection(y[rows, cols], x[rows], w[cols])
    assert torch.equal(y[~split_mask], want[~split_mask])
    res = rnd((M, N), 1.0, 43)
    rd = dv(res)
    call("q3_gemm_ws", P(xd), K, P(wd), M, N, K, _lib.EPI_RESID, P(rd), N, P(ws), S())
    act = dv(torch.empty(M, N // 2, dtype=torch.bfloat16))
    call("q3_gemm_ws", P(xd), K, P(wd), M, N, K, _lib.EPI_SWIGLU, P(act), N // 2, P(ws), S())
    act_ref = dv(torch.empty(M, N // 2, dtype=torch.bfloat16))
    call("q3_swiglu_rows", P(dv(y)), P(act_ref), M, N // 2, S())
    torch.cuda.synchronize()
    assert torch.equal(rd.cpu(), (res.float() + y.float()).bfloat16())
    assert torch.equal(act.cpu(), act_ref.cpu())


@pytest.mark.parametrize("rows,I", [(1, 8), (7, 1024), (300, 9728), (640, 9728)])
def test_swiglu_rows_matches_fused_epilogue(rows, I):
    """q3_swiglu_rows on a stored gate/up projection == the GEMM's fused SwiGLU
    epilogue, bit for bit (both round the accumulator to BF16 first); 640 rows
    take the 256 x 256-tile path."""
    K = 256
    x, w = rnd((rows, K), 1.0, rows + 11), rnd((2 * I, K), 0.05, I + 12)
    xd, wd = dv(x), dv(w)
    gu = dv(torch.empty(rows, 2 * I, dtype=torch.bfloat16))
    fused = dv(torch.empty(rows, I, dtype=torch.bfloat16))
    act = dv(torch.empty(rows, I, dtype=torch.bfloat16))
    call("q3_gemm", P(xd), K, P(wd), rows, 2 * I, K, _lib.EPI_STORE, P(gu), 2 * I, S())
    call("q3_gemm", P(xd), K, P(wd), rows, 2 * I, K, _lib.EPI_SWIGLU, P(fused), I, S())
    call("q3_swiglu_rows", P(gu), P(act), rows, I, S())
    torch.cuda.synchronize()
    assert torch.equal(act.cpu(), fused.cpu())
    g = gu.cpu()
    assert_nearly_exact(act, oc.swiglu(g[:, 0::2], g[:, 1::2]), frac=5e-3)


# -------------------------------------------------------------- attention


def attention_oracle(q, ck, cv, length, scale):
    """q [B, Hq, D] -> [B, Hq, D] over keys 0..length-1 (oracle SDPA, BF16)."""
    out = oc.attention(q.unsqueeze(2), ck[:, :, :length], cv[:, :, :length], scale, length - 1)
    return out[:, :, 0]


@pytest.mark.parametrize("B,C,pos,splits", [(1, 64, 0, 1), (1, 64, 31, 1), (2, 64, 32, 1), (1, 300, 200, 3),
                                            (3, 300, 299, 5), (2, 1536, 1100, 12), (1, 1536, 1535, 12),
                                            (2, 700, 255, 40), (1, 700, 699, 1), (2, 1000, 900, 2),
                                            (1, 2176, 2100, 2), (1, 3000, 2999, 3), (1, 1536, 1300, 1),
                                            (4, 2048, 2047, 1), (40, 300, 290, 1),
                                            # the engine's decode shapes at configs 5 and 4
                                            (8, 16512, 16500, 12), (64, 2176, 2100, 1)])
def test_attn_decode(B, C, pos, splits):
    Hq, Hkv, D = 32, 8, 128
    if B * C >= 100_000:  # a workload shape: the split count is the one the engine uses
        assert call("q3_attn_splits", B, Hkv, C) == splits
    width = (Hq + 2 * Hkv) * D
    qkv = rnd((B, width), 1.5, pos + 1)
    qw = (1 + rnd((D,), 0.2, 2).float()).to(torch.bfloat16)
    kw = (1 + rnd((D,), 0.2, 3).float()).to(torch.bfloat16)
    cos, sin = oc.rope_tables(5e6, D, max(4096, C + 1))
    ck = rnd((B, Hkv, C, D), 1.0, 4)
    cv = rnd((B, Hkv, C, D), 1.0, 5)
    ckd, cvd = ck.to(DEV), cv.to(DEV)
    pacc = torch.empty(B, Hq, splits, D, dtype=torch.float32, device=DEV)
    pml = torch.empty(B, Hq, splits, 2, dtype=torch.float32, device=DEV)
    out = torch.empty(B, Hq * D, dtype=torch.bfloat16, device=DEV)
    posd = torch.tensor([pos], dtype=torch.int64, device=DEV)
    qkvd, qwd, kwd, cosd, sind = dv(qkv), dv(qw), dv(kw), dv(cos), dv(sin)
    call("q3_attn_decode", P(qkvd), width, None, 0, P(qwd), P(kwd), P(cosd), P(sind),
         P(posd), P(ckd), P(cvd), P(pacc), P(pml), None, B, Hq, Hkv, C, splits, 1e-6, D ** -0.5, S())
    call("q3_attn_merge", P(pacc), P(pml), P(out), B, Hq, splits, S())
    # A second call (the row at pos now already holds the new key): same bits.
    again = torch.empty_like(out)
    call("q3_attn_decode", P(qkvd), width, None, 0, P(qwd), P(kwd), P(cosd), P(sind),
         P(posd), P(ckd), P(cvd), P(pacc), P(pml), None, B, Hq, Hkv, C, splits, 1e-6, D ** -0.5, S())
    call("q3_attn_merge", P(pacc), P(pml), P(again), B, Hq, splits, S())
    torch.cuda.synchronize()
    assert torch.equal(again.cpu(), out.cpu())
    if splits == 1:  # direct output: what the merge kernel writes for one split
        direct = torch.empty_like(out)
        call("q3_attn_decode", P(qkvd), width, None, 0, P(qwd), P(kwd), P(cosd), P(sind), P(posd), P(ckd),
             P(cvd), None, None, P(direct), B, Hq, Hkv, C, 1, 1e-6, D ** -0.5, S())
        torch.cuda.synchronize()
        assert torch.equal(direct.cpu(), out.cpu())
    x = qkv.view(B, 1, Hq + 2 * Hkv, D)
    c, s_ = cos[pos].view(1, 1, 1, D), sin[pos].view(1, 1, 1, D)
    q = oc.apply_rope(oc.rms_norm(x[:, :, :Hq], qw, 1e-6), c, s_)[:, 0]
    k = oc.apply_rope(oc.rms_norm(x[:, :, Hq:Hq + Hkv], kw, 1e-6), c, s_)[:, 0]
    ck_ref, cv_ref = ck.clone(), cv.clone()
    ck_ref[:, :, pos] = k
    cv_ref[:, :, pos] = x[:, 0, Hq + Hkv:]
    # The append: exactly one slot changes.
    got_k, got_v = ckd.cpu(), cvd.cpu()
    assert torch.equal(got_v, cv_ref)
    other = torch.ones(C, dtype=torch.bool)
    other[pos] = False
    assert torch.equal(got_k[:, :, other], ck[:, :, other])
    assert_nearly_exact(got_k[:, :, pos], k, frac=5e-3, max_ulp=2)
    want = attention_oracle(q, ck_ref, cv_ref, pos + 1, D ** -0.5).float()
    got = out.cpu().view(B, Hq, D).float()
    err = (got - want).abs()
    assert (err <= 1e-2 + 1e-2 * want.abs()).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("B,T,start", [(1, 1, 0), (2, 37, 0), (1, 64, 0), (2, 20, 30), (3, 50, 13), (1, 300, 0),
                                       (2, 130, 70), (1, 1000, 24), (1, 97, 4000), (16, 256, 0), (4, 600, 9),
                                       (16, 600, 0), (8, 1024, 512)])
def test_attn_prefill(B, T, start):
    """Chunks at offset `start` over a cache of start + T + 5 slots: one and many
    64-key blocks, blocks crossing the diagonal of some but not all queries, a
    ragged last query block, and a long prefix with a short chunk.  Grids of
    fewer than 512 32-query workgroups take 16-query workgroups; the last four
    shapes take 32 (the last two in grids of 2048 or more, over several XCD
    ranges)."""
    Hq, Hkv, D = 32, 8, 128
    C = start + T + 5
    q = rnd((B * T, Hq, D), 1.0, T)
    ck = rnd((B, Hkv, C, D), 1.0, T + 1)
    cv = rnd((B, Hkv, C, D), 1.0, T + 2)
    out = torch.empty(B * T, Hq * D, dtype=torch.bfloat16, device=DEV)
    call("q3_attn_prefill", P(dv(q)), P(dv(ck)), P(dv(cv)), P(out), B, T, start, Hq, Hkv, C,
         D ** -0.5, S())
    torch.cuda.synchronize()
    qt = q.view(B, T, Hq, D).transpose(1, 2)
    want = oc.attention(qt, ck[:, :, :start + T], cv[:, :, :start + T], D ** -0.5, start)
    want = want.transpose(1, 2).reshape(B * T, Hq * D).float()
    got = out.cpu().float()
    err = (got - want).abs()
    assert (err <= 1e-2 + 1e-2 * want.abs()).all(), f"max err {err.max():.3e}"


def test_graph_capture_replays_self_feeding_step():
    """A captured argmax_finish advances pos on every replay (the decode loop's feed)."""
    stream = torch.cuda.Stream()
    pv = torch.tensor([[1.0], [3.0], [3.0]], device=DEV)
    pi = torch.tensor([[5], [9], [2]], dtype=torch.int32, device=DEV)
    tok = torch.zeros(1, dtype=torch.int64, device=DEV)
    pos = torch.zeros(1, dtype=torch.int64, device=DEV)
    import ctypes
    torch.cuda.synchronize()
    call("q3_graph_begin", stream.cuda_stream)
    finish(pv, pi, 3, 1, tok, pos, stream=stream.cuda_stream)
    ex = ctypes.c_void_p()
    call("q3_graph_end", stream.cuda_stream, ctypes.byref(ex))
    for _ in range(3):
        call("q3_graph_launch", ex.value, stream.cuda_stream)
    stream.synchronize()
    call("q3_graph_destroy", ex.value)
    assert tok.item() == 2 and pos.item() == 3


@pytest.mark.parametrize("N,K", [(16, 32), (48, 96), (2560, 9728)])
def test_tile16_layout(N, K):
    """(n, k) -> ((n/16 * K/32 + k/32) * 64 + (k%32)/8 * 16 + n%16) * 8 + k%8."""
    w = torch.arange(N * K, dtype=torch.int32).remainder(65521).to(torch.int16).view(torch.bfloat16).reshape(N, K)
    out = torch.empty_like(dv(w))
    call("q3_tile16", P(dv(w)), N, K, P(out), S())
    torch.cuda.synchronize()
    want = w.view(torch.int16).reshape(N // 16, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(N, K)
    assert torch.equal(out.cpu().view(torch.int16), want)
    n, k = N - 3, K - 7  # one element by the closed form
    flat = out.cpu().view(torch.int16).reshape(-1)
    assert flat[((n // 16 * (K // 32) + k // 32) * 64 + (k % 32) // 8 * 16 + n % 16) * 8 + k % 8] == w.view(torch.int16)[n, k]


@pytest.mark.parametrize("M", [1, 5, 9, 16, 17, 33, 64])
@pytest.mark.parametrize("N,K", [(128, 256), (192, 768), (512, 1024), (2560, 4096), (6144, 2560), (2560, 9728),
                                 (19456, 2560)])
def test_skinny(M, N, K):
    """Weight-streaming MFMA projection (split-K + fixed-order reduce on narrow N)."""
    x, w = rnd((M, K), 1.0, M + 7), rnd((N, K), 0.02, N + K + 7)
    xd, wd = dv(x), dv(w)
    splits = call("q3_skinny_splits", M, N, K)
    ws = torch.empty(splits * M * N, dtype=torch.float32, device=DEV)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    call("q3_skinny", P(xd), K, P(wd), M, N, K, _lib.EPI_STORE, P(y), N, P(ws), S())
    torch.cuda.synchronize()
    check_projection(y, x, w)
    # The tiled layout feeds the same operands in the same order: identical bits.
    wt = torch.empty_like(wd)
    call("q3_tile16", P(wd), N, K, P(wt), S())
    yt = torch.empty_like(y)
    call("q3_skinny_tiled", P(xd), K, P(wt), M, N, K, _lib.EPI_STORE, P(yt), N, P(ws), S())
    torch.cuda.synchronize()
    assert torch.equal(yt, y)
    # Partials only: summed in split order they round to the same bits.
    call("q3_skinny_partials", P(xd), K, P(wt), M, N, K, P(ws), S())
    torch.cuda.synchronize()
    part = ws.view(splits, M, N).cpu()
    acc = part[0].clone()
    for sp in range(1, splits):
        acc += part[sp]
    assert torch.equal(acc.to(torch.bfloat16), y.cpu())
    res = rnd((M, N), 1.0, 9)
    resd = dv(res)
    call("q3_skinny", P(xd), K, P(wd), M, N, K, _lib.EPI_RESID, P(resd), N, P(ws), S())
    act = torch.empty(M, N // 2, dtype=torch.bfloat16, device=DEV)
    call("q3_skinny", P(xd), K, P(wd), M, N, K, _lib.EPI_SWIGLU, P(act), N // 2, P(ws), S())
    torch.cuda.synchronize()
    yc = y.cpu()
    assert torch.equal(resd.cpu(), res + yc)
    assert_nearly_exact(act, oc.swiglu(yc[:, 0::2], yc[:, 1::2]), frac=5e-3)


@pytest.mark.parametrize("M", [1, 5, 16, 33, 64])
@pytest.mark.parametrize("N,K", [(1024, 512), (151936, 256)])
def test_skinny_argmax(M, N, K):
    """LM-head epilogue: per-workgroup maxima + q3_argmax_finish = first-index argmax of the BF16 logits."""
    assert call("q3_skinny_splits", M, N, K) == 1
    x, w = rnd((M, K), 1.0, M + 3), rnd((N, K), 0.02, 11)
    # Two identical dominant rows in different workgroups: the lower index must win.
    w[7] = w[N - 1] = (w[7].float() * 4).to(torch.bfloat16)
    wt = torch.empty(N, K, dtype=torch.bfloat16, device=DEV)
    call("q3_tile16", P(dv(w)), N, K, P(wt), S())
    xd = dv(x)
    want = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(M * N, dtype=torch.float32, device=DEV)
    call("q3_skinny_tiled", P(xd), K, P(wt), M, N, K, _lib.EPI_STORE, P(want), N, P(ws), S())
    parts = N // 64
    pv = torch.empty(parts, M, dtype=torch.float32, device=DEV)
    pi = torch.empty(parts, M, dtype=torch.int32, device=DEV)
    logits = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    tok = torch.empty(M, dtype=torch.int64, device=DEV)
    for store in (False, True):
        call("q3_skinny_argmax", P(xd), K, P(wt), M, N, K, P(logits) if store else None, N, P(pv), P(pi),
             None, None, None, 0, S())
        finish(pv, pi, parts, M, tok)
        torch.cuda.synchronize()
        ref = want.cpu().float()
        assert torch.equal(tok.cpu(), ref.argmax(dim=1)), store
        if store:
            assert torch.equal(logits.cpu(), want.cpu())
    assert (ref[:, 7] == ref[:, N - 1]).all()
    # Step records at position 3 (input at 2): every row fed a chosen token.
    feed = torch.full((5, M), -1, dtype=torch.int64)
    feed[3] = torch.randint(0, N, (M,), generator=torch.Generator().manual_seed(M))
    feedd, rec = dv(feed), torch.zeros(5, M, 4, dtype=torch.int32, device=DEV)
    pos, counter = dv(torch.tensor([2])), torch.zeros(1, dtype=torch.int32, device=DEV)
    call("q3_skinny_argmax", P(xd), K, P(wt), M, N, K, None, N, P(pv), P(pi), P(pos), P(feedd), P(rec), 5, S())
    finish(pv, pi, parts, M, tok, pos, counter, feedd, rec)
    torch.cuda.synchronize()
    r = rec.cpu()
    assert tok.cpu().tolist() == feed[3].tolist() == r[3, :, 3].tolist()
    assert r[3, :, 0].tolist() == ref.argmax(dim=1).tolist()
    assert torch.equal(r[3, :, 1].view(torch.float32), ref.max(dim=1).values)
    assert torch.equal(r[3, :, 2].view(torch.float32), ref.gather(1, feed[3].view(M, 1))[:, 0])
    assert pos.item() == 3 and counter.item() == 0


@pytest.mark.parametrize("M,N,K", [(5, 2560, 4096), (16, 2560, 9728), (64, 2560, 9728), (64, 2560, 4096),
                                   (40, 2560, 4096), (9, 512, 1024)])
def test_add_rmsnorm_partials(M, N, K):
    """Partials + residual + RMSNorm in one kernel == RESID epilogue then q3_rmsnorm, bit for bit."""
    x, w = rnd((M, K), 1.0, 21), rnd((N, K), 0.02, 22)
    res = rnd((M, N), 1.0, 23)
    gain = (1 + rnd((N,), 0.2, 24).float()).to(torch.bfloat16)
    wt = torch.empty(N, K, dtype=torch.bfloat16, device=DEV)
    call("q3_tile16", P(dv(w)), N, K, P(wt), S())
    splits = call("q3_skinny_splits", M, N, K)
    ws = torch.empty(splits * M * N, dtype=torch.float32, device=DEV)
    xd, gd = dv(x), dv(gain)
    r1, r2 = dv(res), dv(res)
    y1 = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    y2 = torch.empty_like(y1)
    call("q3_skinny_tiled", P(xd), K, P(wt), M, N, K, _lib.EPI_RESID, P(r1), N, P(ws), S())
    call("q3_rmsnorm", P(r1), N, P(gd), P(y1), N, M, N, 1e-6, S())
    call("q3_skinny_partials", P(xd), K, P(wt), M, N, K, P(ws), S())
    call("q3_add_rmsnorm_partials", P(ws), splits, P(r2), P(gd), P(y2), M, N, 1e-6, S())
    torch.cuda.synchronize()
    assert torch.equal(r1.cpu(), r2.cpu()) and torch.equal(y1.cpu(), y2.cpu())
    assert not torch.equal(r2.cpu(), res)


def test_attn_fused_applies_to_four_wave_shapes():
    """The fused launch takes shapes whose attention runs four-wave workgroups
    and whose grid is resident at once; eight-wave shapes keep two launches."""
    assert call("q3_attn_fused_grid", 1, 32, 8, 1536, 12) == 1 * (12 * 8 + 16)
    assert call("q3_attn_fused_grid", 4, 32, 8, 1536, 6) == 0     # 256 keys per split: eight waves
    assert call("q3_attn_fused_grid", 1, 32, 8, 4096, 16) == 0    # likewise
    assert call("q3_attn_fused_grid", 1, 32, 8, 1536, 1) == 0
    assert call("q3_attn_fused_grid", 1, 32, 8, 1536, 17) == 0
    assert call("q3_attn_fused_grid", 4, 32, 8, 2048, 12) == 4 * (12 * 8 + 16)  # two per CU
    assert call("q3_attn_fused_grid", 64, 32, 8, 2048, 16) == 0   # 9216 workgroups: not resident


@pytest.mark.parametrize("B,C,pos,splits,qsplits", [(1, 1536, 1100, 12, 0), (1, 1536, 1535, 12, 0),
                                                    (2, 700, 255, 4, 0), (4, 1536, 1000, 8, 0),
                                                    (1, 300, 0, 2, 0), (1, 64, 63, 2, 0), (3, 900, 640, 5, 3),
                                                    (1, 2000, 1999, 16, 9), (4, 2048, 2000, 12, 0)])
def test_attn_decode_fused(B, C, pos, splits, qsplits):
    """Attention + merge in one launch == q3_attn_decode then q3_attn_merge, bit
    for bit, over several layers' flags; a zeroed exchange buffer makes a
    repeated (position, layer) safe."""
    Hq, Hkv, D = 32, 8, 128
    width = (Hq + 2 * Hkv) * D
    assert call("q3_attn_fused_grid", B, Hq, Hkv, C, splits) > 0
    qw = (1 + rnd((D,), 0.2, 2).float()).to(torch.bfloat16)
    kw = (1 + rnd((D,), 0.2, 3).float()).to(torch.bfloat16)
    cos, sin = oc.rope_tables(5e6, D, max(4096, C + 1))
    ck, cv = rnd((B, Hkv, C, D), 1.0, 4), rnd((B, Hkv, C, D), 1.0, 5)
    posd = dv(torch.tensor([pos]))
    xbuf = torch.zeros(call("q3_attn_xbuf_words", B, Hq, splits), dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    for layer, seed in ((0, 7), (1, 8), (0, 9)):
        if layer == 0 and seed == 9:
            xbuf.zero_()  # the same (position, layer) as the first round
        if qsplits:
            part = (torch.randn(qsplits, B, width, generator=torch.Generator().manual_seed(seed)) * 0.7).float()
            src = (None, width, P(dv(part)), qsplits)
        else:
            src = (P(dv(rnd((B, width), 1.5, seed))), width, None, 0)
        outs, caches = [], []
        for fused in (False, True):
            ckd, cvd = dv(ck), dv(cv)
            out = torch.empty(B, Hq * D, dtype=torch.bfloat16, device=DEV)
            if fused:
                call("q3_attn_decode_fused", *src, P(dv(qw)), P(dv(kw)), P(dv(cos)), P(dv(sin)), P(posd),
                     P(ckd), P(cvd), P(xbuf), P(out), B, Hq, Hkv, C, splits, layer, 1e-6, D ** -0.5, P(err), S())
            else:
                pacc = torch.empty(B, Hq, splits, D, dtype=torch.float32, device=DEV)
                pml = torch.empty(B, Hq, splits, 2, dtype=torch.float32, device=DEV)
                call("q3_attn_decode", *src, P(dv(qw)), P(dv(kw)), P(dv(cos)), P(dv(sin)), P(posd), P(ckd),
                     P(cvd), P(pacc), P(pml), None, B, Hq, Hkv, C, splits, 1e-6, D ** -0.5, S())
                call("q3_attn_merge", P(pacc), P(pml), P(out), B, Hq, splits, S())
            torch.cuda.synchronize()
            outs.append(out.cpu())
            caches.append((ckd.cpu(), cvd.cpu()))
        assert torch.equal(outs[0], outs[1]), (layer, seed)
        assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])
    assert err.item() == 0


def test_attn_decode_fused_rejects_layers_past_its_flag():
    """The exchange flag holds (position, layer) with layer < 64: the launcher
    refuses layer 64 and a negative layer before anything is enqueued, and the
    engine keeps two launches for deeper models."""
    Hq, Hkv, D, B, C, splits = 32, 8, 128, 1, 1536, 12
    assert call("q3_attn_fused_grid", B, Hq, Hkv, C, splits) > 0
    qkv = torch.zeros(B, (Hq + 2 * Hkv) * D, dtype=torch.bfloat16, device=DEV)
    gain = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    cos, sin = oc.rope_tables(5e6, D, C + 1)
    cos, sin = dv(cos), dv(sin)
    posd = dv(torch.tensor([5]))
    ck = torch.zeros(B, Hkv, C, D, dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    xbuf = torch.zeros(call("q3_attn_xbuf_words", B, Hq, splits), dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.full((B, Hq * D), 7.0, dtype=torch.bfloat16, device=DEV)
    for layer in (64, -1):
        with pytest.raises(RuntimeError):
            call("q3_attn_decode_fused", P(qkv), qkv.shape[1], None, 0, P(gain), P(gain), P(cos), P(sin), P(posd),
                 P(ck), P(cv), P(xbuf), P(out), B, Hq, Hkv, C, splits, layer, 1e-6, D ** -0.5, P(err), S())
    torch.cuda.synchronize()
    assert bool((out.float() == 7.0).all()) and int(ck.abs().sum()) == 0 and err.item() == 0


@pytest.mark.parametrize("B,Hkv,C,pos,qsplits", [(16, 8, 768, 600, 0),    # config 3's shape
                                                  (16, 8, 768, 383, 5),    # split 1 holds no key yet
                                                  (16, 8, 768, 384, 0),    # its first key
                                                  (16, 8, 1024, 1023, 5),
                                                  (16, 8, 4096, 4000, 9),  # partials summed by the loop
                                                  (64, 2, 600, 599, 3)])   # the tile test model at 64 rows
def test_attn_decode_pair_matches_two_splits_and_merge(B, Hkv, C, pos, qsplits):
    """Two splits in one launch, split 0 folding split 1's flagged record ==
    q3_attn_decode with two splits then q3_attn_merge, bit for bit, output and
    caches, over several layers' flags; a zeroed exchange buffer makes a
    repeated (position, layer) safe."""
    Hq, D = 4 * Hkv, 128
    width = (Hq + 2 * Hkv) * D
    assert call("q3_attn_splits", B, Hkv, C) == 1
    assert call("q3_attn_pair_grid", B, Hq, Hkv, C) == 2 * B * Hkv
    qw = (1 + rnd((D,), 0.2, 2).float()).to(torch.bfloat16)
    kw = (1 + rnd((D,), 0.2, 3).float()).to(torch.bfloat16)
    cos, sin = oc.rope_tables(5e6, D, max(4096, C + 1))
    ck, cv = rnd((B, Hkv, C, D), 1.0, 4), rnd((B, Hkv, C, D), 1.0, 5)
    posd = dv(torch.tensor([pos]))
    xbuf = torch.zeros(call("q3_attn_xbuf_words", B, Hq, 2), dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    for layer, seed in ((0, 7), (1, 8), (0, 9)):
        if layer == 0 and seed == 9:
            xbuf.zero_()  # the same (position, layer) as the first round
        if qsplits:
            part = (torch.randn(qsplits, B, width, generator=torch.Generator().manual_seed(seed)) * 0.7).float()
            src = (None, width, P(dv(part)), qsplits)
        else:
            src = (P(dv(rnd((B, width), 1.5, seed))), width, None, 0)
        outs, caches = [], []
        for pair in (False, True):
            ckd, cvd = dv(ck), dv(cv)
            out = torch.empty(B, Hq * D, dtype=torch.bfloat16, device=DEV)
            if pair:
                call("q3_attn_decode_pair", *src, P(dv(qw)), P(dv(kw)), P(dv(cos)), P(dv(sin)), P(posd), P(ckd),
                     P(cvd), P(xbuf), P(out), B, Hq, Hkv, C, layer, 1e-6, D ** -0.5, P(err), S())
            else:
                pacc = torch.empty(B, Hq, 2, D, dtype=torch.float32, device=DEV)
                pml = torch.empty(B, Hq, 2, 2, dtype=torch.float32, device=DEV)
                call("q3_attn_decode", *src, P(dv(qw)), P(dv(kw)), P(dv(cos)), P(dv(sin)), P(posd), P(ckd),
                     P(cvd), P(pacc), P(pml), None, B, Hq, Hkv, C, 2, 1e-6, D ** -0.5, S())
                call("q3_attn_merge", P(pacc), P(pml), P(out), B, Hq, 2, S())
            torch.cuda.synchronize()
            outs.append(out.cpu())
            caches.append((ckd.cpu(), cvd.cpu()))
        assert torch.equal(outs[0], outs[1]), (layer, seed)
        assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])
    assert err.item() == 0


def test_attn_pair_applies_where_one_split_leaves_cus_idle():
    """The pair launch takes 65-128 (sequence, KV head) pairs where the split
    policy keeps one split, with at least 256 keys per half."""
    assert call("q3_attn_pair_grid", 16, 32, 8, 768) == 256
    assert call("q3_attn_pair_grid", 16, 32, 8, 4096) == 256
    assert call("q3_attn_pair_grid", 16, 32, 8, 4200) == 0   # more than 4096 keys: several splits
    assert call("q3_attn_pair_grid", 16, 32, 8, 480) == 256  # 240 keys per half, ranges rounded to 256
    assert call("q3_attn_pair_grid", 16, 32, 8, 448) == 0    # under 256 keys per half
    assert call("q3_attn_pair_grid", 64, 32, 8, 2176) == 0   # 512 pairs fill the CUs with one split
    assert call("q3_attn_pair_grid", 8, 32, 8, 16512) == 0
    assert call("q3_attn_pair_grid", 1, 32, 8, 1536) == 0


@pytest.mark.parametrize("B,Hkv,K,C,pos,splits,embed", [
    (1, 8, 2560, 1536, 1100, 16, False),   # config 2's shape: 16 splits of 96 keys
    (1, 8, 2560, 1536, 1535, 12, True),    # last slot, layer 0's embedding prologue
    (2, 8, 2560, 700, 255, 4, False),
    (2, 8, 2560, 900, 640, 5, True),
    (1, 8, 2560, 300, 0, 2, False),        # first position: the new key is the only one
    (1, 8, 2560, 64, 63, 2, False),
    (1, 2, 512, 300, 200, 3, True),        # the tile test model's widths
    (2, 2, 512, 700, 650, 6, False)])
def test_qkv_attn_matches_projection_then_fused_attention(B, Hkv, K, C, pos, splits, embed):
    """q3_qkv_attn == q3_gemv (X_NORM / X_EMBED_NORM, EPI_STORE) then
    q3_attn_decode_fused, bit for bit: attention output, both caches and the
    embedding rows copied to the residual; at one row also with the o
    projection in the launch == that then q3_gemv (X_PLAIN, EPI_RESID) on the
    residual.  Over several layers' flags, and again after the exchange words
    are zeroed at a repeated (position, layer)."""
    Hq, D = 4 * Hkv, 128
    N, KO = (Hq + 2 * Hkv) * D, Hq * D
    assert call("q3_qkv_attn_grid", B, Hq, Hkv, C, splits, K, 0) > 0
    with_o = call("q3_qkv_attn_grid", B, Hq, Hkv, C, splits, K, 1) > 0
    assert with_o == (B == 1)
    qw = dv((1 + rnd((D,), 0.2, 2).float()).to(torch.bfloat16))
    kw = dv((1 + rnd((D,), 0.2, 3).float()).to(torch.bfloat16))
    cos, sin = oc.rope_tables(5e6, D, max(4096, C + 1))
    cos, sin = dv(cos), dv(sin)
    ck, cv = rnd((B, Hkv, C, D), 1.0, 4), rnd((B, Hkv, C, D), 1.0, 5)
    posd = dv(torch.tensor([pos]))
    V = 1000
    table = dv(rnd((V, K), 0.5, 6))
    ids = dv(torch.randint(0, V, (B,), generator=torch.Generator().manual_seed(7)))
    xbufs = [torch.zeros(call("q3_attn_xbuf_words", B, Hq, splits), dtype=torch.int32, device=DEV) for _ in range(3)]
    qxs = [torch.zeros(B * N, dtype=torch.int32, device=DEV) for _ in range(2)]
    ox = torch.zeros(B * KO, dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    xm = _lib.X_EMBED_NORM if embed else _lib.X_NORM
    for layer, seed in ((0, 11), (1, 12), (0, 13)):
        if layer == 0 and seed == 13:  # the same (position, layer) as the first round
            for t in xbufs + qxs + [ox]:
                t.zero_()
        x = rnd((B, K), 1.5, seed)
        g = dv((1 + rnd((K,), 0.2, seed + 50).float()).to(torch.bfloat16))
        w = dv(rnd((N, K), 0.05, seed + 100))
        wo = dv(rnd((K, KO), 0.05, seed + 200))
        runs = []
        for mode in ("separate", "fused", "fused_o") if with_o else ("separate", "fused"):
            ckd, cvd = dv(ck), dv(cv)
            out = torch.zeros(B, Hq * D, dtype=torch.bfloat16, device=DEV)
            # The residual stream: the norm prologue's input, joined in place by o.
            resid = dv(x) if not embed else torch.zeros(B, K, dtype=torch.bfloat16, device=DEV)
            src = table if embed else resid
            if mode == "separate":
                qkv = torch.empty(B, N, dtype=torch.bfloat16, device=DEV)
                gemv(xm, src, K, w, B, N, K, _lib.EPI_STORE, qkv, N, ids=ids if embed else None, norm_w=g,
                     resid_out=resid if embed else None)
                call("q3_attn_decode_fused", P(qkv), N, None, 0, P(qw), P(kw), P(cos), P(sin), P(posd), P(ckd),
                     P(cvd), P(xbufs[0]), P(out), B, Hq, Hkv, C, splits, layer, 1e-6, D ** -0.5, P(err), S())
                if with_o:
                    gemv(_lib.X_PLAIN, out, KO, wo, B, K, KO, _lib.EPI_RESID, resid, K)
            else:
                o = mode == "fused_o"
                # With o, also the L2 hint for a following gate/up GEMV (no effect on results).
                call("q3_qkv_attn", xm, P(src), K, P(ids) if embed else None, P(g), 1e-6,
                     P(resid) if embed or o else None, P(w), K, P(qxs[o]), P(qw), P(kw), P(cos), P(sin), P(posd),
                     P(ckd), P(cvd), P(xbufs[1 + o]), None if o else P(out), P(wo) if o else None,
                     P(ox) if o else None, P(w) if o else None, N, 16, B, Hq, Hkv, C, splits, layer, D ** -0.5,
                     P(err), S())
                if not o and with_o:
                    gemv(_lib.X_PLAIN, out, KO, wo, B, K, KO, _lib.EPI_RESID, resid, K)
            torch.cuda.synchronize()
            runs.append((mode, out.cpu(), ckd.cpu(), cvd.cpu(), resid.cpu()))
        ref = runs[0]
        for mode, out, k_, v_, r_ in runs[1:]:
            if mode != "fused_o":
                assert torch.equal(out, ref[1]), (mode, layer, seed)
            assert torch.equal(k_, ref[2]) and torch.equal(v_, ref[3]), (mode, layer, seed)
            assert torch.equal(r_, ref[4]), (mode, layer, seed)
        # Every projected row and attention output reached the exchange words with this step's flag.
        flag = 1 + (pos * 64 + layer) % 65535
        for t in [qxs[0]] + ([qxs[1], ox] if with_o else []):
            assert (t.cpu().numpy().view(np.uint32) >> 16 == flag).all()
    assert err.item() == 0


@pytest.mark.parametrize("Hkv,K,I,C,pos,splits", [
    (8, 2560, 9728, 1536, 1100, 16),  # config 2's shape
    (8, 2560, 9728, 1536, 1535, 16),  # last slot
    (8, 2560, 9728, 64, 0, 2),        # config 1's grid (224: 11-12 down rows a workgroup), first position
    (2, 512, 1024, 300, 200, 3)])     # the tile test model's widths
def test_down_qkv_attn_matches_down_then_qkv_attn(Hkv, K, I, C, pos, splits):
    """q3_down_qkv_attn == q3_gemv (X_PLAIN, EPI_RESID: the previous layer's
    down projection and residual join) then q3_qkv_attn (X_NORM, with the o
    projection), bit for bit: the residual after the o join, both caches and
    the q|k|v and attention-output words; the down words rx hold the joined
    residual with this step's flag.  Over several layers' flags, and again
    after the exchange words are zeroed at a repeated (position, layer)."""
    Hq, D, B = 4 * Hkv, 128, 1
    N, KO = (Hq + 2 * Hkv) * D, Hq * D
    assert call("q3_down_qkv_attn_grid", Hq, Hkv, C, splits, K, I) > 0
    n_down = call("q3_down_qkv_attn_grid", Hq, Hkv, C, splits, K, I)  # every workgroup has down rows
    qw = dv((1 + rnd((D,), 0.2, 2).float()).to(torch.bfloat16))
    kw = dv((1 + rnd((D,), 0.2, 3).float()).to(torch.bfloat16))
    cos, sin = oc.rope_tables(5e6, D, max(4096, C + 1))
    cos, sin = dv(cos), dv(sin)
    ck, cv = rnd((B, Hkv, C, D), 1.0, 4), rnd((B, Hkv, C, D), 1.0, 5)
    posd = dv(torch.tensor([pos]))
    words = call("q3_attn_xbuf_words", B, Hq, splits)
    xbufs = [torch.zeros(words, dtype=torch.int32, device=DEV) for _ in range(2)]
    qxs = [torch.zeros(N, dtype=torch.int32, device=DEV) for _ in range(2)]
    oxs = [torch.zeros(KO, dtype=torch.int32, device=DEV) for _ in range(2)]
    rx = torch.zeros(call("q3_down_rx_words", K), dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    for layer, seed in ((1, 21), (2, 22), (1, 23)):
        if seed == 23:  # the same (position, layer) as the first round
            for t in xbufs + qxs + oxs + [rx]:
                t.zero_()
        resid0 = rnd((B, K), 1.5, seed)
        act = dv(rnd((B, I), 0.5, seed + 1))
        wd = dv(rnd((K, I), 0.02, seed + 2))
        g = dv((1 + rnd((K,), 0.2, seed + 50).float()).to(torch.bfloat16))
        w = dv(rnd((N, K), 0.05, seed + 100))
        wo = dv(rnd((K, KO), 0.05, seed + 200))
        runs = []
        for joined in (False, True):
            ckd, cvd = dv(ck), dv(cv)
            resid = dv(resid0)
            if not joined:
                gemv(_lib.X_PLAIN, act, I, wd, B, K, I, _lib.EPI_RESID, resid, K)
                torch.cuda.synchronize()
                after_down = resid.cpu()
                call("q3_qkv_attn", _lib.X_NORM, P(resid), K, None, P(g), 1e-6, P(resid), P(w), K, P(qxs[0]),
                     P(qw), P(kw), P(cos), P(sin), P(posd), P(ckd), P(cvd), P(xbufs[0]), None, P(wo), P(oxs[0]),
                     P(w), N, 16, B, Hq, Hkv, C, splits, layer, D ** -0.5, P(err), S())
            else:
                call("q3_down_qkv_attn", P(act), P(wd), I, P(rx), P(resid), P(g), 1e-6, P(w), K, P(qxs[1]),
                     P(qw), P(kw), P(cos), P(sin), P(posd), P(ckd), P(cvd), P(xbufs[1]), P(wo), P(oxs[1]), P(w),
                     N, 16, Hq, Hkv, C, splits, layer, D ** -0.5, P(err), S())
            torch.cuda.synchronize()
            runs.append((resid.cpu(), ckd.cpu(), cvd.cpu()))
        (r0, k0, v0), (r1, k1, v1) = runs
        assert torch.equal(r1, r0) and torch.equal(k1, k0) and torch.equal(v1, v0), (layer, seed)
        assert torch.equal(qxs[1], qxs[0]) and torch.equal(oxs[1], oxs[0]), (layer, seed)
        flag = 1 + (pos * 64 + layer) % 65535
        rxv = rx.cpu().numpy().view(np.uint32)
        assert (rxv[:K + n_down] >> 16 == flag).all()
        assert np.array_equal((rxv[:K] & 0xffff).astype(np.uint16), after_down.view(torch.int16).numpy()
                              .view(np.uint16).reshape(-1))
    assert err.item() == 0


def test_down_qkv_attn_refuses_what_it_is_not_built_for():
    """Other widths, and a layer past the flag's field, are refused before
    anything is enqueued."""
    assert call("q3_down_qkv_attn_grid", 32, 8, 1536, 16, 2560, 9728) == 256
    assert call("q3_down_qkv_attn_grid", 32, 8, 64, 2, 2560, 9728) == 224   # 11-12 down rows a workgroup
    assert call("q3_down_qkv_attn_grid", 32, 8, 1536, 16, 2560, 8192) == 0
    assert call("q3_down_qkv_attn_grid", 32, 8, 1536, 1, 2560, 9728) == 0   # one split: no fused attention
    assert call("q3_down_qkv_attn_grid", 32, 8, 1536, 16, 4096, 9728) == 0
    Hq, Hkv, D, C, splits, K, I = 32, 8, 128, 1536, 16, 2560, 9728
    N = (Hq + 2 * Hkv) * D
    z = lambda *shape: torch.zeros(*shape, dtype=torch.bfloat16, device=DEV)  # noqa: E731
    act, wd, resid, w, wo, gain = z(I), z(K, I), z(K), z(N, K), z(K, Hq * D), z(K)
    cos, sin = dv(oc.rope_tables(5e6, D, C + 1)[0]), dv(oc.rope_tables(5e6, D, C + 1)[1])
    ck, cv = z(1, Hkv, C, D), z(1, Hkv, C, D)
    posd = dv(torch.tensor([5]))
    xbuf = torch.zeros(call("q3_attn_xbuf_words", 1, Hq, splits), dtype=torch.int32, device=DEV)
    qx = torch.zeros(N, dtype=torch.int32, device=DEV)
    ox = torch.zeros(Hq * D, dtype=torch.int32, device=DEV)
    rx = torch.zeros(call("q3_down_rx_words", K), dtype=torch.int32, device=DEV)
    for layer, ii in ((64, I), (-1, I), (3, 8192)):
        with pytest.raises(RuntimeError):
            call("q3_down_qkv_attn", P(act), P(wd), ii, P(rx), P(resid), P(gain), 1e-6, P(w), K, P(qx), P(gain),
                 P(gain), P(cos), P(sin), P(posd), P(ck), P(cv), P(xbuf), P(wo), P(ox), None, 0, 0, Hq, Hkv, C,
                 splits, layer, D ** -0.5, None, S())
    torch.cuda.synchronize()
    assert int(rx.abs().sum()) == 0 and int(qx.abs().sum()) == 0 and int(ck.float().abs().sum()) == 0


def test_qkv_attn_refuses_what_it_is_not_built_for():
    """Three rows, other widths, the o projection at two rows and layers past
    the flag's field are refused before anything is enqueued."""
    assert call("q3_qkv_attn_grid", 1, 32, 8, 1536, 16, 2560, 0) > 0
    assert call("q3_qkv_attn_grid", 1, 32, 8, 1536, 16, 2560, 1) > 0
    assert call("q3_qkv_attn_grid", 2, 32, 8, 700, 4, 2560, 1) == 0
    assert call("q3_qkv_attn_grid", 3, 32, 8, 1536, 6, 2560, 0) == 0
    assert call("q3_qkv_attn_grid", 1, 32, 8, 1536, 16, 4096, 0) == 0
    assert call("q3_qkv_attn_grid", 1, 32, 8, 1536, 1, 2560, 0) == 0   # one split: no fused attention
    Hq, Hkv, D, B, C, splits, K = 32, 8, 128, 1, 1536, 16, 2560
    N = (Hq + 2 * Hkv) * D
    x = torch.zeros(B, K, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(N, K, dtype=torch.bfloat16, device=DEV)
    gain = torch.ones(K, dtype=torch.bfloat16, device=DEV)
    cos, sin = oc.rope_tables(5e6, D, C + 1)
    cos, sin = dv(cos), dv(sin)
    posd = dv(torch.tensor([5]))
    ck = torch.zeros(B, Hkv, C, D, dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    xbuf = torch.zeros(call("q3_attn_xbuf_words", B, Hq, splits), dtype=torch.int32, device=DEV)
    qx = torch.zeros(B * N, dtype=torch.int32, device=DEV)
    out = torch.full((B, Hq * D), 7.0, dtype=torch.bfloat16, device=DEV)
    for layer, xm in ((64, _lib.X_NORM), (-1, _lib.X_NORM), (3, _lib.X_PLAIN)):
        with pytest.raises(RuntimeError):
            call("q3_qkv_attn", xm, P(x), K, None, P(gain), 1e-6, None, P(w), K, P(qx), P(gain), P(gain), P(cos),
                 P(sin), P(posd), P(ck), P(cv), P(xbuf), P(out), None, None, None, 0, 0, B, Hq, Hkv, C, splits,
                 layer, D ** -0.5, None, S())
    # The o projection without its exchange words or residual; the L2 hint
    # without the o projection, or with a row group that does not divide.
    with pytest.raises(RuntimeError):
        call("q3_qkv_attn", _lib.X_NORM, P(x), K, None, P(gain), 1e-6, None, P(w), K, P(qx), P(gain), P(gain),
             P(cos), P(sin), P(posd), P(ck), P(cv), P(xbuf), None, P(w), None, None, 0, 0, B, Hq, Hkv, C, splits,
             3, D ** -0.5, None, S())
    with pytest.raises(RuntimeError):
        call("q3_qkv_attn", _lib.X_NORM, P(x), K, None, P(gain), 1e-6, None, P(w), K, P(qx), P(gain), P(gain),
             P(cos), P(sin), P(posd), P(ck), P(cv), P(xbuf), P(out), None, None, P(w), N, 16, B, Hq, Hkv, C,
             splits, 3, D ** -0.5, None, S())
    ox = torch.zeros(Hq * D, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError):
        call("q3_qkv_attn", _lib.X_NORM, P(x), K, None, P(gain), 1e-6, P(x), P(w), K, P(qx), P(gain), P(gain),
             P(cos), P(sin), P(posd), P(ck), P(cv), P(xbuf), None, P(w), P(ox), P(w), N, 7, B, Hq, Hkv, C,
             splits, 3, D ** -0.5, None, S())
    torch.cuda.synchronize()
    assert bool((out.float() == 7.0).all()) and int(ck.abs().sum()) == 0 and int(qx.abs().sum()) == 0


@pytest.mark.parametrize("B,C,pos,qsplits", [(1, 300, 200, 1), (5, 700, 650, 3), (16, 1000, 999, 6),
                                              # configs 5 and 4: qkv from the skinny projection's partials
                                              (8, 16512, 16500, 5), (64, 2176, 2100, 5)])
def test_attn_decode_qkv_partials(B, C, pos, qsplits):
    """q/k/v from FP32 split partials == from their in-order sum rounded to BF16, bit for bit."""
    Hq, Hkv, D = 32, 8, 128
    width = (Hq + 2 * Hkv) * D
    part = (torch.randn(qsplits, B, width, generator=torch.Generator().manual_seed(pos)) * 0.7).float()
    acc = part[0].clone()
    for sp in range(1, qsplits):
        acc += part[sp]
    qkv = acc.to(torch.bfloat16)
    qw = (1 + rnd((D,), 0.2, 2).float()).to(torch.bfloat16)
    kw = (1 + rnd((D,), 0.2, 3).float()).to(torch.bfloat16)
    cos, sin = oc.rope_tables(5e6, D, max(4096, C + 1))
    ck, cv = rnd((B, Hkv, C, D), 1.0, 4), rnd((B, Hkv, C, D), 1.0, 5)
    splits = call("q3_attn_splits", B, Hkv, C)
    outs, caches = [], []
    for use_part in (False, True):
        ckd, cvd = dv(ck), dv(cv)
        pacc = torch.empty(B, Hq, splits, D, dtype=torch.float32, device=DEV)
        pml = torch.empty(B, Hq, splits, 2, dtype=torch.float32, device=DEV)
        out = torch.empty(B, Hq * D, dtype=torch.bfloat16, device=DEV)
        src = (None, width, P(dv(part)), qsplits) if use_part else (P(dv(qkv)), width, None, 0)
        call("q3_attn_decode", *src, P(dv(qw)), P(dv(kw)), P(dv(cos)), P(dv(sin)),
             P(dv(torch.tensor([pos]))), P(ckd), P(cvd), P(pacc), P(pml), None, B, Hq, Hkv, C, splits, 1e-6,
             D ** -0.5, S())
        call("q3_attn_merge", P(pacc), P(pml), P(out), B, Hq, splits, S())
        torch.cuda.synchronize()
        outs.append(out.cpu())
        caches.append((ckd.cpu(), cvd.cpu()))
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])
