"""The engine at the benchmark workloads, on the full seeded Qwen3-4B.

One engine (8 GB of weights) serves every test here; each workload rebuilds
its caches and graph at its own (batch, capacity).

The bar, with its numbers measured rather than chosen:
  * TOL_FULL = 0.25 (8 BF16 ulps at the logits' scale, top logits 4-6):
    per-step logit max-abs against HF / the CPU oracle.  A legal reordering
    of HF's own arithmetic -- the CPU oracle (bit-identical to HF at config 1)
    with its projections summed by torch's FP32 GEMM -- already moves logits
    by 0.14-0.17 at config 1 (tests/test_oracle.py::test_reorder_floor_config1)
    and by 0.174 over 512 teacher-forced steps at config 2 (on the fixture's
    512-id subset), flipping the argmax at 46 of those steps at HF gaps up to
    0.156.  The north star's "max-abs <= 5e-2" is below that floor for any
    BF16 forward that sums in another order than HF's CPU path.
  * the first step's logits over the whole vocabulary (151,936 values, an
    extreme-value statistic of that noise): max-abs and mean-abs within
    FLOOR_FACTOR of the same reordering's at that step
    (tests/golden/reorder_floor.json, written by make_reorder_floor.py: 0.156
    and 0.027-0.030 at configs 1 and 2).  Measured at config 2: the engine at
    0.253 / 0.035 with the prompt pass's split-K residual projections, 0.213 /
    0.037 without them -- the split sums sit closer to HF on average (a third
    fewer logits off by more than 0.125), and one logit's excursion decides
    the max.
  * FLOOR_FACTOR = 2: at configs 3-5 (no HF fixtures: the oracle from a
    pre-filled cache) the test measures that floor beside the engine, on the
    same cache and stream, and bounds the engine's max-abs and mean-abs by
    twice the floor's.  Measured: the engine sits at 1.3-1.45x the floor
    (mean 0.040-0.043 against 0.028-0.030), about sqrt(2): the linears'
    reordering plus one more source of the same size, attention rounding P to
    BF16 before P.V as the reference's GQA kernel does (fused.py:699-701).
    Indexing or reduction bugs move logits by whole units, 10-30x the floor.
  * NEAR_TIE = 0.0625: where a free-running stream first leaves the
    reference's, the reference's top-2 gap there must be at most this, two
    BF16 ulps at the logit scale (ulp 0.03125).  The north star asks for
    "the first near-tie (gap < 1e-2)"; below one ulp that is only an exact
    tie, and HF's config-2 stream has 26 exact ties and 61 one-ulp gaps in
    512 steps (the FP32-GEMM reorder leaves it at step 0, gap 0.031).
  * teacher-forced, a token may differ from the reference's argmax only where
    the reference's gap is within 2 * TOL_FULL (what the logit bound implies).
"""

import numpy as np
import pytest
import torch

from oracle import qwen3_cpu as oc
from oracle.compare import check_stream, replay_judge
from starter_amd import engine as engine_mod
from starter_amd.checkpoint import load_checkpoint
from starter_amd.workloads import WORKLOADS

pytestmark = pytest.mark.gpu

TOL_FULL = 0.25
NEAR_TIE = 0.0625
FLOOR_FACTOR = 2.0
PREFILLED_STEPS = 4


def golden(name):
    from conftest import GOLDEN
    return np.load(GOLDEN / f"{name}.npz")


def _reorder_floor():
    import json

    from conftest import GOLDEN
    return json.loads((GOLDEN / "reorder_floor.json").read_text())


REORDER_FLOOR = _reorder_floor()


@pytest.fixture(scope="module")
def full_engine(full_ckpt):
    eng = engine_mod.Engine(str(full_ckpt))
    yield eng
    eng.graph_key_reset()


@pytest.fixture(scope="module")
def oracle_4b(full_ckpt):
    cfg, tensors = load_checkpoint(full_ckpt)
    return oc.Qwen3Oracle(cfg, tensors, torch.bfloat16)


def hf_logit(g, i, tok):
    """HF's logit of ``tok`` at step i, from the fixture's top-16 (-inf if not there)."""
    hit = np.nonzero(g["top_ids"][i] == tok)[0]
    return g["top_logits"][i][hit[0]] if len(hit) else -np.inf


def first_divergence(got, want):
    return next((i for i in range(len(want)) if got[i] != want[i]), len(want))


def check_against_hf(eng, name, n):
    """Free-running stream, production-graph replay of HF's stream, and stored
    logits of the teacher-forced stream, each against the HF fixture."""
    g = golden(name)
    ids = g["ids"].tolist()
    want = g["tokens"].tolist()[:n]
    got = [s[0] for s in eng.generate(ids, n)]
    d = first_divergence(got, want)
    gap = None
    if d < n:
        gap = g["top_logits"][d][0] - hf_logit(g, d, got[d])
        assert gap <= NEAR_TIE, (f"{name}: free-running stream leaves HF's at step {d} where HF's gap is "
                                 f"{gap:.4f} (> {NEAR_TIE}): chose {got[d]}, HF {want[d]}")
    # HF's stream replayed through the production decode graph (feed table):
    # the max logit and HF's token's logit at every step.
    r = eng.replay(ids, [[t] for t in want])
    hf_top = g["top_logits"][:n, 0]
    top_err = np.abs(r["top"][:, 0] - hf_top).max()
    tok_err = np.abs(r["logit"][:, 0] - hf_top).max()  # HF's token is HF's argmax
    short = r["top"][:, 0] - r["logit"][:, 0]
    assert top_err <= TOL_FULL and tok_err <= TOL_FULL, (top_err, tok_err)
    flips = [i for i in range(n) if r["argmax"][i, 0] != want[i]]
    for i in flips:  # a flip only where HF's own gap is within what the logit bound allows
        assert g["top_logits"][i][0] - hf_logit(g, i, r["argmax"][i, 0]) <= 2 * TOL_FULL, i
    # Full logits (stored-logits variant of the same step) over HF's subset.
    steps, logits = eng.trace_logits(ids, n, forced=[[t] for t in want])
    lg = logits[:, 0].float().numpy()
    sub = np.abs(lg[:, g["subset"]] - g["subset_logits"][:n]).max(axis=1)
    first = np.abs(lg[0] - g["logits_first"]).max()
    first_mean = np.abs(lg[0] - g["logits_first"]).mean()
    last = np.abs(lg[-1] - g["logits_last"]).max() if n == len(g["tokens"]) else 0.0
    assert [s[0] for s in steps] == r["argmax"][:, 0].tolist()  # the two graphs choose alike
    print(f"{name}: free-running equal to HF through step {d - 1} of {n} (gap there {gap}); "
          f"teacher-forced: logit max-abs first {first:.3f} (mean {first_mean:.4f}) last {last:.3f} "
          f"subset {sub.max():.3f}, "
          f"replay top {top_err:.3f} token {tok_err:.3f}; argmax flips at {len(flips)} steps, "
          f"worst shortfall {short.max():.4f}", flush=True)
    floor = REORDER_FLOOR[name]
    assert first <= FLOOR_FACTOR * floor["first_max_abs"], (first, floor)
    assert first_mean <= FLOOR_FACTOR * floor["first_mean_abs"], (first_mean, floor)
    assert last <= TOL_FULL and sub.max() <= TOL_FULL
    return got


def test_full_checkpoint_matches_manifest(full_ckpt):
    """Every tensor of the GPU box's seeded checkpoint hashes to the committed manifest."""
    import json

    from conftest import GOLDEN
    from starter_amd.checkpoint import manifest_of

    want = json.loads((GOLDEN / "qwen3_4b_seed0_manifest.json").read_text())["sha256"]
    _, tensors = load_checkpoint(full_ckpt)
    assert manifest_of(tensors, threads=16) == want


def test_config1_matches_hf(full_engine):
    """B=1, P=32, 32 greedy tokens."""
    check_against_hf(full_engine, "config1_bf16", 32)


def test_config2_matches_hf(full_engine):
    """B=1, P=1024, 512 greedy tokens (the headline workload)."""
    check_against_hf(full_engine, "config2_bf16", 512)


def test_replay_judge_config1(full_engine, oracle_4b):
    """The contest's quality rule on the engine's config-1 stream, both ways:
    replayed through the engine's own production graph (every token is the
    replay's argmax: the captured step is deterministic) and through the CPU
    oracle, i.e. native Qwen (every token the argmax or a near-tie)."""
    g = golden("config1_bf16")
    ids = g["ids"].tolist()
    emitted = list(full_engine.generate(ids, 32))
    r = full_engine.replay(ids, emitted)
    assert r["argmax"][:, 0].tolist() == [e[0] for e in emitted]
    assert np.array_equal(r["top"], r["logit"])
    assert full_engine.replay_check(ids, emitted) == []
    j = replay_judge(oracle_4b, ids, emitted, margin=engine_mod.TIE_MARGIN_LOGITS)
    print(f"config1 judged by the CPU oracle: shortfalls {np.round(j['shortfall'][:, 0], 4).tolist()}", flush=True)
    assert j["failures"] == []
    assert j["shortfall"].max() <= 2 * TOL_FULL


def teacher_forced(orc, first, P, steps, forced=None):
    """``steps`` decode steps of ``orc`` from its cache, the first fed ``first``
    at P, step k >= 1 fed ``forced[k - 1]`` (its own choice when None).
    Returns (choices [steps][B], logits [steps, B, V] FP32)."""
    B = len(first)
    tok = torch.tensor(first, dtype=torch.int64).view(B, 1)
    choices, logits = [], []
    for k in range(steps):
        lg = orc.forward(tok, P + k)
        logits.append(lg.float())
        choices.append(oc.argmax_first(lg).tolist())
        nxt = forced[k] if forced is not None and k < len(forced) else choices[-1]
        tok = torch.tensor(nxt, dtype=torch.int64).view(B, 1)
    return choices, torch.stack(logits)


@pytest.mark.parametrize("config", [3, 4, 5])
def test_prefilled_cache_decode_matches_oracle(full_engine, oracle_4b, config):
    """BASELINE configs 3-5 at their real (batch, capacity): the KV cache's
    prompt positions filled with seeded N(0, 1) values on the device, copied
    to the CPU oracle; then decode steps from the same first tokens, the
    engine teacher-forced on the oracle's stream (the prompt pass itself is
    covered by the prefill tests; a decode step's arithmetic does not depend
    on how the cache was filled).

    Beside the engine, the same steps through the oracle with FP32-GEMM
    projections (a legal reordering of the oracle's own arithmetic) show the
    noise floor at this workload; both are printed, and the engine must stay
    within FLOOR_FACTOR of it (max-abs and mean-abs), with argmax flips only
    at gaps within 2 * TOL_FULL."""
    wl = WORKLOADS[config]
    B, P, N = wl.batch, wl.prompt, wl.new_tokens
    eng, orc = full_engine, oracle_4b
    first = np.random.Generator(np.random.PCG64(70 + config)).integers(0, 151643, B).tolist()
    orc.reset(B, P + N)
    eng.prepare_trace(B, P, N)
    try:
        assert eng.skinny == (B > engine_mod.GEMV_BATCH_MAX)
        gen = torch.Generator(device=eng.device).manual_seed(1000 + config)
        for layer in range(eng.LAYERS):
            for cache, host in ((eng.cache_k, orc.cache_k), (eng.cache_v, orc.cache_v)):
                seg = cache[layer, :, :, :P]
                seg.normal_(generator=gen)
                host[layer][:, :, :P].copy_(seg.cpu())
        torch.cuda.synchronize()
        want, want_logits = teacher_forced(orc, first, P, PREFILLED_STEPS)
        got, got_logits = eng.trace_decode(first, P, PREFILLED_STEPS, forced=want)
    finally:
        eng.end_trace()
    orc.linear = oc.f32_linear()
    try:
        _, floor_logits = teacher_forced(orc, first, P, PREFILLED_STEPS, forced=want)
    finally:
        orc.linear = oc.linear
        orc.cache_k = orc.cache_v = None  # 20 GB at config 4
    err = (got_logits.float() - want_logits).abs()
    floor = (floor_logits - want_logits).abs()
    top = want_logits.max(dim=-1).values
    flips = [(k, b) for k in range(PREFILLED_STEPS) for b in range(B) if got[k][b] != want[k][b]]
    shorts = [float(top[k, b] - want_logits[k, b, got[k][b]]) for k, b in flips]
    print(f"config{config} from a pre-filled cache (B={B}, context {P}..{P + PREFILLED_STEPS}, top logits "
          f"{top.min():.2f}..{top.max():.2f}): engine logit max-abs {err.max():.3f} mean {err.mean():.4f}; "
          f"FP32-GEMM reorder floor max-abs {floor.max():.3f} mean {floor.mean():.4f}; engine argmax flips "
          f"{len(flips)} of {B * PREFILLED_STEPS}, worst shortfall {max(shorts, default=0.0):.4f}", flush=True)
    assert err.max() <= FLOOR_FACTOR * floor.max() and err.mean() <= FLOOR_FACTOR * floor.mean()
    assert max(shorts, default=0.0) <= 2 * TOL_FULL
