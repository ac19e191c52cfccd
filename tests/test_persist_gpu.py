"""The one-kernel decode step of one sequence (``q3_decode_persistent``).

At batch 1 the engine runs each decode step as a single persistent kernel
(one workgroup per CU, cross-workgroup exchange through flagged words) instead
of one kernel per op.  Its projections, norms, SwiGLU, residual joins and
argmax use the same arithmetic in the same order as the kernel-per-op step;
only the attention's summation order differs (split-K partials, per-lane
online softmax).  So against the kernel-per-op engine the logits agree to the
attention reordering (measured here), and against the CPU oracle / HF fixtures
the same parity rule as every other engine test applies.
"""

import numpy as np
import pytest
import torch

from oracle import qwen3_cpu as oc
from oracle.compare import check_stream
from starter_amd import engine as engine_mod
from starter_amd.checkpoint import load_checkpoint

pytestmark = pytest.mark.gpu

TOL_TILE = 0.06


@pytest.fixture(scope="module")
def tile_engine(tile_ckpt):
    return engine_mod.Engine(str(tile_ckpt))


def _trace(engine, ids, n, persistent):
    saved = engine_mod.PERSISTENT_DECODE
    engine_mod.PERSISTENT_DECODE = persistent
    try:
        steps, logits = engine.trace_logits(ids, n)
        assert engine.persist == persistent
    finally:
        engine_mod.PERSISTENT_DECODE = saved
    return steps, logits


@pytest.mark.parametrize("prompt", [1, 7, 40])
def test_persistent_step_matches_oracle(tile_engine, tile_ckpt, prompt):
    cfg, tensors = load_checkpoint(tile_ckpt)
    orc = oc.Qwen3Oracle(cfg, tensors, torch.bfloat16)
    rng = np.random.Generator(np.random.PCG64(500 + prompt))
    ids = rng.integers(0, cfg.vocab_size, (1, prompt)).tolist()
    want, want_logits = orc.generate(ids, 12, keep_logits=True)
    steps, logits = _trace(tile_engine, ids, 12, True)
    firsts = check_stream(steps, logits.float().numpy(), want, torch.stack(want_logits).float().numpy(), TOL_TILE)
    print(f"prompt {prompt}: first divergence {firsts} of 12")


def test_persistent_step_matches_kernel_per_op(tile_engine):
    """Same prompt through both decode steps: the logits differ only by the
    attention's reordering (measured bound below), tokens agree."""
    rng = np.random.Generator(np.random.PCG64(77))
    ids = rng.integers(0, 1024, (1, 33)).tolist()
    a_steps, a_logits = _trace(tile_engine, ids, 16, True)
    b_steps, b_logits = _trace(tile_engine, ids, 16, False)
    diff = (a_logits.float() - b_logits.float()).abs()
    print(f"persistent vs kernel-per-op: max |dlogit| {diff.max():.4f}, mean {diff.mean():.5f}; "
          f"tokens equal {sum(x == y for x, y in zip(a_steps, b_steps))}/16")
    # Prefill (step 0) is shared, so step 0 is identical; later steps move by the
    # attention reordering only (a few BF16 ulps of logits on this model).
    assert torch.equal(a_logits[0], b_logits[0])
    assert diff.max() <= 0.06
    d = next((i for i in range(16) if a_steps[i] != b_steps[i]), 16)
    if d < 16:
        lg = b_logits[d, 0].float()
        assert lg.max() - lg[a_steps[d][0]] <= 0.12  # a near-tie of the other path


@pytest.fixture
def persistent_on():
    saved = engine_mod.PERSISTENT_DECODE
    engine_mod.PERSISTENT_DECODE = True
    yield
    engine_mod.PERSISTENT_DECODE = saved


def test_persistent_generate_resets_between_calls(tile_engine, persistent_on):
    """Positions restart at each call and the step epoch carries on: a second
    call, and a call after a different shape, stream what a fresh trace does."""
    rng = np.random.Generator(np.random.PCG64(3))
    first = rng.integers(0, 1024, (1, 9)).tolist()
    second = rng.integers(0, 1024, (1, 9)).tolist()
    want_second, _ = _trace(tile_engine, second, 8, True)
    list(tile_engine.generate(first, 8))
    assert list(tile_engine.generate(second, 8)) == want_second
    list(tile_engine.generate(rng.integers(0, 1024, (2, 5)).tolist(), 4))  # another shape in between
    assert list(tile_engine.generate(second, 8)) == want_second
    assert tile_engine.persist


def test_persistent_long_run_is_deterministic(tile_engine, persistent_on):
    """Many replays of the captured step (the epoch advances every step): two
    identical calls give identical streams."""
    ids = [[5, 6, 7, 8, 9, 10, 11]]
    a = list(tile_engine.generate(ids, 60))
    b = list(tile_engine.generate(ids, 60))
    assert a == b and len(a) == 60
