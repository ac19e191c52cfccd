"""Host-side logic of ``Engine`` that needs no GPU: the step check and the
replay judge's rule, on an engine object built without ``__init__`` (which
would load weights onto a device)."""

import numpy as np
import pytest
import torch

from starter_amd import engine as engine_mod


def bare_engine(**attrs):
    eng = engine_mod.Engine.__new__(engine_mod.Engine)
    eng.graph = None
    eng.batch = eng.capacity = 0
    eng.VOCAB = 100
    for k, v in attrs.items():
        setattr(eng, k, v)
    return eng


def test_check_step_raises_on_a_fused_attention_timeout():
    eng = bare_engine(attn_fused=True, attn_err=torch.tensor([1], dtype=torch.int32))
    eng.batch, eng.capacity = 4, 100
    with pytest.raises(RuntimeError, match="did not complete"):
        eng._check_step()
    assert eng.batch == 0 and eng.capacity == 0  # the next call rebuilds the step


def test_check_step_passes_clean_steps():
    bare_engine(attn_fused=True, attn_err=torch.tensor([0], dtype=torch.int32))._check_step()
    # A stale error word is not consulted when the fused launch is not part of the step.
    bare_engine(attn_fused=False, attn_err=torch.tensor([1], dtype=torch.int32))._check_step()


def test_replay_check_applies_the_tie_margin():
    """Emitted tokens pass when they are the replay's argmax or within the margin
    of its maximum (reference QWEN_ENGINE_CONTRACT.md "The quality rule")."""
    rec = {"argmax": np.array([[5, 6], [7, 8], [9, 9]]),
           "top": np.array([[4.0, 4.0], [4.0, 4.0], [4.0, 4.0]]),
           "logit": np.array([[4.0, 4.0], [3.0, 1.5], [4.0, 2.0]])}
    eng = bare_engine()
    eng.replay = lambda ids, emitted: rec
    emitted = [[5, 6], [1, 2], [9, 3]]
    assert eng.replay_check([[0]] * 2, emitted) == [(1, 1, 2.5)]
    assert eng.replay_check([[0]] * 2, emitted, margin=0.5) == [(1, 0, 1.0), (1, 1, 2.5), (2, 1, 2.0)]


def test_stream_validation():
    eng = bare_engine()
    assert eng._stream_tensor([[1, 2], [3, 4]], 2, "x").shape == (2, 2)
    with pytest.raises(ValueError):
        eng._stream_tensor([[1, 2, 3]], 2, "x")
    with pytest.raises(ValueError):
        eng._stream_tensor([[1, 100]], 2, "x")


def test_no_fallback_without_the_library(monkeypatch, tmp_path):
    """The product path fails loudly when the HIP library is missing."""
    from starter_amd import _lib
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "missing.so")
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(ImportError, match="no non-HIP path"):
        _lib.lib()


def test_archive_root_engine_forwards_patched_globals():
    """The drop-in engine/engine.py is the engine module itself, so the reference
    harness's assignments (tests/test_equivalence.py:25-27,90-92) reach it."""
    import importlib
    import pathlib
    import sys

    root = pathlib.Path(__file__).resolve().parents[1]
    sys.path.insert(0, str(root / "engine"))
    try:
        sys.modules.pop("engine", None)
        mod = importlib.import_module("engine")
    finally:
        sys.path.remove(str(root / "engine"))
    assert mod is engine_mod and mod.Engine is engine_mod.Engine
    saved = engine_mod.PREFILL_CHUNK_TOKENS
    try:
        mod.PREFILL_CHUNK_TOKENS = 48
        assert engine_mod.PREFILL_CHUNK_TOKENS == 48
    finally:
        mod.PREFILL_CHUNK_TOKENS = saved


def test_engine_refuses_cpu_device_and_non_bf16_dtype(monkeypatch):
    """The reference's CPU test patches DEVICE = "cpu" and LOAD_DTYPE = float32;
    this engine has one (GPU, BF16) path and says so instead of running another."""
    monkeypatch.setattr(engine_mod, "LOAD_DTYPE", torch.float32)
    with pytest.raises(ValueError, match="BF16"):
        engine_mod.Engine("/nonexistent")
    monkeypatch.setattr(engine_mod, "LOAD_DTYPE", torch.bfloat16)
    monkeypatch.setattr(engine_mod, "DEVICE", "cpu")
    with pytest.raises(RuntimeError, match="no CPU path"):
        engine_mod.Engine("/nonexistent")
