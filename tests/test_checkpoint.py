"""Seeded checkpoint writer / safetensors reader."""

import json
import pathlib

import numpy as np

from make_golden import TINY
from starter_amd import checkpoint as ck

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def test_roundtrip_and_layout(tmp_path):
    manifest = ck.write_seeded_checkpoint(tmp_path, TINY, seed=3, std=0.05, gain_std=0.1)
    cfg, tensors = ck.load_checkpoint(tmp_path)
    assert cfg == TINY
    specs = ck.tensor_specs(TINY)
    assert set(tensors) == {n for n, _, _ in specs}
    assert "lm_head.weight" not in tensors  # tied
    for name, shape, kind in specs:
        t = tensors[name]
        assert t.shape == shape and t.dtype == np.uint16
        assert np.array_equal(t, ck.seeded_tensor(name, shape, kind, 3, 0.05, 0.1))
    assert ck.manifest_of(tensors) == manifest


def test_seeded_values_are_normal():
    t = ck.seeded_tensor("x", (1 << 20,), "normal", 0, 0.02)
    f = (t.astype(np.uint32) << 16).view(np.float32)
    assert abs(f.mean()) < 1e-4 and abs(f.std() - 0.02) < 1e-4
    ones = ck.seeded_tensor("model.norm.weight", (2560,), "ones")
    assert np.all(ones == ck.BF16_ONE)


def test_stream_depends_on_name_and_seed_only():
    a = ck.seeded_tensor("model.layers.0.mlp.up_proj.weight", (64, 64), "normal", 0)
    b = ck.seeded_tensor("model.layers.0.mlp.up_proj.weight", (64, 64), "normal", 0)
    c = ck.seeded_tensor("model.layers.0.mlp.up_proj.weight", (64, 64), "normal", 1)
    d = ck.seeded_tensor("model.layers.1.mlp.up_proj.weight", (64, 64), "normal", 0)
    assert np.array_equal(a, b) and not np.array_equal(a, c) and not np.array_equal(a, d)
    # A prefix of a longer draw is the shorter draw (element i depends only on i).
    e = ck.seeded_tensor("model.layers.0.mlp.up_proj.weight", (64 * 64 + 3,), "normal", 0)
    assert np.array_equal(a.reshape(-1), e[:64 * 64])


def test_committed_manifest_pins_the_generator():
    """The full model's per-tensor SHA-256 (committed) for a few small tensors."""
    manifest = json.loads((GOLDEN / "qwen3_4b_seed0_manifest.json").read_text())["sha256"]
    specs = {n: (s, k) for n, s, k in ck.tensor_specs(ck.QWEN3_4B)}
    import hashlib
    for name in ("model.layers.0.self_attn.k_proj.weight", "model.layers.35.self_attn.v_proj.weight",
                 "model.norm.weight", "model.layers.7.self_attn.q_norm.weight"):
        shape, kind = specs[name]
        t = ck.seeded_tensor(name, shape, kind, 0)
        assert hashlib.sha256(t.data).hexdigest() == manifest[name], name


def test_prompts():
    p = ck.seeded_prompt(1, 2, 32)
    assert len(p) == 2 and all(len(r) == 32 for r in p)
    assert all(0 <= x < 151643 for r in p for x in r)
    assert p[0] != p[1]
    assert ck.seeded_prompt(1, 2, 32) == p
