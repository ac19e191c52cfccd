"""The bench's reported figures (CPU only): prefill flop and decode step bytes
against counts taken from the checkpoint's own tensor shapes."""

import math

import bench
from starter_amd.checkpoint import tensor_specs
from starter_amd.workloads import MODEL


def _projection_weights():
    """Matrix weights of the 36 layers (q, k, v, o, gate, up, down) and the tied embedding."""
    layers = sum(math.prod(shape) for name, shape, kind in tensor_specs(MODEL)
                 if name.startswith("model.layers.") and kind == "normal")
    embed = math.prod(dict((n, s) for n, s, _ in tensor_specs(MODEL))["model.embed_tokens.weight"])
    return layers, embed


def test_prefill_flop_count():
    layers, embed = _projection_weights()
    assert layers == 36 * 100_925_440 and embed == 388_956_160  # BASELINE's 8,044,544,000 B of weights
    for B, P in [(1, 1), (1, 1024), (8, 16384)]:
        got = bench.prefill_figures(B, P, 1.0)["flop"]
        D, Hq = MODEL.head_dim, MODEL.num_attention_heads
        pairs = P * (P + 1) // 2                      # causal (query, key <= query) pairs
        want = 2 * B * P * layers + 2 * B * embed + 4 * D * B * Hq * MODEL.num_hidden_layers * pairs
        assert got == want, (B, P)
    f = bench.prefill_figures(1, 1024, 10.0)
    assert math.isclose(f["achieved"], f["flop"] / 1e-2 / 1e12, rel_tol=1e-3)
    assert math.isclose(f["frac"], f["achieved"] / 2500.0, rel_tol=1e-3)
    assert f["tokens_per_s"] == 102400.0


def test_weight_bytes_per_step_matches_checkpoint():
    layers, embed = _projection_weights()
    norms = sum(math.prod(s) for n, s, k in tensor_specs(MODEL) if k == "ones")
    assert 2 * (layers + embed) == 8_044_544_000
    assert 2 * (layers + embed + norms) == 8_044_936_192  # BASELINE.json's per-step weight bytes
    assert bench.KV_BYTES_PER_TOKEN == 147_456
