"""The streaming protocol and gates (starter_amd/protocol.py) on the CPU, with a
scripted engine in the child process: timing arithmetic, stream-shape checks
and the gate limits of reference QWEN_ENGINE_CONTRACT.md "Gates and failure"."""

import pathlib
import sys

import pytest

from starter_amd import protocol

ROOT = pathlib.Path(__file__).resolve().parents[1]

#: A child that speaks the protocol: first step after `first` seconds, then one
#: every `every` seconds; `steps_off` emits that many extra (or fewer) steps;
#: `load` seconds pass before the warmup, and the step numbered `stall` (when
#: >= 0) waits 60 s first (a hung engine).
FAKE = """
import sys, time
sys.path.insert(0, {root!r})
from starter_amd.protocol import serve

class Fake:
    VOCAB = 100
    calls = 0
    def generate(self, ids, new):
        Fake.calls += 1
        time.sleep({first})
        for k in range(new + {steps_off}):
            if k:
                time.sleep({every})
            if Fake.calls > 1 and k == {stall}:
                time.sleep(60)
            yield [(r + k) % 100 for r in range(len(ids))]

time.sleep({load})
serve(Fake(), [[1, 2]], 2)
"""


def fake_cmd(first=0.05, every=0.01, steps_off=0, load=0.0, stall=-1):
    return [sys.executable, "-c", FAKE.format(root=str(ROOT), first=first, every=every, steps_off=steps_off,
                                              load=load, stall=stall)]


def test_client_times_the_stream():
    prompts = [[[1, 2, 3], [4, 5, 6]]] * 3
    run = protocol.run_workload(fake_cmd(first=0.05, every=0.01), prompts, 6)
    assert len(run.samples) == 3
    for s in run.samples:
        assert s.steps == [[k % 100, (1 + k) % 100] for k in range(6)]
        assert 0.05 <= s.ttft < 0.5
        assert 0.01 <= s.tpot < 0.1
        assert s.total == s.arrivals[-1] and abs(s.tpot * 5 - (s.total - s.ttft)) < 1e-9
    summ = run.summary()
    assert summ["tokens_per_s"] == pytest.approx(2 * 6 / summ["total_s_median"])
    assert summ["spread"] >= 0 and summ["peak_bytes"] == 0  # no GPU in the child


def test_wrong_step_count_is_an_error():
    with pytest.raises(protocol.ProtocolError, match="wrong stream shape"):
        protocol.run_workload(fake_cmd(steps_off=-1), [[[1, 2]]], 4)


@pytest.mark.parametrize("load,stall", [(60.0, -1), (0.0, 2)], ids=["load", "mid_sample"])
def test_silent_child_is_killed_at_its_budget(load, stall):
    """A child that stops writing (during load, or in the middle of a sample's
    stream) does not block the client: the read waits only until the budget,
    the run raises, and the child is killed."""
    import time

    t0 = time.perf_counter()
    with pytest.raises(protocol.ProtocolError, match="time budget"):
        protocol.run_workload(fake_cmd(load=load, stall=stall), [[[1, 2]]], 4,
                              load_budget_s=2.0, sample_budget_s=1.0)
    assert time.perf_counter() - t0 < 20


def test_native_attention_matches_oracle_attention():
    """The GPU native's attention (two batched products per KV head, scores as
    K . Q^T) against the oracle's SDPA, in float32 on the CPU: decode, a whole
    causal prompt, and a later chunk over a cached prefix."""
    import torch

    from oracle import qwen3_cpu as oc
    from oracle.native_server import attention_bmm

    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, D, C = 2, 8, 2, 16, 40
    for T, start in ((1, 17), (9, 0), (6, 11)):
        q = torch.randn(B, Hq, T, D, generator=g)
        ck = torch.randn(B, Hkv, C, D, generator=g)
        cv = torch.randn(B, Hkv, C, D, generator=g)
        k, v = ck[:, :, :start + T], cv[:, :, :start + T]
        want = oc.attention(q, k, v, D ** -0.5, start)
        got = attention_bmm(q, k, v, D ** -0.5, start)
        assert torch.allclose(got, want, atol=1e-5, rtol=1e-5), (T, start)


def test_gates():
    native = {"ttft_s_median": 1.0, "tpot_s_median": 0.1, "spread": 0.0, "peak_bytes": 0, "device_bytes": 0,
              "load_s": 0.0, "warmup_s": 0.0}
    ok = {"ttft_s_median": 1.1, "tpot_s_median": 0.05, "spread": 0.25, "peak_bytes": 90, "device_bytes": 100,
          "load_s": 100.0, "warmup_s": 200.0}
    g = protocol.gates(ok, native)
    assert g["passed"] and g["ttft"]["value"] == pytest.approx(1.1)
    for key, bad in (("ttft_s_median", 1.2), ("tpot_s_median", 0.12), ("spread", 0.3), ("peak_bytes", 91),
                     ("load_s", 101.0)):
        g = protocol.gates({**ok, key: bad}, native)
        assert not g["passed"], key
    assert not protocol.gates(ok, native, failing_tokens=1)["passed"]


def test_prompt_lookup_drafts_miss_on_the_seeded_streams():
    """Why exact-verification speculative decoding is not built: on the seeded
    random-init workloads a prompt-lookup draft (the next k tokens after the
    latest earlier match of the last n tokens of prompt + output) is never the
    greedy continuation, so every verification pass would be pure cost.
    Measured on the HF greedy streams of configs 1 and 2 (committed fixtures)."""
    import numpy as np
    golden = pathlib.Path(__file__).resolve().parent / "golden"
    for name in ("config1_bf16", "config2_bf16"):
        d = np.load(golden / f"{name}.npz")
        ctx, out = d["ids"][0].tolist(), d["tokens"].tolist()
        for n in (1, 2, 3):
            accepted, i, c = 0, 0, list(ctx)
            while i < len(out):
                key = c[-n:]
                draft = next((c[j + n:j + n + 4] for j in range(len(c) - n - 1, -1, -1) if c[j:j + n] == key), [])
                a = 0
                while a < len(draft) and i + a < len(out) and draft[a] == out[i + a]:
                    a += 1
                accepted += a
                c += out[i:i + a + 1]
                i += a + 1
            assert accepted == 0, (name, n, accepted)
