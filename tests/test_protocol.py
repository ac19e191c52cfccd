"""The streaming protocol and gates (starter_amd/protocol.py) on the CPU, with a
scripted engine in the child process: timing arithmetic, stream-shape checks
and the gate limits of reference QWEN_ENGINE_CONTRACT.md "Gates and failure"."""

import pathlib
import sys

import pytest

from starter_amd import protocol

ROOT = pathlib.Path(__file__).resolve().parents[1]

#: A child that speaks the protocol: first step after `first` seconds, then one
#: every `every` seconds; `steps_off` emits that many extra (or fewer) steps.
FAKE = """
import sys, time
sys.path.insert(0, {root!r})
from starter_amd.protocol import serve

class Fake:
    VOCAB = 100
    def generate(self, ids, new):
        time.sleep({first})
        for k in range(new + {steps_off}):
            if k:
                time.sleep({every})
            yield [(r + k) % 100 for r in range(len(ids))]

serve(Fake(), [[1, 2]], 2)
"""


def fake_cmd(first=0.05, every=0.01, steps_off=0):
    return [sys.executable, "-c", FAKE.format(root=str(ROOT), first=first, every=every, steps_off=steps_off)]


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
