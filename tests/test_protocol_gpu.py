"""The contest's streaming protocol end to end at BASELINE config 1 (B=1, P=32, 32 tokens):
the engine in a child process (``python -m starter_amd.protocol``) and native Qwen (the CPU
oracle, ``python -m oracle.native_server``) timed by the same client through the same pipe,
five samples each with fresh prompts; then the contest's gates (reference
QWEN_ENGINE_CONTRACT.md "Gates and failure") and its quality rule, every emitted token
replayed teacher-forced through native Qwen."""

import json
import pathlib
import sys

import pytest
import torch

from oracle.compare import replay_judge
from oracle.qwen3_cpu import Qwen3Oracle
from starter_amd import protocol
from starter_amd.checkpoint import load_checkpoint, seeded_prompt
from starter_amd.engine import TIE_MARGIN_LOGITS

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parents[1]
B, P, N, SAMPLES = 1, 32, 32, 5


def test_protocol_gates_at_config1(full_ckpt):
    prompts = [seeded_prompt(500 + s, B, P) for s in range(SAMPLES)]
    args = [str(full_ckpt), str(B), str(P), str(N)]
    engine = protocol.run_workload([sys.executable, "-m", "starter_amd.protocol", *args], prompts, N, cwd=ROOT)
    native = protocol.run_workload([sys.executable, "-m", "oracle.native_server", *args], prompts, N, cwd=ROOT)
    cfg, tensors = load_checkpoint(full_ckpt)
    judge = Qwen3Oracle(cfg, tensors, torch.bfloat16)
    failing, worst = 0, 0.0
    for ids, sample in zip(prompts, engine.samples):
        j = replay_judge(judge, ids, sample.steps, margin=TIE_MARGIN_LOGITS)
        failing += len(j["failures"])
        worst = max(worst, float(j["shortfall"].max()))
    cand, nat = engine.summary(), native.summary()
    g = protocol.gates(cand, nat, failing)
    print("protocol at config 1: " + json.dumps({
        "engine": {k: round(v, 5) if isinstance(v, float) else v for k, v in cand.items()},
        "native_cpu": {k: round(v, 5) if isinstance(v, float) else v for k, v in nat.items()},
        "gates": {k: ({"value": round(v["value"], 4), "ok": v["ok"]} if isinstance(v, dict) else v)
                  for k, v in g.items()},
        "worst_replay_shortfall": worst}), flush=True)
    assert g["passed"], g
    assert engine.samples[0].steps != engine.samples[1].steps  # fresh prompts, fresh streams
