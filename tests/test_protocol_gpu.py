"""The contest's streaming protocol end to end at BASELINE configs 1 and 3.

The engine in a child process (``python -m starter_amd.protocol``) and native
Qwen on the same GPU (``python -m oracle.native_server --gpu``: HF's op
sequence eagerly on ``cuda:0``) are timed by the same client through the same
pipe, with fresh prompts per sample; then the contest's gates (reference
QWEN_ENGINE_CONTRACT.md "Gates and failure", :94-96,125-133) -- TTFT and TPOT
within 1.10x native's medians, peak device memory within 90%, spread within
25%, load within 300 s -- and its quality rule, every emitted token replayed
teacher-forced through native Qwen (the CPU oracle, bit-identical to HF's CPU
path, at config 1; the GPU native at config 3, whose 16 x 256-token streams
the CPU would take minutes to replay)."""

import json
import pathlib
import sys

import pytest
import torch

from oracle.compare import replay_judge
from oracle.native_server import NativeGpu
from oracle.qwen3_cpu import Qwen3Oracle
from starter_amd import protocol
from starter_amd.checkpoint import load_checkpoint, seeded_prompt
from starter_amd.engine import TIE_MARGIN_LOGITS
from starter_amd.workloads import WORKLOADS

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _round(d):
    return {k: round(v, 5) if isinstance(v, float) else v for k, v in d.items()}


@pytest.mark.parametrize("config,samples", [(1, 5), (3, 3)])
def test_protocol_gates(full_ckpt, config, samples):
    wl = WORKLOADS[config]
    B, P, N = wl.batch, wl.prompt, wl.new_tokens
    prompts = [seeded_prompt(500 + 10 * config + s, B, P) for s in range(samples)]
    args = [str(full_ckpt), str(B), str(P), str(N)]
    # The children report device-wide used bytes: return what this process's
    # allocator cached from earlier tests first.
    torch.cuda.empty_cache()
    print(f"protocol at config {config}: engine", flush=True)
    engine = protocol.run_workload([sys.executable, "-m", "starter_amd.protocol", *args], prompts, N, cwd=ROOT)
    print(f"protocol at config {config}: native on the GPU", flush=True)
    native = protocol.run_workload([sys.executable, "-m", "oracle.native_server", *args, "--gpu"], prompts, N,
                                   cwd=ROOT)
    if config == 1:
        cfg, tensors = load_checkpoint(full_ckpt)
        judge = Qwen3Oracle(cfg, tensors, torch.bfloat16)
    else:
        judge = NativeGpu(str(full_ckpt))
    failing, worst = 0, 0.0
    for ids, sample in zip(prompts, engine.samples):
        j = replay_judge(judge, ids, sample.steps, margin=TIE_MARGIN_LOGITS)
        failing += len(j["failures"])
        worst = max(worst, float(j["shortfall"].max()))
    del judge
    cand, nat = engine.summary(), native.summary()
    g = protocol.gates(cand, nat, failing)
    print(f"protocol at config {config}: " + json.dumps({
        "engine": _round(cand), "native_gpu": _round(nat),
        "gates": {k: ({"value": round(v["value"], 4), "ok": v["ok"]} if isinstance(v, dict) else v)
                  for k, v in g.items()},
        "worst_replay_shortfall": worst}), flush=True)
    assert g["passed"], g
    assert engine.samples[0].steps != engine.samples[1].steps  # fresh prompts, fresh streams
    # native's own streams are a GPU reordering of the same model: a check that
    # the comparator computed Qwen3 and not something cheaper.
    agree = sum(a == b for e, n in zip(engine.samples, native.samples) for a, b in zip(e.steps[0], n.steps[0]))
    assert agree >= 0.7 * B * samples, agree
