"""Write tests/golden/reorder_floor.json: what reordering alone moves the
first step's logits by, over the whole vocabulary, at BASELINE configs 1 and 2.

The CPU oracle (``oracle/qwen3_cpu.py``, bit-identical to HF's CPU path on the
config-1 fixture) runs the fixture's prompt with every projection summed by
torch's FP32 GEMM instead (``oc.f32_linear``: the same BF16 products and one
rounding, another summation order), and its last-position logits are compared
with HF's (``logits_first`` of ``config{1,2}_bf16.npz``): the max-abs and the
mean-abs over the 151,936 logits.  tests/test_workloads_gpu.py bounds the
engine's first-step logits by FLOOR_FACTOR times these.

Run (in this container, about 4 minutes on 8 cores; the seeded checkpoint is
written first if missing):
    python tests/golden/make_reorder_floor.py
"""

from __future__ import annotations

import json
import os
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import qwen3_cpu as oc  # noqa: E402
from starter_amd.checkpoint import ensure_seeded_checkpoint, load_checkpoint  # noqa: E402
from starter_amd.workloads import MODEL, MODEL_SEED  # noqa: E402


def main() -> None:
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    base = pathlib.Path(os.environ.get("Q3_CKPT_DIR", "/tmp/q3_seeded_qwen3_4b"))
    cfg, tensors = load_checkpoint(ensure_seeded_checkpoint(base, MODEL, MODEL_SEED))
    orc = oc.Qwen3Oracle(cfg, tensors, torch.bfloat16)
    del tensors
    orc.linear = oc.f32_linear()
    out = {}
    for name in ("config1_bf16", "config2_bf16"):
        g = np.load(HERE / f"{name}.npz")
        ids = torch.from_numpy(g["ids"])
        orc.reset(ids.shape[0], ids.shape[1] + 1)
        lg = orc.prefill(ids)[0].float().numpy().astype(np.float64)
        d = np.abs(lg - g["logits_first"].astype(np.float64))
        out[name] = {"first_max_abs": round(float(d.max()), 6), "first_mean_abs": round(float(d.mean()), 6),
                     "prompt_tokens": int(ids.shape[1])}
        print(name, out[name], flush=True)
    out["method"] = ("oracle/qwen3_cpu.py with f32_linear (FP32 GEMM of the BF16 operands, one rounding) "
                     "against HF's logits_first, over the whole vocabulary")
    (HERE / "reorder_floor.json").write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main()
