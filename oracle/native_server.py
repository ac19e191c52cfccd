"""Native Qwen behind the contest's streaming protocol -- TEST INFRASTRUCTURE.

The contest times native Qwen (Transformers' greedy loop) through the same
pipe and clock as the candidate, and its TTFT/TPOT medians set the candidate's
latency gates (reference QWEN_ENGINE_CONTRACT.md "What is measured").  Here
native Qwen is the CPU oracle (``qwen3_cpu.Qwen3Oracle``, bit-identical to
HF's CPU path on the seeded model), streamed one step at a time:

    python -m oracle.native_server MODEL_PATH BATCH PROMPT NEW

Only tests use it, as the native side of ``starter_amd.protocol.run_workload``.
"""

from __future__ import annotations

import sys
import time

import torch

from oracle.qwen3_cpu import Qwen3Oracle, argmax_first


class NativeCpu:
    """The baseline greedy loop (reference tests/test_equivalence.py:72-86), yielding per step."""

    def __init__(self, model_path: str):
        from starter_amd.checkpoint import load_checkpoint
        cfg, tensors = load_checkpoint(model_path)
        self.VOCAB = cfg.vocab_size
        self.orc = Qwen3Oracle(cfg, tensors, torch.bfloat16)

    @torch.inference_mode()
    def generate(self, input_ids, max_new_tokens: int):
        ids = torch.tensor(input_ids, dtype=torch.int64)
        B, P = ids.shape
        self.orc.reset(B, P + max_new_tokens)
        logits = self.orc.prefill(ids)
        for step in range(max_new_tokens):
            tok = argmax_first(logits)
            yield tok.tolist()
            if step + 1 < max_new_tokens:
                logits = self.orc.forward(tok.view(B, 1), P + step)


def main(argv) -> int:
    from starter_amd.protocol import serve
    model_path, batch, prompt, new = argv[0], int(argv[1]), int(argv[2]), int(argv[3])
    t0 = time.perf_counter()
    native = NativeCpu(model_path)
    warm = [[(7 * r + 13 * t) % native.VOCAB for t in range(prompt)] for r in range(batch)]
    serve(native, warm, new, load_s=time.perf_counter() - t0)
    return 0


if __name__ == "__main__":
    raise SystemExit(main(sys.argv[1:]))
