"""The benchmark workloads: seeded Qwen3-4B, five (batch, prompt, new-token) shapes.

Every config uses the same seeded random-init BF16 model (N(0, 0.02) matrices,
norm gains 1.0, seed 0) and prompts of uniform ids in [0, 151643) with an
independent stream per row; the prompt stream's seed is the config number.
"""

from __future__ import annotations

import dataclasses

from .checkpoint import QWEN3_4B, Qwen3Config, seeded_prompt

PROMPT_VOCAB = 151643
MODEL_SEED = 0


@dataclasses.dataclass(frozen=True)
class Workload:
    number: int
    batch: int
    prompt: int
    new_tokens: int
    note: str

    @property
    def name(self) -> str:
        return f"config{self.number}-b{self.batch}-p{self.prompt}-n{self.new_tokens}"

    def prompt_ids(self) -> list[list[int]]:
        return seeded_prompt(self.number, self.batch, self.prompt, PROMPT_VOCAB)


WORKLOADS = {
    1: Workload(1, 1, 32, 32, "correctness config; the CPU oracle runs it in full"),
    2: Workload(2, 1, 1024, 512, "batch-1 weight-streaming decode"),
    3: Workload(3, 16, 512, 256, "skinny-GEMM regime, moderate KV"),
    4: Workload(4, 64, 2048, 128, "MFMA projections, heavy KV"),
    5: Workload(5, 8, 16384, 128, "long-context, attention-dominated"),
}

MODEL: Qwen3Config = QWEN3_4B
