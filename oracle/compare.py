"""Test infrastructure: the token/logit parity criteria used by the GPU tests and smoke().

Per sequence, the contest's quality rule (reference QWEN_ENGINE_CONTRACT.md
"The quality rule") with the tie margin narrowed from 2.0 logits to what BF16
reordering moves:
  * until the candidate's token first differs from the reference's, every
    step's logits are within ``tol`` (max-abs over the vocabulary);
  * at that first differing step, the candidate's token is within ``margin``
    of the reference's maximum logit, i.e. the reference's top-2 gap there
    was a near-tie (``margin`` defaults to 2 * tol).

``replay_judge`` is the contest judge's own check: a stream replayed
teacher-forced through a reference model, every emitted token the argmax or
within the tie margin of it.
"""

from __future__ import annotations

import numpy as np
import torch


def check_stream(got_tokens, got_logits, want_tokens, want_logits, tol: float,
                 margin: float | None = None) -> list[int]:
    """Assert the criterion; return each row's first divergence step (N if none).

    Tokens are [N, B]; logits [N, B, V] (numpy).
    """
    margin = 2 * tol if margin is None else margin
    got_tokens, want_tokens = np.asarray(got_tokens), np.asarray(want_tokens)
    got_logits, want_logits = np.asarray(got_logits), np.asarray(want_logits)
    assert got_tokens.shape == want_tokens.shape, (got_tokens.shape, want_tokens.shape)
    N, B = want_tokens.shape
    firsts = []
    for r in range(B):
        diff = np.nonzero(got_tokens[:, r] != want_tokens[:, r])[0]
        d = int(diff[0]) if len(diff) else N
        for i in range(min(d + 1, N)):
            err = np.abs(got_logits[i, r] - want_logits[i, r]).max()
            assert err <= tol, f"row {r} step {i}: logit max-abs {err:.3f} > {tol}"
        if d < N:
            ref = want_logits[d, r]
            short = ref.max() - ref[got_tokens[d, r]]
            assert short <= margin, (f"row {r} step {d}: chose {got_tokens[d, r]}, {short:.4f} below "
                                     f"the reference's max (reference chose {want_tokens[d, r]}; "
                                     f"margin {margin})")
        firsts.append(d)
    return firsts


@torch.inference_mode()
def replay_judge(model, input_ids, emitted, margin: float = 2.0) -> dict:
    """Replay ``emitted`` ([N][B] ids) teacher-forced through ``model`` (a
    ``Qwen3Oracle``) after the prompt, as the contest judge does with native
    Qwen (reference QWEN_ENGINE_CONTRACT.md "The quality rule").  Returns the
    per-step shortfalls [N, B] (max logit minus the emitted token's logit,
    0 where the emitted token is the argmax) and the failing (step, row)."""
    ids = torch.tensor(input_ids, dtype=torch.int64)
    em = torch.tensor(emitted, dtype=torch.int64)
    B, P = ids.shape
    N = em.shape[0]
    model.reset(B, P + N)
    logits = model.prefill(ids)
    short = np.zeros((N, B))
    for k in range(N):
        lg = logits.float().cpu()
        arg = lg.argmax(dim=-1)
        val = lg.gather(1, em[k].view(B, 1))[:, 0]
        short[k] = torch.where(arg == em[k], torch.zeros_like(val), lg.max(dim=-1).values - val).numpy()
        if k + 1 < N:
            logits = model.forward(em[k].view(B, 1), P + k)
    bad = [(int(k), int(b)) for k, b in zip(*np.nonzero(short > margin))]
    return {"shortfall": short, "failures": bad}
