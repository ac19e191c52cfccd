"""Test infrastructure: the token/logit parity criterion used by the GPU tests and smoke().

Per sequence, the contest's quality rule (reference QWEN_ENGINE_CONTRACT.md
"The quality rule") with a margin of 2*tol logits instead of 2.0: until the
candidate's token first differs from the reference's, every step's logits are
within tol (max-abs over the vocabulary); at that first differing step the
candidate's token is within 2*tol of the reference's maximum logit, i.e. the
reference's top-2 gap there was a near-tie at BF16 reordering precision.
"""

from __future__ import annotations

import numpy as np


def check_stream(got_tokens, got_logits, want_tokens, want_logits, tol: float) -> list[int]:
    """Assert the criterion; return each row's first divergence step (N if none).

    Tokens are [N, B]; logits [N, B, V] (numpy).
    """
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
            assert short <= 2 * tol, (f"row {r} step {d}: chose {got_tokens[d, r]}, {short:.3f} below "
                                      f"the reference's max (reference chose {want_tokens[d, r]})")
        firsts.append(d)
    return firsts
