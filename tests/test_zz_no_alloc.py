"""The no-allocation entry point (q3_skinny_tiled_noalloc) against the entry
point it varies (q3_skinny_tiled with a caller workspace): the same bits, on
calls in a row through the C ABI, each smaller than the one before, so a
later call's partials land on array memory that an earlier, larger call
left filled."""

import pytest
import torch

from starter_amd import _lib
from starter_amd._lib import call

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def S():
    return torch.cuda.current_stream().cuda_stream


def both(M, N, K, epi, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wt = torch.empty_like(w)
    call("q3_tile16", w.data_ptr(), N, K, wt.data_ptr(), S())
    cols = N // 2 if epi == _lib.EPI_SWIGLU else N
    y0 = torch.randn(M, cols, generator=g).to(torch.bfloat16).to(DEV)  # the residual for EPI_RESID
    y1 = y0.clone()
    ws = torch.empty(max(call("q3_skinny_ws_floats", M, N, K), 1), dtype=torch.float32, device=DEV)
    call("q3_skinny_tiled", x.data_ptr(), K, wt.data_ptr(), M, N, K, epi, y0.data_ptr(), cols, ws.data_ptr(), S())
    call("q3_skinny_tiled_noalloc", x.data_ptr(), K, wt.data_ptr(), M, N, K, epi, y1.data_ptr(), cols, S())
    torch.cuda.synchronize()
    return y0.cpu(), y1.cpu()


def test_noalloc_matches_the_workspace_entry_point():
    limit = call("q3_skinny_scratch_floats")
    cases = [(64, 2560, 9728, _lib.EPI_RESID, 1),   # down at 64 rows: 8 splits, the largest decode partials
             (64, 6144, 2560, _lib.EPI_STORE, 5),   # qkv at 64 rows: 2 splits (both on the loader-wave kernel)
             (16, 2560, 9728, _lib.EPI_RESID, 2),   # down at 16 rows: 8 splits
             (9, 2560, 4096, _lib.EPI_STORE, 3),    # o at 9 rows: 8 splits, smaller still
             (5, 19456, 2560, _lib.EPI_SWIGLU, 4)]  # gate/up: one split, no partials
    sizes = [call("q3_skinny_ws_floats", M, N, K) for M, N, K, _, _ in cases]
    assert sizes == sorted(sizes, reverse=True) and 0 < sizes[0] <= limit
    for M, N, K, epi, seed in cases:
        want, got = both(M, N, K, epi, seed)
        assert torch.equal(got, want), (M, N, K, epi)


def test_noalloc_rejects_shapes_beyond_its_array():
    M, N, K = 64, 4160, 10240
    assert call("q3_skinny_ws_floats", M, N, K) > call("q3_skinny_scratch_floats")
    x = torch.zeros(M, K, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(N, K, dtype=torch.bfloat16, device=DEV)
    y = torch.zeros(M, N, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="q3_skinny_tiled_noalloc failed"):
        call("q3_skinny_tiled_noalloc", x.data_ptr(), K, w.data_ptr(), M, N, K, _lib.EPI_STORE, y.data_ptr(), N, S())
