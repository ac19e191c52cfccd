"""The C ABI: libq3.so loads and exports every entry point include/q3.h declares.

No compute calls here (there is no GPU in the CPU suite); argument checks that
fail before any launch are exercised, since they return an error code without
touching the device.
"""

import ctypes
import pathlib
import re

import pytest

from starter_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parents[1]


def header_functions() -> list[str]:
    text = (ROOT / "include" / "q3.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q3_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    names = header_functions()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name


def test_python_binding_covers_the_header():
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_header_constants_match_binding():
    text = (ROOT / "include" / "q3.h").read_text()
    consts = dict(re.findall(r"#define (Q3_\w+) (\d+)", text))
    for name in ("X_PLAIN", "X_NORM", "X_EMBED_NORM", "EPI_STORE", "EPI_RESID", "EPI_SWIGLU",
                 "EPI_ARGMAX", "EPI_STORE_ARGMAX", "GEMV_MAX_M", "GEMV_MAX_NORM_K"):
        assert int(consts["Q3_" + name]) == getattr(_lib, name), name


def test_error_string():
    assert _lib.error_string(0)
    assert _lib.error_string(1)  # hipErrorInvalidValue


def test_bad_arguments_raise_without_launching():
    # M = 0 and K not a multiple of 8 are rejected before any device work.
    with pytest.raises(RuntimeError, match="q3_gemv failed"):
        _lib.call("q3_gemv", 0, None, 0, None, None, 0.0, None, None, 0, 4, 8, 0, None, 0, None, None, None,
                  None, None, 0, None)
    # Step records need the argmax epilogue, a position and a feed table.
    with pytest.raises(RuntimeError, match="q3_argmax_finish failed"):
        _lib.call("q3_argmax_finish", 1, 1, 4, 2, 1, 1, None, None, None, 0, None)  # B > 1 advancing pos: counter
    with pytest.raises(RuntimeError, match="q3_argmax_finish failed"):
        _lib.call("q3_argmax_finish", 1, 1, 4, 1, 1, None, None, 1, 1, 8, None)   # records without a position
    with pytest.raises(RuntimeError, match="q3_gemm failed"):
        _lib.call("q3_gemm", None, 0, None, 4, 4, 60, 0, None, 0, None)
    with pytest.raises(RuntimeError, match="q3_attn_decode failed"):
        _lib.call("q3_attn_decode", None, 0, None, 0, None, None, None, None, None, None, None, None, None,
                  None, 1, 32, 7, 64, 1, 1e-6, 0.1, None)


def test_attention_splits_policy():
    # One split from 128 (sequence, KV head) pairs at moderate context or 512 at any;
    # else about 512 workgroups (768 from 64 pairs) of >= 256 keys, 128-key splits while CUs would idle.
    assert _lib.call("q3_attn_splits", 1, 8, 64) == 2     # two one-block splits (config 1)
    assert _lib.call("q3_attn_splits", 1, 8, 63) == 1
    assert _lib.call("q3_attn_splits", 4, 8, 64) == 1
    assert _lib.call("q3_attn_splits", 1, 8, 1536) == 16   # 96 keys per split
    assert _lib.call("q3_attn_splits", 1, 8, 2048) == 16   # 128 (96 would take 22)
    assert _lib.call("q3_attn_splits", 1, 8, 3000) == 24
    assert _lib.call("q3_attn_splits", 16, 8, 768) == 1
    assert _lib.call("q3_attn_splits", 16, 8, 16384) == 6
    assert _lib.call("q3_attn_splits", 64, 8, 2176) == 1
    assert _lib.call("q3_attn_splits", 8, 8, 16512) == 12
    assert _lib.call("q3_attn_splits", 4, 8, 1536) == 6
    assert _lib.call("q3_attn_splits", 200, 8, 100) == 1


def test_gemv_partials():
    assert _lib.call("q3_gemv_partials", 1, 151936, _lib.EPI_ARGMAX) == 151936 // 4 // 4
    assert _lib.call("q3_gemv_partials", 8, 151936, _lib.EPI_ARGMAX) == 151936 // 2 // 4
    assert _lib.call("q3_gemv_partials", 1, 2560, _lib.EPI_STORE) == 2560 // 4


def test_noalloc_projection_rejects_oversize_before_any_launch():
    """q3_skinny_tiled_noalloc checks its fixed 8 MiB array against the shape's
    split partials before touching a device (hipErrorOutOfMemory)."""
    M, N, K = 64, 4160, 10240
    assert _lib.call("q3_skinny_scratch_floats") == 2 * 1024 * 1024
    assert _lib.call("q3_skinny_ws_floats", M, N, K) > _lib.call("q3_skinny_scratch_floats")
    rc = _lib.lib().q3_skinny_tiled_noalloc(1, K, 1, M, N, K, _lib.EPI_STORE, 1, N, None)
    assert rc == 2  # hipErrorOutOfMemory
    # Every decode projection at 64 rows fits (o and down, 8 splits, are the largest).
    for N, K in ((6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728)):
        assert _lib.call("q3_skinny_ws_floats", 64, N, K) <= _lib.call("q3_skinny_scratch_floats")


def test_prompt_gemm_split_policy():
    """Split-K on the 256 x 256 tiling only below its tile threshold: about one
    workgroup per CU, three splits from 128 tiles, at most 16 splits of >= 4
    K steps; none for decode-sized M or where whole tiles fill the CUs."""
    H = 2560
    assert _lib.call("q3_gemm_splits", 1024, H, 4096) == 6
    assert _lib.call("q3_gemm_splits", 1024, H, 9728) == 6
    assert _lib.call("q3_gemm_splits", 256, H, 4096) == 16
    assert _lib.call("q3_gemm_splits", 512, H, 4096) == 12
    assert _lib.call("q3_gemm_splits", 3840, H, 4096) == 3
    assert _lib.call("q3_gemm_splits", 3072, H, 9728) == 2
    assert _lib.call("q3_gemm_splits", 255, H, 4096) == 0       # narrow tiles
    assert _lib.call("q3_gemm_splits", 4096, H, 4096) == 0      # 160 whole tiles
    assert _lib.call("q3_gemm_splits", 8192, H, 9728) == 0
    assert _lib.call("q3_gemm_splits", 1024, H, 320) == 0       # 5 K steps: no split of >= 4 steps
    assert _lib.call("q3_gemm_splits", 700, 3800, 576) == 2
    with pytest.raises(RuntimeError, match="q3_gemm_partials failed"):
        _lib.call("q3_gemm_partials", None, 4096, None, 1024, H, 4096, None, 17, None)  # > 16 splits
