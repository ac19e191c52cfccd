"""ctypes binding of ``libq3.so`` (the C ABI declared in ``include/q3.h``).

Every launcher returns a hipError_t code; ``call`` turns a non-zero code into
``RuntimeError(name, code, hipGetErrorString)``.  There is no fallback: if the
library is missing the import fails loudly (the reference instead fell back to
eager PyTorch when its Triton kernels were unavailable,
``engine/engine.py:45-65``; this engine has exactly one path).
"""

from __future__ import annotations

import ctypes
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libq3.so"

# Mirrors of the #defines in include/q3.h.
X_PLAIN, X_NORM, X_EMBED_NORM = 0, 1, 2
EPI_STORE, EPI_RESID, EPI_SWIGLU, EPI_ARGMAX, EPI_STORE_ARGMAX = 0, 1, 2, 3, 4
GEMV_MAX_M = 8
GEMV_MAX_NORM_K = 4096

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t

#: name -> argtypes (restype int unless listed in _RESTYPES)
SIGNATURES = {
    "q3_error_string": [_I],
    "q3_gemv": [_I, _P, _I, _P, _P, _F, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P, _P, _P, _P, _I, _P],
    "q3_gemv_partials": [_I, _I, _I],
    "q3_gemm": [_P, _I, _P, _I, _I, _I, _I, _P, _I, _P],
    "q3_gemm_tiles_wide": [_I, _I],
    "q3_gemm_splits": [_I, _I, _I],
    "q3_gemm_partials": [_P, _I, _P, _I, _I, _I, _P, _I, _P],
    "q3_gemm_ws_floats": [_I, _I, _I],
    "q3_gemm_ws": [_P, _I, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "q3_swiglu_rows": [_P, _P, _I, _I, _P],
    "q3_skinny": [_P, _I, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "q3_skinny_tiled": [_P, _I, _P, _I, _I, _I, _I, _P, _I, _P, _P],
    "q3_skinny_partials": [_P, _I, _P, _I, _I, _I, _P, _P],
    "q3_skinny_tiled_noalloc": [_P, _I, _P, _I, _I, _I, _I, _P, _I, _P],
    "q3_skinny_scratch_floats": [],
    "q3_skinny_argmax": [_P, _I, _P, _I, _I, _I, _P, _I, _P, _P, _P, _P, _P, _I, _P],
    "q3_tile16": [_P, _I, _I, _P, _P],
    "q3_skinny_splits": [_I, _I, _I],
    "q3_skinny_ws_floats": [_I, _I, _I],
    "q3_rmsnorm": [_P, _I, _P, _P, _I, _I, _I, _F, _P],
    "q3_add_rmsnorm_partials": [_P, _I, _P, _P, _P, _I, _I, _F, _P],
    "q3_add_rmsnorm": [_P, _P, _P, _P, _P, _I, _I, _F, _P],
    "q3_embed_rmsnorm": [_P, _P, _P, _P, _P, _I, _I, _F, _P],
    "q3_qk_norm_rope_kv": [_P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "q3_attn_decode": [_P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _P],
    "q3_attn_merge": [_P, _P, _P, _I, _I, _I, _P],
    "q3_attn_splits": [_I, _I, _I],
    "q3_attn_decode_fused": [_P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _F,
                             _P, _P],
    "q3_attn_fused_grid": [_I, _I, _I, _I, _I],
    "q3_attn_xbuf_words": [_I, _I, _I],
    "q3_attn_decode_pair": [_P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _P, _P],
    "q3_attn_pair_grid": [_I, _I, _I, _I],
    "q3_qkv_attn": [_I, _P, _I, _P, _P, _F, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I,
                    _I, _I, _I, _I, _I, _I, _F, _P, _P],
    "q3_qkv_attn_grid": [_I, _I, _I, _I, _I, _I, _I],
    "q3_down_qkv_attn": [_P, _P, _I, _P, _P, _P, _F, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                         _I, _I, _I, _I, _I, _I, _F, _P, _P],
    "q3_down_qkv_attn_grid": [_I, _I, _I, _I, _I, _I],
    "q3_down_rx_words": [_I],
    "q3_attn_prefill": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P],
    "q3_argmax_finish": [_P, _P, _I, _I, _P, _P, _P, _P, _P, _I, _P],
    "q3_argmax_rows": [_P, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P],
    "q3_graph_begin": [_P],
    "q3_graph_end": [_P, ctypes.POINTER(ctypes.c_void_p)],
    "q3_graph_launch": [_P, _P],
    "q3_graph_destroy": [_P],
}
_RESTYPES = {"q3_error_string": ctypes.c_char_p}

#: entry points that return a count, not an error code
_COUNTS = {"q3_gemv_partials", "q3_attn_splits", "q3_attn_fused_grid", "q3_attn_xbuf_words", "q3_qkv_attn_grid",
           "q3_attn_pair_grid", "q3_down_qkv_attn_grid", "q3_down_rx_words",
           "q3_skinny_splits", "q3_skinny_ws_floats", "q3_skinny_scratch_floats", "q3_gemm_tiles_wide",
           "q3_gemm_splits", "q3_gemm_ws_floats"}

_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load libq3.so once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m starter_amd.build` "
                "(__graft_entry__.build()); the engine has no non-HIP path")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _LIB = handle
    return _LIB


def error_string(code: int) -> str:
    return lib().q3_error_string(code).decode(errors="replace")


def call(name: str, *args) -> int:
    """Invoke ``name``; a non-zero hipError_t raises RuntimeError."""
    rc = getattr(lib(), name)(*args)
    if name in _COUNTS:
        return rc
    if rc != 0:
        raise RuntimeError(f"{name} failed: hipError {rc} ({error_string(rc)})")
    return 0
