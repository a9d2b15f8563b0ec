"""ctypes binding of ``libflashloop_amd.so`` (the C ABI declared in include/flashloop_amd.h).

The library is loaded from this package directory.  There is no fallback: if the
library is missing or a call fails, a ``RuntimeError`` is raised with the library's
own message (``fl_last_error``), mirroring how the reference refuses to run without
its extension (flashloop/kivi_backend.py:38-49).
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("FLASHLOOP_AMD_LIB", Path(__file__).resolve().parent / "libflashloop_amd.so"))

FL_OK = 0
FL_E_INVALID = -1
FL_E_LAUNCH = -2
FL_E_CAPACITY = -3

HEAD_DIM = 128
GROUP = 64


class FlCacheView(C.Structure):
    """Mirror of ``fl_cache_view`` (include/flashloop_amd.h)."""

    _fields_ = [
        ("batch", C.c_int32),
        ("heads", C.c_int32),
        ("token_capacity", C.c_int32),
        ("tail_capacity", C.c_int32),
        ("row_capacity", C.c_int32 * 4),
        ("key_codes", C.c_void_p * 4),
        ("key_meta", C.c_void_p * 4),
        ("value_codes", C.c_void_p * 4),
        ("value_meta", C.c_void_p * 4),
        ("rank", C.c_void_p * 2),
        ("tail_key", C.c_void_p * 4),
        ("tail_value", C.c_void_p * 4),
        ("packed_tokens", C.c_void_p),
        ("tail_tokens", C.c_void_p),
        ("max_packed_tokens", C.c_int32),
        ("max_tail_tokens", C.c_int32),
        ("value_meta_token", C.c_void_p),
        ("key_meta_half", C.c_void_p * 4),
        ("value_meta_half", C.c_void_p * 4),
    ]


_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64
_F32 = C.c_float
_F64 = C.c_double
_SZ = C.c_size_t
_VIEW = C.POINTER(FlCacheView)
_PP = C.POINTER(C.c_void_p)

# name -> (restype, argtypes); every symbol include/flashloop_amd.h declares
SIGNATURES = {
    "fl_last_error": (C.c_char_p, []),
    "fl_abi_version": (_I32, []),
    "fl_pack_kv_groups": (_I32, [_VIEW, _I32, _PP, _PP, _I64, _I32, _PP, _I64, _P, _I32, _PP, _PP, _P]),
    "fl_decode_attn_dense_workspace": (_SZ, [_VIEW]),
    "fl_decode_attn_dense": (_I32, [_VIEW, _I32, _P, _P, _P, _F32, _P, _P, _I64, _P, _SZ, _P]),
    "fl_decode_attn_dense_noalloc_max_bytes": (_SZ, []),
    "fl_decode_attn_dense_noalloc": (_I32, [_VIEW, _I32, _P, _P, _P, _F32, _P, _P, _I64, _P]),
    "fl_decode_attn_dense_pair_workspace": (_SZ, [_VIEW]),
    "fl_decode_attn_dense_pair": (_I32, [_VIEW, _P, _P, _P, _P, _P, _P, _P, _P, _F32, _P, _I64, _P, _SZ, _P]),
    "fl_profile_dense_reader": (_I32, [_I32, _I32]),
    "fl_profile_dense_reader_read": (_I32, [C.POINTER(_F32), C.POINTER(_I32)]),
    "fl_decode_topk": (_I32, [_P, _I64, _I32, _P, _I32, _F64, _I32, _P, _P, _P, _P, _P, _P, _P]),
    "fl_decode_attn_dense_select": (_I32, [_VIEW, _I32, _P, _P, _P, _F32, _P, _P, _I64, _F64, _I32, _P, _P, _P, _P,
                                           _P, _P, _P, _SZ, _P]),
    "fl_decode_selected_workspace": (_SZ, [_VIEW, _I32]),
    "fl_decode_selected_pv": (_I32, [_VIEW, _I32, _P, _P, _P, _I32, _P, _P, _P, _P, _SZ, _P]),
    "fl_decode_attn_sparse_delta": (
        _I32,
        [_VIEW, _I32, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _F32, _P, _P, _SZ, _P],
    ),
    "fl_decode_attn_sparse_delta_fused": (
        _I32,
        [_VIEW, _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _F32, _P, _P, _P, _SZ, _P],
    ),
    "fl_gather_rows": (_I32, [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "fl_scatter_rows": (_I32, [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "fl_hidden_delta_score": (_I32, [_P, _P, _I64, _I32, _P, _P]),
    "fl_select_tokens": (_I32, [_P, _I32, _I32, _F64, _P, _I32, _P, _P, _P, _P, _P]),
    "fl_gemv_bf16": (_I32, [_P, _I32, _I64, _I32, _I32, _PP, _I32, _I32, _PP, _I64, _P, _I64, _P, _P, _I32, _P]),
    "fl_norm_chain": (_I32, [_I32, _I32, _F32, _P, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "fl_gemv_bf16_chain": (_I32, [_I32, _I32, _F32, _P, _P, _P, _P, _P, _P, _I64, _PP, _I32, _I32, _PP, _I64, _P,
                                  _I64, _P, _P, _I32, _P]),
    "fl_append_tail": (_I32, [_VIEW, _PP, _PP, _PP, _P, _P]),
}

_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m flashloop_amd.build` "
                "(flashloop_amd has no CPU fallback)"
            )
        lib = C.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != FL_OK:
        msg = load().fl_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def ptr_array(ptrs) -> C.Array:
    arr = (C.c_void_p * len(ptrs))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr
