"""ctypes binding of libtq_hip.so (declarations in include/turboquant_amd.h).

The library is built in-tree by ``python -m turboquant_amd.build`` (or
``__graft_entry__.build()``).  Loading never falls back to anything: if the
library is missing or fails to load, every op raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtq_hip.so")

TQ_F32, TQ_F16, TQ_BF16 = 0, 1, 2

# symbol -> (restype, argtypes); mirrors include/turboquant_amd.h
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float
SIGNATURES = {
    "tq_quantize_write_kv_cache": (_I32, [_P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _P, _P,
                                          _I64, _I32, _I32, _I32, _I32, _I32, _I64, _P]),
    "tq_decode_paged_splitkv": (_I32, [_P, _I64, _I64, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                       _I32, _I32, _I32, _I32, _I64, _F32, _P, _I32, _I32,
                                       _P, _P, _P, _P]),
    "tq_decode_paged_balanced": (_I32, [_P, _I64, _I64, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                        _I32, _I32, _I32, _I32, _I64, _F32, _P, _I32, _P, _P,
                                        _P, _P, _P]),
    "tq_decode_paged_balanced_noalloc": (_I32, [_P, _I64, _I64, _P, _P, _P, _P, _P, _I32, _I32,
                                                _I32, _I32, _I32, _I32, _I32, _I64, _F32, _P,
                                                _P, _P]),
    "tq_decode_partials_balanced": (_I32, [_P, _I64, _I64, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                           _I32, _I32, _I32, _I32, _I64, _F32, _P, _I32, _P,
                                           _P, _P, _P]),
    "tq_decode_balanced_rows": (_I32, [_I32, _I32, _I32, _I32]),
    "tq_decode_partials": (_I32, [_P, _I64, _I64, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                                  _I32, _I32, _I64, _F32, _P, _I32, _I32, _P, _P, _P]),
    "tq_diag_decode_stream": (_I32, [_P, _I64, _I64, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                                     _I32, _I32, _I64, _F32, _P, _I32, _I32, _P, _P, _I32, _P]),
    "tq_diag_stream_read": (_I32, [_P, _I64, _P, _P]),
    "tq_combine_splits": (_I32, [_P, _P, _I32, _I32, _I32, _I32, _P, _P, _P]),
    "tq_dequant_paged": (_I32, [_P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I64, _P, _P,
                                _P, _I64, _P]),
    "tq_prefill_attention": (_I32, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64,
                                    _I64, _I32, _I32, _I32, _I32, _I32, _F32, _P]),
    "tq_prefill_attention_ws": (_I32, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P,
                                       _I64, _I64, _I32, _I32, _I32, _I32, _I32, _F32, _P, _I64,
                                       _P]),
    "tq_prefill_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32, _I32]),
    "tq_mse_quantize": (_I32, [_P, _I64, _I32, _I32, _I32, _P, _P, _P, _P, _P]),
    "tq_mse_dequantize": (_I32, [_P, _P, _I64, _I32, _I32, _I32, _P, _P, _P, _P]),
    "tq_prod_quantize": (_I32, [_P, _I64, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P]),
    "tq_prod_dequantize": (_I32, [_P, _P, _P, _P, _I64, _I32, _I32, _I32, _P, _P, _P, _P]),
    "tq_prod_quantize_qjl": (_I32, [_P, _I64, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _P, _P]),
    "tq_prod_dequantize_qjl": (_I32, [_P, _P, _P, _P, _I64, _I32, _I32, _I32, _P, _P, _P, _P,
                                      _P, _P]),
    "tq_diag_mse_bucketize": (_I32, [_I32]),
    "tq_e2e_add_rms_norm": (_I32, [_P, _P, _P, _P, _I64, _I32, _F32, _P]),
    "tq_e2e_qk_norm_rope": (_I32, [_P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _I32, _I32, _I32,
                                   _F32, _P, _P, _P]),
    "tq_e2e_silu_mul": (_I32, [_P, _P, _I64, _I32, _P]),
    "tq_last_error": (ctypes.c_char_p, []),
    "tq_abi_version": (_I32, []),
}
ABI_VERSION = 9

_lib = None


class TQError(RuntimeError):
    """A tq_* entry point returned non-zero."""


def load():
    """Load libtq_hip.so once; raise if it is absent (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"TurboQuant HIP library not built: {LIB_PATH} is missing. "
            "Run `python -m turboquant_amd.build` (hipcc, gfx950).")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    v = lib.tq_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"libtq_hip.so ABI {v} != expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().tq_last_error().decode(errors="replace")
        raise TQError(f"{what} failed (rc={rc}): {msg}")
