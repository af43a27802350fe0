"""CPU oracle for the TurboQuant quantized paged-KV hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, where it is the checker, never the thing
measured or shipped.  The product (turboquant_amd) never imports it.

numpy wrappers over libtq_oracle.so (built from tq_oracle.c by the Makefile in
this directory).  The C file carries the reference citations per function.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libtq_oracle.so")
_lib = None


def build() -> str:
    """Compile libtq_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "libtq_oracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64, i32, f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.tq_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.tq_oracle_f16_to_f32.restype = f32
        L.tq_oracle_f32_to_f16.argtypes = [f32]
        L.tq_oracle_f32_to_f16.restype = ctypes.c_uint16
        L.tq_oracle_inv_sqrt_pd.argtypes = [i32]
        L.tq_oracle_inv_sqrt_pd.restype = f32
        L.tq_oracle_bucketize.argtypes = [f32, P]
        L.tq_oracle_bucketize.restype = i32
        L.tq_oracle_fwht_f32.argtypes = [P, i32]
        L.tq_oracle_fwht_f32.restype = None
        L.tq_oracle_codebook.restype = ctypes.POINTER(f32)
        L.tq_oracle_boundaries.restype = ctypes.POINTER(f32)
        L.tq_oracle_quantize_vec.argtypes = [P, i32, i32, P, P]
        L.tq_oracle_quantize_vec.restype = None
        L.tq_oracle_write_kv_cache.argtypes = [P, P, P, P, i64, i64, i64, i64, P, P,
                                               i64, i32, i32, i32, i32, i32, i64]
        L.tq_oracle_write_kv_cache.restype = i32
        L.tq_oracle_decode.argtypes = [P, i64, i64, P, P, P, P, P, i32, i32, i32, i32,
                                       i32, i32, f32, P, P]
        L.tq_oracle_decode.restype = i32
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def codebook() -> np.ndarray:
    return np.ctypeslib.as_array(lib().tq_oracle_codebook(), shape=(16,)).copy()


def boundaries() -> np.ndarray:
    return np.ctypeslib.as_array(lib().tq_oracle_boundaries(), shape=(15,)).copy()


def inv_sqrt_pd(pd: int) -> np.float32:
    return np.float32(lib().tq_oracle_inv_sqrt_pd(pd))


def bucketize(val: float, scaled_boundaries: np.ndarray) -> int:
    b = np.ascontiguousarray(scaled_boundaries, dtype=np.float32)
    return lib().tq_oracle_bucketize(float(np.float32(val)), _ptr(b))


def fwht_f32(x: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().tq_oracle_fwht_f32(_ptr(v), v.shape[-1])
    return v


def f32_to_f16_bits(x: float) -> int:
    return int(lib().tq_oracle_f32_to_f16(float(np.float32(x))))


def quantize_vec(x: np.ndarray, pd: int, signs: np.ndarray) -> np.ndarray:
    """One vector -> qbytes codes + fp16 norm repeated pd/64 times (uint8)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    s = np.ascontiguousarray(signs, dtype=np.float32)
    out = np.zeros(pd // 2 + 2 * (pd // 64), dtype=np.uint8)
    lib().tq_oracle_quantize_vec(_ptr(x), x.shape[0], pd, _ptr(s), _ptr(out))
    return out


def write_kv_cache(kv_cache: np.ndarray, key: np.ndarray, value: np.ndarray,
                   signs: np.ndarray, slot_mapping: np.ndarray, head_dim: int,
                   padded_dim: int) -> None:
    """In-place scatter-quantize into kv_cache uint8 [2, num_blocks, bs, H, ebs].

    key/value: float16 [N, H, head_dim] (any strides on the first two dims).
    """
    assert kv_cache.dtype == np.uint8 and kv_cache.ndim == 5 and kv_cache.shape[0] == 2
    assert kv_cache.flags.c_contiguous
    assert key.dtype == np.float16 and value.dtype == np.float16
    key = key if key.strides[-1] == 2 else np.ascontiguousarray(key)
    value = value if value.strides[-1] == 2 else np.ascontiguousarray(value)
    n, h = key.shape[0], key.shape[1]
    _, nb, bs, hk, ebs = kv_cache.shape
    assert hk == h
    slots = np.ascontiguousarray(slot_mapping, dtype=np.int32)
    s = np.ascontiguousarray(signs, dtype=np.float32)
    k_slab = kv_cache[0]
    v_slab = kv_cache[1]
    rc = lib().tq_oracle_write_kv_cache(
        _ptr(k_slab), _ptr(v_slab), _ptr(key), _ptr(value),
        key.strides[0] // 2, key.strides[1] // 2, value.strides[0] // 2, value.strides[1] // 2,
        _ptr(s), _ptr(slots), n, h, head_dim, padded_dim, bs, ebs, nb)
    if rc != 0:
        raise ValueError(f"tq_oracle_write_kv_cache rc={rc}")


def decode(q: np.ndarray, kv_cache: np.ndarray, indices: np.ndarray, indptr: np.ndarray,
           seq_lens: np.ndarray, num_kv_heads: int, padded_dim: int, sm_scale: float,
           signs: np.ndarray | None) -> np.ndarray:
    """Dequantize-then-attend.  q float16 [B, Hq, pd] -> float32 [B, Hq, pd]."""
    assert q.dtype == np.float16 and q.strides[-1] == 2
    b, hq, pd = q.shape
    assert pd == padded_dim
    _, nb, bs, hk, ebs = kv_cache.shape
    assert hk == num_kv_heads and kv_cache.flags.c_contiguous
    out = np.zeros((b, hq, pd), dtype=np.float32)
    ind = np.ascontiguousarray(indices, dtype=np.int32)
    ip = np.ascontiguousarray(indptr, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    sp = None
    if signs is not None:
        s = np.ascontiguousarray(signs, dtype=np.float32)
        sp = _ptr(s)
    rc = lib().tq_oracle_decode(
        _ptr(q), q.strides[0] // 2, q.strides[1] // 2, _ptr(kv_cache[0]), _ptr(kv_cache[1]),
        _ptr(ind), _ptr(ip), _ptr(sl), b, hq, num_kv_heads, pd, bs, ebs,
        float(sm_scale), sp, _ptr(out))
    if rc != 0:
        raise ValueError(f"tq_oracle_decode rc={rc}")
    return out
