"""Independent float64 numpy restatement used to pin the C oracle.

It shares no code with oracle/tq_oracle.c: the rotation is an explicit
Sylvester-Hadamard matrix (scipy.linalg.hadamard) instead of butterflies, the
codes come from np.searchsorted(side='right') instead of a binary search, and
decode attends in the ORIGINAL domain (inverse-rotated K^/V^ against the
original q) instead of the rotated one.  Agreement therefore pins the
butterfly order, sign placement, boundary set and tie rule, nibble order and
the rotation / inverse rotation of the decode path.
"""
from __future__ import annotations

import numpy as np
from scipy.linalg import hadamard

# Reference values (turboquant/codebook.py:37-55, 4-bit), in float64.
CENTROIDS_F64 = np.array([
    -2.7326368237440100, -2.0693470280837980, -1.6180344937899930, -1.2562490887894980,
    -0.9423683558764893, -0.6567591430551046, -0.3880823046410021, -0.1284153814744918,
    0.1284153814744918, 0.3880823046410021, 0.6567591430551046, 0.9423683558764893,
    1.2562490887894980, 1.6180344937899930, 2.0693470280837980, 2.7326368237440100])


def rotation_matrix(pd: int, signs: np.ndarray) -> np.ndarray:
    """R with y = R x = H (s * x) / sqrt(pd); R is orthogonal, R^-1 = R^T."""
    h = hadamard(pd).astype(np.float64)
    return h * np.asarray(signs, np.float64)[None, :] / np.sqrt(pd)


def quantize_rows(x: np.ndarray, pd: int, signs: np.ndarray):
    """x float [N, hd] -> (codes uint8 [N, pd], norms float64 [N], rotated float64 [N, pd])."""
    n, hd = x.shape
    xp = np.zeros((n, pd))
    xp[:, :hd] = x
    norms = np.sqrt((xp * xp).sum(axis=1))
    unit = np.where(norms[:, None] > 1e-8, xp / np.where(norms > 1e-8, norms, 1)[:, None], 0.0)
    rot = unit @ rotation_matrix(pd, signs).T
    bounds = (CENTROIDS_F64[:-1] + CENTROIDS_F64[1:]) / 2 / np.sqrt(pd)
    codes = np.searchsorted(bounds, rot, side="right").astype(np.uint8)
    return codes, norms, rot


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """[..., pd] codes -> [..., pd/2] bytes, even dim in the high nibble."""
    return ((codes[..., 0::2] << 4) | codes[..., 1::2]).astype(np.uint8)


def unpack_codes(packed: np.ndarray) -> np.ndarray:
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), np.uint8)
    out[..., 0::2] = packed >> 4
    out[..., 1::2] = packed & 0x0F
    return out


def gather_entries(kv_cache: np.ndarray, indices, indptr, seq_len: int, b: int, kvh: int):
    """-> (K entries, V entries) uint8 [seq_len, ebs] of sequence b, head kvh."""
    bs = kv_cache.shape[2]
    t = np.arange(seq_len)
    pages = np.asarray(indices)[np.asarray(indptr)[b] + t // bs]
    ent = t % bs
    return kv_cache[0, pages, ent, kvh], kv_cache[1, pages, ent, kvh]


def dequant_original(entries: np.ndarray, pd: int, signs: np.ndarray, codebook32) -> np.ndarray:
    """Entries -> vectors in the ORIGINAL domain (float64 [L, pd])."""
    qb = pd // 2
    codes = unpack_codes(entries[:, :qb])
    norms = entries[:, qb:qb + 2].copy().view(np.float16).astype(np.float64)[:, 0]
    rot = np.asarray(codebook32, np.float64)[codes] * (norms[:, None] / np.sqrt(pd))
    return rot @ rotation_matrix(pd, signs)  # R^T y, row-vector form


def decode_original(q: np.ndarray, kv_cache: np.ndarray, indices, indptr, seq_lens,
                    num_kv_heads: int, pd: int, sm_scale: float, signs, codebook32):
    """Attention of fp16 q [B, Hq, pd] over the dequantized cache, original domain."""
    b_, hq, _ = q.shape
    ratio = hq // num_kv_heads
    out = np.zeros((b_, hq, pd))
    for b in range(b_):
        L = int(seq_lens[b])
        if L == 0:
            continue
        for kvh in range(num_kv_heads):
            ke, ve = gather_entries(kv_cache, indices, indptr, L, b, kvh)
            K = dequant_original(ke, pd, signs, codebook32)
            V = dequant_original(ve, pd, signs, codebook32)
            for r in range(ratio):
                h = kvh * ratio + r
                s = K @ q[b, h].astype(np.float64) * sm_scale
                s -= s.max()
                p = np.exp(s)
                out[b, h] = p @ V / p.sum()
    return out
