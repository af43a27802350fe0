"""Cache geometry, rotation signs and the split heuristic.

Geometry follows the reference backend (turboquant/vllm_backend_fused.py:24-25,
56-86): pd = next_pow2(head_dim), dc = pd/64 chunks of 64 dims, 32 code bytes
and one fp16 norm per chunk, entry padded to 16 bytes.
"""
from __future__ import annotations

import functools
import math

TILE_DIMS = 64
QUANT_BYTES_PER_CHUNK = 32
SIGN_SEED = 42


def next_pow2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def padded_dim(head_size: int) -> int:
    """pd = next_pow2(head_size), at least 64 (one 64-dim chunk)."""
    return max(TILE_DIMS, next_pow2(head_size))


def entry_bytes(head_size: int) -> tuple[int, int, int]:
    """(qbytes, nbytes, ebs) for one (token, kv head) entry: 32/80/144 style."""
    pd = padded_dim(head_size)
    dc = pd // TILE_DIMS
    qbytes = dc * QUANT_BYTES_PER_CHUNK
    nbytes = dc * 2
    ebs = (qbytes + nbytes + 15) & ~15
    return qbytes, nbytes, ebs


@functools.lru_cache(maxsize=None)
def _signs_list(pd: int) -> tuple[float, ...]:
    import torch
    gen = torch.Generator(device="cpu")
    gen.manual_seed(SIGN_SEED)
    s = torch.sign(torch.randn(pd, generator=gen))
    s[s == 0] = 1.0
    return tuple(float(v) for v in s.tolist())


def hadamard_signs(pd: int, device="cpu"):
    """+-1 fp32 [pd]: sign(randn(pd)) from a CPU torch.Generator seeded with 42,
    zeros mapped to +1 (TurboQuantFusedImpl._ensure, vllm_backend_fused.py:217-224)."""
    import torch
    return torch.tensor(_signs_list(pd), dtype=torch.float32, device=device)


# Decode split heuristic for MI355X.  A workgroup serves (sequence, split,
# group of G kv heads) with one wave per kv head, and holds a double-buffered
# LDS staging area sized for the largest G of its head size.  The split count
# is chosen so the grid fills the workgroup slots of all CUs once: a second,
# partial round of workgroups would leave most CUs idle at the end.  Each
# split keeps at least MIN_CHUNK_TOKENS tokens to amortise the per-workgroup
# q rotation and the LSE merge.
MIN_CHUNK_TOKENS = 256
CHUNK_ALIGN = 16
MI355X_CUS = 256
LDS_BYTES_PER_CU = 160 * 1024
# waves per SIMD the decode kernel's register use allows, by padded head size
_WAVES_PER_SIMD = {64: 6, 128: 4, 256: 2}


def decode_workgroup_shape(num_qo_heads: int, num_kv_heads: int, pd: int) -> tuple[int, int]:
    """(G, splits resident per CU) of the decode kernel; G mirrors the
    launcher in tq_decode.hip (largest divisor of num_kv_heads up to 8 (4 for
    pd 256) whose rotated-q scratch fits the first LDS slot)."""
    ebs = entry_bytes(pd)[2]
    maxg = 4 if pd == 256 else 8
    slot_bytes = maxg * 2 * 16 * ebs  # V of one two-tile step for each of maxg waves
    ratio = max(1, num_qo_heads // max(1, num_kv_heads))
    G = 1
    for g in range(maxg, 0, -1):
        if num_kv_heads % g == 0 and g * ratio * pd * 4 <= slot_bytes:
            G = g
            break
    spw = decode_splits_per_workgroup(num_qo_heads, num_kv_heads, pd)
    table = 65536 if spw == 2 else 1024  # the dequant table (64 copies with two splits)
    by_lds = LDS_BYTES_PER_CU // (2 * slot_bytes * spw + table)
    by_waves = 4 * _WAVES_PER_SIMD.get(pd, 2) // (G * spw)
    return G, spw * max(1, min(by_lds, by_waves))


def decode_splits_per_workgroup(num_qo_heads: int, num_kv_heads: int, pd: int) -> int:
    """Splits one decode workgroup serves: 2 (one 16-wave workgroup per CU)
    when q' fits the register path and pd >= 128, else 1 (mirrors the
    launcher in tq_decode.hip)."""
    ratio = max(1, num_qo_heads // max(1, num_kv_heads))
    return 2 if (ratio * pd <= 1024 and pd >= 128) else 1


def choose_splits(batch: int, max_len: int, num_kv_heads: int, num_qo_heads: int | None = None,
                  padded_dim: int = 128, num_cus: int = MI355X_CUS) -> tuple[int, int]:
    """Return (num_splits, kv_chunk_size) with kv_chunk_size a multiple of 16
    and num_splits * kv_chunk_size >= max_len.  Pure function of its inputs,
    so a captured graph keeps its split layout."""
    max_len = max(1, int(max_len))
    hq = num_qo_heads if num_qo_heads else 4 * num_kv_heads
    G, per_cu = decode_workgroup_shape(hq, num_kv_heads, padded_dim)
    units = max(1, batch * (num_kv_heads // G))
    want = max(1, (num_cus * per_cu) // units)
    by_len = max(1, max_len // MIN_CHUNK_TOKENS)
    splits = max(1, min(want, by_len))
    chunk = math.ceil(max_len / splits)
    # the decode kernel walks 16-token tiles
    chunk = (chunk + CHUNK_ALIGN - 1) // CHUNK_ALIGN * CHUNK_ALIGN
    splits = math.ceil(max_len / chunk)
    return splits, chunk
