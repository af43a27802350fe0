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
# group of kv heads); each split should hold enough 16-token tiles to amortise
# the per-workgroup q rotation, and the grid should carry several waves per
# SIMD (256 CUs x 4 SIMDs) to keep enough loads in flight.
MIN_CHUNK_TOKENS = 256
CHUNK_ALIGN = 16
TARGET_WAVES = 256 * 4 * 6


def choose_splits(batch: int, max_len: int, num_kv_heads: int) -> tuple[int, int]:
    """Return (num_splits, kv_chunk_size) with kv_chunk_size a multiple of 16
    and num_splits * kv_chunk_size >= max_len.  Pure function of its inputs,
    so a captured graph keeps its split layout."""
    max_len = max(1, int(max_len))
    want = max(1, TARGET_WAVES // max(1, batch * num_kv_heads))
    by_len = max(1, max_len // MIN_CHUNK_TOKENS)
    splits = max(1, min(want, by_len))
    chunk = math.ceil(max_len / splits)
    # the decode kernel walks 16-token tiles
    chunk = (chunk + CHUNK_ALIGN - 1) // CHUNK_ALIGN * CHUNK_ALIGN
    splits = math.ceil(max_len / chunk)
    return splits, chunk
