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
# group of G kv heads) with one wave per kv head, and holds the 32 KB dequant
# table plus a ring of two LDS tile slots (16 token rows of the group's
# entries, K and V).  The split count is chosen so the grid fills the
# workgroup slots of all CUs once: a second, partial round of workgroups
# would leave most CUs idle at the end.  Each split keeps at least
# MIN_CHUNK_TOKENS tokens to amortise the per-workgroup q rotation and the
# LSE merge.
MIN_CHUNK_TOKENS = 256
CHUNK_ALIGN = 16
MI355X_CUS = 256
LDS_BYTES_PER_CU = 160 * 1024


def _waves_per_simd(pd: int, ratio: int) -> int:
    """Occupancy the decode kernel is compiled for (amdgpu_waves_per_eu)."""
    if pd == 256:
        return 2
    return 4 if ratio <= 8 else 3


RING_SLOTS = 2


def lut_bytes(pd: int, g: int) -> int:
    """Dequant-table bytes of a decode workgroup (tq_decode.hip lut_copies):
    256 entries x 32 bank-spread copies, 16 copies for head size 128 with
    fewer than 8 kv heads per workgroup and for head size 256."""
    copies = 32 if pd == 64 or (pd == 128 and g == 8) else 16
    return 256 * 4 * copies


def ring_lds_bytes(pd: int, g: int) -> int:
    """LDS bytes of one decode workgroup of g kv heads (tq_decode.hip
    RingGeom::LDS): the table + RING_SLOTS tile slots x 2 regions of NI 1 KB
    copies, rows padded to an odd number of 16-byte chunks."""
    ech = entry_bytes(pd)[2] // 16
    rch = (g * ech) | 1
    ni = (16 * rch + 63) // 64
    return lut_bytes(pd, g) + RING_SLOTS * 2 * ni * 1024


def decode_group_size(pd: int, num_kv_heads: int, ratio: int) -> int:
    """Heads (waves) per decode workgroup, as the launcher picks them: the
    largest of 8, 4, 2, 1 (at most 4 for pd 256) dividing num_kv_heads whose
    q scratch fits the table and ring when q' is formed in LDS (ratio * pd > 1024)."""
    maxg = 4 if pd == 256 else 8
    g = maxg
    while g >= 1:
        if num_kv_heads % g == 0 and (ratio * pd <= 1024 or
                                      g * ratio * pd * 4 <= ring_lds_bytes(pd, g)):
            return g
        g //= 2
    return 0


def decode_workgroup_shape(num_qo_heads: int, num_kv_heads: int, pd: int) -> tuple[int, int]:
    """(G, workgroups resident per CU) of the decode kernel."""
    ratio = max(1, num_qo_heads // max(1, num_kv_heads))
    G = max(1, decode_group_size(pd, num_kv_heads, ratio))
    by_lds = LDS_BYTES_PER_CU // ring_lds_bytes(pd, G)
    by_waves = 4 * _waves_per_simd(pd, ratio) // G
    return G, max(1, min(by_lds, by_waves))


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

# Sequences one balanced decode plan takes (tq_decode.hip kPlanMaxBatch; the
# plan stages per-sequence lengths in LDS).  Larger decode batches take the
# static-split op.
BALANCED_MAX_BATCH = 1024
