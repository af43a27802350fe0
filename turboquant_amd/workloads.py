"""Seeded synthetic workloads of the benchmark configurations (numpy PCG64),
shared by bench.py and the tests.

cfg1: q [1,32,128], K/V [1024,8,128] ~ N(0,1), seed 1, contiguous pages.
cfg2: K/V [8192,8,128] ~ N(0,1) with 4 fixed outlier channels per head x20,
      slots a seeded permutation of 8192 slots in 512 pages, seed 2.
cfg3: q [8,32,128]; 8 x 32768 tokens of N(0,1) K/V; 16384 pages assigned by
      a seeded permutation, seed 3.
cfg4: B=64, L ~ U[1024, 32768], K Student-t(3), V N(0,1), seed 4; also
      hd 64 (16q/4kv) and hd 256 (16q/2kv).
The generators return host numpy arrays; build_cache, decode_inputs and
device_case put a workload on a GPU through this package's write kernel.
"""
from __future__ import annotations

import math

import numpy as np

BLOCK = 16


def outlier_channels(rng, num_heads: int, head_dim: int, count: int = 4) -> np.ndarray:
    return np.stack([rng.choice(head_dim, size=count, replace=False) for _ in range(num_heads)])


def write_inputs(rng, n: int, h: int, hd: int, outliers: bool = False, k_dist: str = "normal"):
    if k_dist == "t3":
        k = rng.standard_t(3, size=(n, h, hd))
    else:
        k = rng.standard_normal((n, h, hd))
    v = rng.standard_normal((n, h, hd))
    if outliers:
        ch = outlier_channels(rng, h, hd)  # same channels for K and V
        for hh in range(h):
            k[:, hh, ch[hh]] *= 20.0
            v[:, hh, ch[hh]] *= 20.0
    return k.astype(np.float16), v.astype(np.float16)


def cfg1(seed: int = 1):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((1, 32, 128)).astype(np.float16)
    k, v = write_inputs(rng, 1024, 8, 128)
    pages = 1024 // BLOCK
    return dict(q=q, k=k, v=v, num_blocks=pages, slots=np.arange(1024, dtype=np.int32),
                block_table=np.arange(pages, dtype=np.int32)[None, :],
                seq_lens=np.array([1024], np.int32), num_kv_heads=8, head_dim=128)


def cfg2(seed: int = 2, n: int = 8192, pages: int = 512):
    rng = np.random.default_rng(seed)
    k, v = write_inputs(rng, n, 8, 128, outliers=True)
    slots = rng.permutation(pages * BLOCK)[:n].astype(np.int32)
    return dict(k=k, v=v, slots=slots, num_blocks=pages, num_kv_heads=8, head_dim=128)


def paged_layout(rng, seq_lens, max_pages: int | None = None):
    """Random permutation of a page pool; block_table [B, max_pages] int32 and
    slot_mapping for writing every token of every sequence."""
    seq_lens = np.asarray(seq_lens, np.int64)
    npg = [math.ceil(int(l) / BLOCK) for l in seq_lens]
    total = int(sum(npg))
    max_pages = max_pages or max(1, max(npg))
    perm = rng.permutation(total).astype(np.int32)
    bt = np.zeros((len(seq_lens), max_pages), np.int32)
    slots = []
    off = 0
    for b, p in enumerate(npg):
        bt[b, :p] = perm[off:off + p]
        off += p
        t = np.arange(int(seq_lens[b]))
        slots.append(bt[b, t // BLOCK] * BLOCK + t % BLOCK)
    slots = np.concatenate(slots).astype(np.int32) if slots else np.zeros(0, np.int32)
    return bt, slots, max(total, 1)


def decode_case(seed: int, batch: int, seq_lens, hq: int, hkv: int, hd: int,
                k_dist: str = "normal"):
    rng = np.random.default_rng(seed)
    seq_lens = np.asarray(seq_lens, np.int32)
    q = rng.standard_normal((batch, hq, hd)).astype(np.float16)
    bt, slots, nb = paged_layout(rng, seq_lens)
    n = int(seq_lens.sum())
    k, v = write_inputs(rng, n, hkv, hd, k_dist=k_dist)
    return dict(q=q, k=k, v=v, slots=slots, block_table=bt, seq_lens=seq_lens,
                num_blocks=nb, num_kv_heads=hkv, head_dim=hd)


def cfg3(seed: int = 3, batch: int = 8, seq_len: int = 32768):
    return decode_case(seed, batch, [seq_len] * batch, 32, 8, 128)


def cfg4(seed: int = 4, batch: int = 64, hd: int = 128, lo: int = 1024, hi: int = 32768):
    hq, hkv = {64: (16, 4), 128: (32, 8), 256: (16, 2)}[hd]
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=batch)
    return decode_case(seed + 1000 * hd, batch, lens, hq, hkv, hd, k_dist="t3")


def cache_bytes(num_blocks: int, hkv: int, hd: int) -> tuple[tuple[int, ...], int]:
    pd = max(64, 1 << (hd - 1).bit_length())
    dc = pd // 64
    ebs = (dc * 32 + dc * 2 + 15) & ~15
    return (2, num_blocks, BLOCK, hkv, ebs), pd


def algorithmic_decode_bytes(seq_lens, hkv: int, hd: int, hq: int) -> int:
    """codes+norms of every (token, kv head, K/V) + page-table entries + q + o."""
    pd = max(64, 1 << (hd - 1).bit_length())
    per = pd // 2 + 2 * (pd // 64)
    sl = np.asarray(seq_lens, np.int64)
    b = len(sl)
    return int(sl.sum() * hkv * 2 * per + np.ceil(sl / BLOCK).sum() * 4 + 2 * b * hq * pd * 2)


def algorithmic_write_bytes(n: int, h: int, hd: int, in_bytes: int = 2) -> int:
    pd = max(64, 1 << (hd - 1).bit_length())
    per = pd // 2 + 2 * (pd // 64)
    return int(2 * n * h * hd * in_bytes + n * 4 + 2 * n * h * per)


# ----------------------------------------------------------- on the device

def build_cache(case, device="cuda:0"):
    """The case's K/V written into a fresh cache on `device` by the write
    kernel; returns (cache, padded_dim)."""
    import torch

    from . import ops
    from .geometry import hadamard_signs
    dev = torch.device(device)
    hkv, hd = case["num_kv_heads"], case["head_dim"]
    shape, pd = cache_bytes(case["num_blocks"], hkv, hd)
    cache = torch.zeros(shape, dtype=torch.uint8, device=dev)
    k = torch.from_numpy(case["k"]).to(dev)
    v = torch.from_numpy(case["v"]).to(dev)
    if k.shape[0]:
        ops.quantize_write_kv_cache(cache, k, v, hadamard_signs(pd, dev),
                                    torch.from_numpy(case["slots"]).to(dev), hd, pd)
    return cache, pd


def decode_inputs(case, pd, device="cuda:0"):
    """Device tensors of a case: padded q, strided page table, seq_lens."""
    import torch
    dev = torch.device(device)
    q = case["q"]
    b, hq, hd = q.shape
    qp = np.zeros((b, hq, pd), np.float16)
    qp[:, :, :hd] = q
    bt = torch.from_numpy(case["block_table"]).to(dev)
    return dict(
        qp=qp, q=torch.from_numpy(qp).to(dev), indices=bt.reshape(-1).contiguous(),
        indptr=(torch.arange(b + 1, dtype=torch.int32, device=dev) * bt.shape[1]).contiguous(),
        seq=torch.from_numpy(np.asarray(case["seq_lens"], np.int32)).to(dev))


def device_case(seed, seq_lens, hq, hkv, hd, k_dist="normal", chunk_tokens=1 << 16,
                device="cuda:0"):
    """A decode case too large for host-generated K/V: q, page table and slot
    mapping from numpy (seeded), K/V drawn on the GPU (seeded torch generator;
    K ~ Student-t(3) for k_dist "t3") and written through the write kernel,
    whose bytes are pinned against the oracle by the write tests.  Returns
    (case, cache, pd); case has no "k"/"v"."""
    import torch

    from . import ops
    from .geometry import hadamard_signs
    dev = torch.device(device)
    rng = np.random.default_rng(seed)
    seq_lens = np.asarray(seq_lens, np.int32)
    b = len(seq_lens)
    q = rng.standard_normal((b, hq, hd)).astype(np.float16)
    bt, slots, nb = paged_layout(rng, seq_lens)
    shape, pd = cache_bytes(nb, hkv, hd)
    cache = torch.zeros(shape, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    signs = hadamard_signs(pd, dev)
    st = torch.from_numpy(slots).to(dev)
    for a in range(0, len(slots), chunk_tokens):
        n = min(chunk_tokens, len(slots) - a)
        if k_dist == "t3":
            # Student-t(3) = N(0,1) / sqrt(chi2_3 / 3), chi2_3 = sum of 3 squared normals
            z = torch.randn((n, hkv, hd), generator=g, device=dev)
            c2 = torch.randn((3, n, hkv, hd), generator=g, device=dev).square().sum(0)
            k = (z / torch.sqrt(c2 / 3.0)).half()
        else:
            k = torch.randn((n, hkv, hd), generator=g, device=dev).half()
        v = torch.randn((n, hkv, hd), generator=g, device=dev).half()
        ops.quantize_write_kv_cache(cache, k, v, signs, st[a:a + n], hd, pd)
    torch.cuda.synchronize()
    case = dict(q=q, slots=slots, block_table=bt, seq_lens=seq_lens, num_blocks=nb,
                num_kv_heads=hkv, head_dim=hd)
    return case, cache, pd
