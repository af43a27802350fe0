"""The fp16 write kernel's bucketize (tq_write.hip, write_f16_kernel) restated
in numpy and checked against the oracle's binary search (the reference's
quantize_write_kernel.cuh:34-46) on every boundary, its fp32 neighbours, signed
zeros and random values, for each head size.

The kernel clamps 2|v| (integer bits, minus 2 for v < 0) to the four binades
above the smallest scaled boundary and looks up a 64-entry table indexed by
the exponent's low three bits and the top three mantissa bits.  This is exact
only if every 1/8-binade bin holds at most one boundary, which is checked
here too.  CPU only.
"""
import numpy as np
import pytest

import oracle

PDS = (64, 128, 256)


def _scale(pd):
    # the launcher's constant: 1.0f / sqrtf((float)pd) in fp32
    return np.float32(1.0) / np.sqrt(np.float32(pd))


def _table(scale):
    T = [int(np.float32(b * scale).view(np.uint32)) for b in oracle.boundaries()[8:]]
    e0 = T[0] >> 23
    thr2 = np.full(64, 0xFFFFFFFF, np.uint64)
    below8 = np.full(64, 8, np.uint64)
    for idx in range(64):
        e = e0 + (((idx >> 3) - e0) & 7)
        if e > e0 + 3:
            continue
        start = (e << 23) | ((idx & 7) << 20)
        end = start + (1 << 20)
        below8[idx] = 8 + sum(t < start for t in T)
        inside = [t for t in T if start <= t < end]
        assert len(inside) <= 1, f"bin {idx} holds {len(inside)} boundaries"
        if inside:
            thr2[idx] = 2 * inside[0]
    lo2 = e0 << 24
    hi2 = ((e0 + 4) << 24) - 1
    return T, thr2, below8, lo2, hi2


def _fast_codes(v, scale):
    _, thr2, below8, lo2, hi2 = _table(scale)
    v = np.asarray(v, np.float32) + np.float32(0.0)  # the fma's +0 addend: -0 -> +0
    bits = v.view(np.uint32).astype(np.uint64)
    m = np.where(bits >> 31, 0xFFFFFFFF, 0).astype(np.uint64)
    av2 = (((bits + m) & 0xFFFFFFFF) << 1) & 0xFFFFFFFF
    off = (np.clip(av2, lo2, hi2) >> 18) & 0x1F8
    idx = (off // 8).astype(np.int64)
    cnt8 = below8[idx] + (av2 >= thr2[idx]).astype(np.uint64)
    return ((cnt8 ^ m) & 15).astype(np.int64)


@pytest.mark.parametrize("pd", PDS)
def test_bins_hold_at_most_one_boundary(pd):
    T, _, _, lo2, hi2 = _table(_scale(pd))
    assert all(lo2 <= 2 * t <= hi2 for t in T)


@pytest.mark.parametrize("pd", PDS)
def test_fast_bucketize_equals_binary_search(pd):
    scale = _scale(pd)
    assert scale == oracle.inv_sqrt_pd(pd)
    bs = (oracle.boundaries() * scale).astype(np.float32)
    vals = [0.0, -0.0, np.inf, -np.inf, 1e-30, -1e-30, 5.0, -5.0, 1e-45, -1e-45]
    for b in bs:
        u = np.float32(b).view(np.uint32)
        for d in range(-3, 4):
            if int(u) + d >= 0:
                w = np.uint32(int(u) + d).view(np.float32)
                vals += [w, -w]
    rng = np.random.default_rng(pd)
    vals += list(rng.standard_normal(4000).astype(np.float32) * scale * 2)
    vals += list(rng.standard_t(2, 2000).astype(np.float32) * scale)
    # every bin edge of the table's range and its neighbours
    e0 = int(np.float32(bs[8]).view(np.uint32)) >> 23
    for e in range(e0 - 1, e0 + 5):
        for m3 in range(8):
            edge = (e << 23) | (m3 << 20)
            for d in (-1, 0, 1):
                w = np.uint32(edge + d).view(np.float32)
                vals += [w, -w]
    vals = np.array(vals, np.float32)
    want = np.array([oracle.bucketize(x, bs) for x in vals])
    got = _fast_codes(vals, scale)
    bad = np.nonzero(want != got)[0]
    assert bad.size == 0, f"{bad.size} mismatches, e.g. {vals[bad[:5]]} -> {got[bad[:5]]} vs {want[bad[:5]]}"
