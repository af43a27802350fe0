"""Seeded random sweep over geometries the fixed cases do not combine: decode
(balanced plan and the reference's static splits) against the fp64 oracle
at the north-star tolerance, and the write bit-exact against the oracle.
Every case draws head size, kv heads, GQA ratio, batch and ragged lengths
(zeros included) from its own seed, printed before it runs."""
import numpy as np
import pytest
import torch

from tests import gpu_cases as G
from turboquant_amd import workloads as W
from tests.test_gpu_write import _diff_report, _gpu_cache, _oracle_cache

pytestmark = pytest.mark.gpu


def _decode_geometry(seed):
    rng = np.random.default_rng(5000 + seed)
    hd = int(rng.choice([64, 96, 128, 192, 256]))
    hkv = int(rng.choice([1, 2, 4, 8, 16]))
    ratio = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 12, 16]))
    while hkv * ratio > 64:
        ratio //= 2
    b = int(rng.integers(1, 25))
    budget = 24000 // max(1, hkv)  # oracle time: tokens x kv heads
    lens = rng.integers(0, 3001, size=b)
    lens[rng.random(b) < 0.15] = 0
    lens[rng.random(b) < 0.15] = rng.integers(1, 40)
    while lens.sum() > budget:
        lens = lens // 2
    return hd, hkv, ratio, b, lens.astype(np.int32), ("t3" if seed % 3 == 0 else "normal")


@pytest.mark.parametrize("seed", range(40))
def test_decode_sweep(seed):
    hd, hkv, ratio, b, lens, kd = _decode_geometry(seed)
    hq = hkv * ratio
    print(f"case: decode sweep seed={seed} hd={hd} {hq}/{hkv} B={b} tokens={int(lens.sum())} "
          f"K {kd}", flush=True)
    c = W.decode_case(7000 + seed, b, lens, hq, hkv, hd, k_dist=kd)
    cache, pd = G.build_cache(c)
    cache_np = cache.cpu().numpy()
    got_b, qp, scale, _ = G.run_balanced(c, cache, pd)
    ref = G.oracle_decode(c, cache_np, qp, pd, scale)
    G.assert_close(got_b, ref, f"balanced seed {seed}")
    got_s, _, _ = G.run_decode(c, cache, pd)
    G.assert_close(got_s, ref, f"static seed {seed}")
    empty = lens == 0
    assert np.all(got_b[empty] == 0) and np.all(got_s[empty] == 0)


@pytest.mark.parametrize("seed", range(20))
def test_write_sweep(seed):
    rng = np.random.default_rng(9000 + seed)
    hd = int(rng.choice([64, 80, 96, 128, 192, 256]))
    h = int(rng.choice([1, 2, 4, 8]))
    n = int(rng.integers(1, 1500))
    nb = (n + 15) // 16 + int(rng.integers(0, 8))
    dtype = [torch.float16, torch.float32, torch.bfloat16][seed % 3]
    print(f"case: write sweep seed={seed} hd={hd} H={h} n={n} {dtype}", flush=True)
    k, v = W.write_inputs(rng, n, h, hd, outliers=bool(seed % 2), k_dist="t3" if seed % 4 == 1 else "normal")
    if dtype == torch.bfloat16:  # values exactly representable in both
        k = torch.from_numpy(k).to(torch.bfloat16).to(torch.float16).numpy()
        v = torch.from_numpy(v).to(torch.bfloat16).to(torch.float16).numpy()
    slots = rng.permutation(nb * 16)[:n].astype(np.int32)
    slots[rng.random(n) < 0.05] = -1  # skipped tokens (padding)
    shape, pd = W.cache_bytes(nb, h, hd)
    ref = _oracle_cache(shape, k, v, slots, hd, pd, fill=0x5A)
    got = _gpu_cache(shape, k, v, slots, hd, pd, fill=0x5A, dtype=dtype)
    assert np.array_equal(ref, got), _diff_report(ref, got)
