"""GPU parity of the split-KV decode against the fp32/fp64 dequantize-then-attend
oracle (max-abs 2e-3 / rel 1e-2), at the BASELINE shapes and edge cases."""
import numpy as np
import pytest
import torch

from tests import gpu_cases as G
from turboquant_amd import workloads as W

pytestmark = pytest.mark.gpu


def _check(case, what, **kw):
    cache, pd = G.build_cache(case)
    got, qp, scale = G.run_decode(case, cache, pd, **kw)
    ref = G.oracle_decode(case, cache.cpu().numpy(), qp, pd, scale, signs=kw.get("signs", True))
    G.assert_close(got, ref, what)
    return got, ref


def test_cfg1_decode():
    print("case: cfg1 decode B=1 L=1024 32/8/128", flush=True)
    c = W.cfg1()
    got, _ = _check(c, "cfg1")
    import os
    want = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1_decode.npy"))
    G.assert_close(got, want, "cfg1 vs golden fixture")


def test_cfg3_decode_full_size():
    print("case: cfg3 decode B=8 L=32768 32/8/128 random page permutation", flush=True)
    _check(W.cfg3(), "cfg3")


@pytest.mark.parametrize("hd", [128, 64, 256])
def test_cfg4_ragged(hd):
    batch = {128: 16, 64: 8, 256: 8}[hd]
    print(f"case: cfg4 ragged hd={hd} B={batch} Student-t K", flush=True)
    _check(W.cfg4(batch=batch, hd=hd), f"cfg4 hd{hd}")


@pytest.mark.parametrize("splits,chunk", [(1, None), (3, None), (7, 300), (128, 16), (56, 37)])
def test_split_invariance(splits, chunk):
    """Any split layout covering max_len (2048 here), including chunks that are
    not page multiples, gives the same attention within tolerance."""
    print(f"case: split invariance splits={splits} chunk={chunk}", flush=True)
    c = W.decode_case(21, 3, [1000, 37, 2048], 32, 8, 128)
    _check(c, f"splits={splits}", num_splits=splits, chunk=chunk)


@pytest.mark.parametrize("hd,b,hq,hkv,chunk", [
    (128, 8, 32, 8, 64), (128, 8, 32, 8, 67), (128, 8, 32, 8, 80), (128, 8, 32, 8, 512),
    (64, 8, 32, 8, 80), (256, 4, 16, 8, 80)])
def test_pair_share_grid(hd, b, hq, hkv, chunk):
    """A grid of exactly two workgroups per CU (sequences x 64 splits x head
    groups = 512) serves split pairs with an uneven token share; ragged
    lengths leave some pairs partly or wholly past the end."""
    print(f"case: pair-share grid hd={hd} B={b} {hq}/{hkv} S=64 chunk={chunk}", flush=True)
    lens = [0, 1, 17, 100, 1000, 2047, 2048, 4095][8 - b:]
    c = W.decode_case(41 + chunk + hd, b, lens, hq, hkv, hd)
    _check(c, f"pair hd={hd} chunk={chunk}", num_splits=64, chunk=chunk)


def test_edge_lengths_and_gqa():
    """seq_len 0, 1, 15, 16, 17 and a partial last page; GQA ratios 1, 2, 8, 16."""
    for hq, hkv in ((8, 8), (16, 8), (16, 2), (16, 1)):
        print(f"case: edge lengths hq={hq} hkv={hkv}", flush=True)
        c = W.decode_case(31 + hq, 6, [0, 1, 15, 16, 17, 333], hq, hkv, 128)
        got, ref = _check(c, f"edges {hq}/{hkv}", num_splits=4, chunk=96)
        assert np.all(got[0] == 0)  # empty sequence -> zeros


def test_no_rotation_signs_none():
    print("case: signs=None", flush=True)
    c = W.decode_case(41, 2, [500, 77], 32, 8, 128)
    _check(c, "no rotation", signs=False)


def test_out_of_range_page_is_empty():
    """A page id outside the cache contributes nothing (instead of faulting)."""
    print("case: out of range page", flush=True)
    c = W.decode_case(51, 1, [64], 32, 8, 128)
    cache, pd = G.build_cache(c)
    c2 = dict(c)
    bt = c["block_table"].copy()
    bt[0, 3] = 1 << 20  # last 16 tokens point outside the pool
    c2["block_table"] = bt
    got, qp, scale = G.run_decode(c2, cache, pd, num_splits=2, chunk=32)
    c3 = dict(c)
    c3["seq_lens"] = np.array([48], np.int32)
    ref = G.oracle_decode(c3, cache.cpu().numpy(), qp, pd, scale)
    G.assert_close(got, ref, "oob page")


def test_graph_replay_matches_eager():
    """The op captured in a HIP graph: every replay equals the eager result."""
    print("case: graph replay", flush=True)
    from turboquant_amd import ops
    from turboquant_amd.geometry import hadamard_signs
    c = W.decode_case(61, 4, [700, 1300, 64, 2000], 32, 8, 128)
    cache, pd = G.build_cache(c)
    eager, qp, scale = G.run_decode(c, cache, pd, num_splits=5, chunk=416)
    dev = G.DEV
    qt = torch.from_numpy(qp).to(dev)
    bt = torch.from_numpy(c["block_table"]).to(dev)
    ind = bt.reshape(-1).contiguous()
    ip = torch.arange(5, dtype=torch.int32, device=dev) * bt.shape[1]
    sl = torch.from_numpy(c["seq_lens"]).to(dev)
    o = torch.empty((4, 32, pd), dtype=torch.float16, device=dev)
    po = torch.empty((20, 32, pd), dtype=torch.float32, device=dev)
    pl = torch.empty((20, 32), dtype=torch.float32, device=dev)
    s = hadamard_signs(pd, dev)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        ops.decode_paged_splitkv(qt, cache, ind, ip, sl, 8, 128, pd, scale, s, o, po, pl, 5, 416)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        ops.decode_paged_splitkv(qt, cache, ind, ip, sl, 8, 128, pd, scale, s, o, po, pl, 5, 416)
    for i in range(4):
        o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(o.float().cpu().numpy(), eager), f"replay {i}"


@pytest.mark.parametrize("bs", [32, 64])
def test_larger_pages(bs):
    """Pages of 32 and 64 tokens (block_size a multiple of 16): the write
    scatters into them and the decode walks two or four tiles per page."""
    print(f"case: block_size {bs}", flush=True)
    import math

    import oracle
    from turboquant_amd import ops
    from turboquant_amd.geometry import choose_splits, hadamard_signs
    rng = np.random.default_rng(bs)
    hq, hkv, hd = 32, 8, 128
    lens = [1000, 77, 2 * bs, 3 * bs + 5]
    npg = [math.ceil(l / bs) for l in lens]
    nb = sum(npg) + 3
    perm = rng.permutation(nb).astype(np.int32)
    maxp = max(npg)
    bt = np.zeros((len(lens), maxp), np.int32)
    slots, off = [], 0
    for b, p in enumerate(npg):
        bt[b, :p] = perm[off:off + p]
        off += p
        t = np.arange(lens[b])
        slots.append(bt[b, t // bs] * bs + t % bs)
    slots = np.concatenate(slots).astype(np.int32)
    k, v = W.write_inputs(rng, len(slots), hkv, hd)
    q = rng.standard_normal((len(lens), hq, hd)).astype(np.float16)
    dev = G.DEV
    cache = torch.zeros((2, nb, bs, hkv, 80), dtype=torch.uint8, device=dev)
    signs = hadamard_signs(128, dev)
    ops.quantize_write_kv_cache(cache, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
                                signs, torch.from_numpy(slots).to(dev), hd, 128)
    ref_cache = np.zeros(tuple(cache.shape), np.uint8)
    oracle.write_kv_cache(ref_cache, k, v, hadamard_signs(128).numpy(), slots, hd, 128)
    got_cache = cache.cpu().numpy()
    assert np.array_equal(got_cache, ref_cache)
    b = len(lens)
    max_len = maxp * bs
    S, cs = choose_splits(b, max_len, hkv, hq, 128)
    o = torch.empty((b, hq, 128), dtype=torch.float16, device=dev)
    po = torch.empty((b * S, hq, 128), dtype=torch.float32, device=dev)
    pl = torch.empty((b * S, hq), dtype=torch.float32, device=dev)
    indptr = np.arange(b + 1, dtype=np.int32) * maxp
    ops.decode_paged_splitkv(torch.from_numpy(q).to(dev), cache,
                             torch.from_numpy(bt.reshape(-1)).to(dev),
                             torch.from_numpy(indptr).to(dev),
                             torch.tensor(lens, dtype=torch.int32, device=dev), hkv, hd, 128,
                             1.0 / np.sqrt(hd), signs, o, po, pl, S, cs)
    torch.cuda.synchronize()
    ref = oracle.decode(q, got_cache, bt.reshape(-1), indptr, np.array(lens, np.int32), hkv, 128,
                        1.0 / np.sqrt(hd), hadamard_signs(128).numpy())
    G.assert_close(o.float().cpu().numpy(), ref, f"block_size {bs}")
