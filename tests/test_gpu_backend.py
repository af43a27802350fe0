"""The vLLM-facing backend driven with a stand-in attention-metadata object:
prefill writes the cache through do_kv_cache_update, decode goes through
forward(), and the result matches the oracle."""
from dataclasses import dataclass

import numpy as np
import pytest
import torch

from tests import gpu_cases as G
from turboquant_amd import workloads as W

pytestmark = pytest.mark.gpu


@dataclass
class Meta:
    max_query_len: int
    num_actual_tokens: int
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    query_start_loc: torch.Tensor
    slot_mapping: torch.Tensor


@pytest.mark.parametrize("forced", ["", "gfx950_static"])
def test_backend_write_then_decode(forced, monkeypatch):
    print(f"case: backend write+decode forced={forced!r}", flush=True)
    from turboquant_amd import decoder_dispatch as dd
    from turboquant_amd.vllm_backend_fused import TurboQuantBackend, TurboQuantFusedImpl
    monkeypatch.setenv("TQ_FORCE_KERNEL", forced)
    dd.pick_decode_op.cache_clear()
    dev = G.DEV
    hq, hkv, hd, bs = 32, 8, 128, 16
    lens = [300, 1000, 17]
    c = W.decode_case(71, 3, lens, hq, hkv, hd)
    nb = c["num_blocks"]
    shape = TurboQuantBackend.get_kv_cache_shape(nb, bs, hkv, hd, "fp8")
    assert TurboQuantBackend.get_kv_cache_page_size(bs, hkv, hd, torch.float16, "fp8") == \
        2 * bs * hkv * 80
    cache = torch.zeros(shape, dtype=torch.uint8, device=dev)
    impl = TurboQuantFusedImpl(hq, hd, 1.0 / np.sqrt(hd), hkv, None, None, "fp8")
    k = torch.from_numpy(c["k"]).to(dev).view(-1, hkv * hd)
    v = torch.from_numpy(c["v"]).to(dev).view(-1, hkv * hd)
    slots = torch.from_numpy(c["slots"]).to(dev)
    impl.do_kv_cache_update(None, k.view(-1, hkv, hd), v.view(-1, hkv, hd), cache, slots)
    b = len(lens)
    q = torch.from_numpy(c["q"]).to(dev).view(b, hq * hd)
    meta = Meta(1, b, torch.from_numpy(c["block_table"]).to(dev),
                torch.tensor(lens, dtype=torch.int32, device=dev),
                torch.arange(b + 1, dtype=torch.int32, device=dev), slots[:b])
    out = torch.empty((b, hq * hd), dtype=torch.float16, device=dev)
    impl.forward(None, q, None, None, cache, meta, output=out)
    torch.cuda.synchronize()
    ref = G.oracle_decode(c, cache.cpu().numpy(), c["q"], 128, 1.0 / np.sqrt(hd))
    G.assert_close(out.float().cpu().numpy().reshape(b, hq, hd), ref, "backend")
    # the balanced op by default, the reference op name when forced
    assert impl._decode_op_name == (dd.STATIC_KERNEL_NAME if forced else dd.KERNEL_NAME)
    dd.pick_decode_op.cache_clear()


def test_backend_prefill_fresh_attention():
    print("case: backend prefill", flush=True)
    from turboquant_amd.vllm_backend_fused import TurboQuantFusedImpl
    dev = G.DEV
    hq, hkv, hd = 8, 2, 64
    impl = TurboQuantFusedImpl(hq, hd, 0.125, hkv, None, None, "fp8")
    lens = [5, 9]
    n = sum(lens)
    g = torch.Generator().manual_seed(0)
    q = torch.randn(n, hq * hd, generator=g).half().to(dev)
    k = torch.randn(n, hkv * hd, generator=g).half().to(dev)
    v = torch.randn(n, hkv * hd, generator=g).half().to(dev)
    meta = Meta(9, n, None, None, torch.tensor([0, 5, 14], dtype=torch.int32, device=dev), None)
    out = impl.forward(None, q, k, v, None, meta)
    q3, k3, v3 = (x.float().cpu().view(n, -1, hd) for x in (q, k, v))
    for a, b in ((0, 5), (5, 14)):
        for h in range(hq):
            kk, vv = k3[a:b, h // 4], v3[a:b, h // 4]
            s = q3[a:b, h] @ kk.T * 0.125
            s = s + torch.triu(torch.full_like(s, float("-inf")), 1)
            ref = torch.softmax(s, -1) @ vv
            got = out.float().cpu().view(n, hq, hd)[a:b, h]
            assert torch.allclose(got, ref, atol=2e-2), (a, h)


@pytest.mark.parametrize("hq,hkv,hd,cpu_copies", [(32, 8, 128, False), (8, 2, 64, False),
                                                   (32, 8, 128, True), (16, 2, 256, False),
                                                   (16, 2, 96, False)])
def test_backend_mixed_batch_with_cached_context(hq, hkv, hd, cpu_copies):
    """A max_query_len > 1 batch: a fresh prompt, two chunks of longer prompts
    whose earlier tokens are already cached, and a decode row.  Chunks attend
    the dequantized cached context plus their fresh K/V (causal); the decode
    row attends the dequantized cache; the fresh prompt its own K/V.  All
    against a float64 reference (tests/npref.py dequantization)."""
    print(f"case: backend mixed batch {hq}/{hkv}/{hd}", flush=True)
    import oracle
    from tests import npref
    from turboquant_amd.geometry import hadamard_signs, padded_dim
    from turboquant_amd.vllm_backend_fused import TurboQuantBackend, TurboQuantFusedImpl
    dev = G.DEV
    rng = np.random.default_rng(hd + hq)
    ctxs = [0, 300, 500, 16]
    qls = [20, 37, 1, 5]
    lens = [c + q for c, q in zip(ctxs, qls)]
    bt, slots, nb = W.paged_layout(rng, lens)
    n_all = int(sum(lens))
    k_all, v_all = W.write_inputs(rng, n_all, hkv, hd)
    q_new = rng.standard_normal((sum(qls), hq, hd)).astype(np.float16)
    shape = TurboQuantBackend.get_kv_cache_shape(nb, W.BLOCK, hkv, hd, "fp8")
    cache = torch.zeros(shape, dtype=torch.uint8, device=dev)
    scale = 1.0 / np.sqrt(hd)
    impl = TurboQuantFusedImpl(hq, hd, scale, hkv, None, None, "fp8")
    impl.do_kv_cache_update(None, torch.from_numpy(k_all).to(dev), torch.from_numpy(v_all).to(dev),
                            cache, torch.from_numpy(slots).to(dev))
    # the batch's new tokens are the last qls[i] tokens of each request
    starts = np.concatenate([[0], np.cumsum(lens)])
    new_idx = np.concatenate([np.arange(starts[i] + ctxs[i], starts[i + 1]) for i in range(4)])
    kn = torch.from_numpy(k_all[new_idx]).to(dev).view(-1, hkv * hd)
    vn = torch.from_numpy(v_all[new_idx]).to(dev).view(-1, hkv * hd)
    qn = torch.from_numpy(q_new).to(dev).view(-1, hq * hd)
    qsl = np.concatenate([[0], np.cumsum(qls)]).astype(np.int32)
    meta = Meta(max(qls), int(sum(qls)), torch.from_numpy(bt).to(dev),
                torch.tensor(lens, dtype=torch.int32, device=dev),
                torch.from_numpy(qsl).to(dev), None)
    if cpu_copies:  # vLLM's host copies of the boundaries: no device read
        meta.query_start_loc_cpu = torch.from_numpy(qsl)
        meta.seq_lens_cpu = torch.tensor(lens, dtype=torch.int32)
    out = impl.forward(None, qn, kn, vn, cache, meta)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(-1, hq, hd)

    pd = padded_dim(hd)
    signs = hadamard_signs(pd).numpy()
    cb = oracle.codebook()
    cache_np = cache.cpu().numpy()
    indptr = np.arange(5, dtype=np.int32) * bt.shape[1]
    ref = np.zeros_like(got, dtype=np.float64)
    g = hq // hkv
    for i in range(4):
        a, b = qsl[i], qsl[i + 1]
        for kvh in range(hkv):
            ke, ve = npref.gather_entries(cache_np, bt.reshape(-1), indptr, lens[i], i, kvh)
            kd = npref.dequant_original(ke, pd, signs, cb)[:, :hd]
            vd = npref.dequant_original(ve, pd, signs, cb)[:, :hd]
            fk = k_all[starts[i] + ctxs[i]:starts[i + 1], kvh].astype(np.float64)
            fv = v_all[starts[i] + ctxs[i]:starts[i + 1], kvh].astype(np.float64)
            if qls[i] == 1 and ctxs[i] > 0:  # decode row: the whole cache
                K, V = kd, vd
            else:  # cached context, then the fresh chunk
                K = np.concatenate([kd[:ctxs[i]], fk])
                V = np.concatenate([vd[:ctxs[i]], fv])
            for r in range(g):
                h = kvh * g + r
                for j in range(qls[i]):
                    vis = ctxs[i] + j + 1
                    s = K[:vis] @ q_new[a + j, h].astype(np.float64) * scale
                    p = np.exp(s - s.max())
                    ref[a + j, h] = p @ V[:vis] / p.sum()
    G.assert_close(got, ref, "mixed batch")


def test_dequant_paged_matches_float64_dequantization():
    print("case: dequant_paged", flush=True)
    import oracle
    from tests import npref
    from turboquant_amd import ops
    from turboquant_amd.geometry import hadamard_signs, padded_dim
    for hd, hkv in ((128, 8), (64, 4), (256, 2), (96, 2)):
        c = W.decode_case(200 + hd, 1, [333], 4 * hkv, hkv, hd)
        cache, pd = G.build_cache(c)
        pages = torch.from_numpy(c["block_table"][0]).to(G.DEV).contiguous()
        out_k = torch.full((340, hkv, hd), 7.0, dtype=torch.float16, device=G.DEV)
        out_v = torch.full_like(out_k, 7.0)
        signs = hadamard_signs(pd, G.DEV)
        ops.dequant_paged(cache, pages, 333, hkv, hd, pd, signs, out_k, out_v)
        torch.cuda.synchronize()
        cache_np = cache.cpu().numpy()
        indptr = np.array([0, c["block_table"].shape[1]], np.int32)
        for kvh in range(hkv):
            ke, ve = npref.gather_entries(cache_np, c["block_table"].reshape(-1), indptr, 333, 0, kvh)
            for ent, got in ((ke, out_k), (ve, out_v)):
                want = npref.dequant_original(ent, pd, signs.cpu().numpy(), oracle.codebook())[:, :hd]
                g = got[:333, kvh].float().cpu().numpy()
                assert np.abs(g - want).max() <= 2e-3 * max(1.0, np.abs(want).max()), hd
        assert (out_k[333:] == 7.0).all()  # rows past num_tokens untouched
        # rows with a wider stride (not packed): the same values, bit for bit
        wide_k = torch.full((340, hkv + 1, hd), 7.0, dtype=torch.float16, device=G.DEV)
        wide_v = torch.full_like(wide_k, 7.0)
        ops.dequant_paged(cache, pages, 333, hkv, hd, pd, signs, wide_k[:, :hkv], wide_v[:, :hkv])
        torch.cuda.synchronize()
        assert torch.equal(wide_k[:333, :hkv], out_k[:333])
        assert torch.equal(wide_v[:333, :hkv], out_v[:333])
        assert (wide_k[:, hkv:] == 7.0).all() and (wide_k[333:] == 7.0).all()


def test_backend_decode_batches_beyond_one_balanced_plan():
    """A balanced plan takes at most 1024 sequences: a 1100-sequence decode
    batch goes through the reference's static-split op (same kernels), and
    the 1030 decode rows of a mixed batch through the balanced op in chunks
    of at most 1024; both against the oracle."""
    print("case: backend decode of 1100 sequences and a mixed batch of 1030 + 1", flush=True)
    from turboquant_amd import decoder_dispatch as dd
    from turboquant_amd.geometry import BALANCED_MAX_BATCH
    from turboquant_amd.vllm_backend_fused import TurboQuantBackend, TurboQuantFusedImpl
    dd.pick_decode_op.cache_clear()
    assert BALANCED_MAX_BATCH == 1024
    dev = G.DEV
    hq, hkv, hd, bs = 8, 2, 128, 16
    rng = np.random.default_rng(5)
    lens = rng.integers(1, 70, size=1100).tolist()
    c = W.decode_case(72, len(lens), lens, hq, hkv, hd)
    shape = TurboQuantBackend.get_kv_cache_shape(c["num_blocks"], bs, hkv, hd, "fp8")
    cache = torch.zeros(shape, dtype=torch.uint8, device=dev)
    impl = TurboQuantFusedImpl(hq, hd, 1.0 / np.sqrt(hd), hkv, None, None, "fp8")
    k = torch.from_numpy(c["k"]).to(dev)
    v = torch.from_numpy(c["v"]).to(dev)
    slots = torch.from_numpy(c["slots"]).to(dev)
    impl.do_kv_cache_update(None, k.view(-1, hkv, hd), v.view(-1, hkv, hd), cache, slots)
    b = len(lens)
    bt = torch.from_numpy(c["block_table"]).to(dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    q = torch.from_numpy(c["q"]).to(dev).view(b, hq * hd)
    ref = G.oracle_decode(c, cache.cpu().numpy(), c["q"], 128, 1.0 / np.sqrt(hd))
    # pure decode batch of 1100
    meta = Meta(1, b, bt, sl, torch.arange(b + 1, dtype=torch.int32, device=dev), slots[:b])
    out = torch.empty((b, hq * hd), dtype=torch.float16, device=dev)
    impl.forward(None, q, None, None, cache, meta, output=out)
    torch.cuda.synchronize()
    G.assert_close(out.float().cpu().numpy().reshape(b, hq, hd), ref, "decode of 1100")
    # mixed batch: 1030 sequences decode one token each (ctx > 0),
    # the last one brings a 2-token chunk (its output is not checked here)
    dec = [i for i in range(b) if lens[i] >= 2][:1030]  # ctx = len - 1 > 0: decode rows
    last = b - 1
    while lens[last] < 3:
        last -= 1
    rows = dec + [last]
    qsl = list(range(len(dec) + 1)) + [len(dec) + 2]
    n = qsl[-1]
    qm = torch.zeros((n, hq * hd), dtype=torch.float16, device=dev)
    qm[:len(dec)] = q[dec]
    km = torch.zeros((n, hkv * hd), dtype=torch.float16, device=dev)
    vm = torch.zeros_like(km)
    meta = Meta(2, n, bt[rows], sl[rows], torch.tensor(qsl, dtype=torch.int32, device=dev),
                slots[:n])
    out = torch.zeros((n, hq * hd), dtype=torch.float16, device=dev)
    impl.forward(None, qm, km, vm, cache, meta, output=out)
    torch.cuda.synchronize()
    got = out[:len(dec)].float().cpu().numpy().reshape(len(dec), hq, hd)
    assert len(dec) == 1030
    G.assert_close(got, ref[dec], "mixed decode rows")
    dd.pick_decode_op.cache_clear()
