"""The vLLM-facing backend driven with a stand-in attention-metadata object:
prefill writes the cache through do_kv_cache_update, decode goes through
forward(), and the result matches the oracle."""
from dataclasses import dataclass

import numpy as np
import pytest
import torch

from tests import gpu_cases as G
from tests import workloads as W

pytestmark = pytest.mark.gpu


@dataclass
class Meta:
    max_query_len: int
    num_actual_tokens: int
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    query_start_loc: torch.Tensor
    slot_mapping: torch.Tensor


def test_backend_write_then_decode():
    print("case: backend write+decode", flush=True)
    from turboquant_amd.vllm_backend_fused import TurboQuantBackend, TurboQuantFusedImpl
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
    # the same through the registered reference op name
    assert impl._decode_op_name == "gfx950_hip_paged_splitkv"


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
