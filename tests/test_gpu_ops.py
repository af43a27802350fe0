"""The reference's other decode op names (decode_v5_tc_binding.cu:948-994) on
the same kernels: the graph-safe non-split op decode_v5_from_cache_ws, the
gather-then-split op decode_v5_from_cache_splitkv_ws and the eager
decode_v5_from_cache, checked against the oracle and, under HIP-graph capture,
against their own eager result on every replay (tests/test_v5_graph.py:115-226
in the reference)."""
import numpy as np
import pytest
import torch

from tests import gpu_cases as G
from turboquant_amd import workloads as W
from turboquant_amd import ops
from turboquant_amd.geometry import hadamard_signs

pytestmark = pytest.mark.gpu


def _inputs(lens, hq=32, hkv=8, hd=128, seed=91):
    c = W.decode_case(seed, len(lens), lens, hq, hkv, hd)
    cache, pd = G.build_cache(c)
    b = len(lens)
    bt = torch.from_numpy(c["block_table"]).to(G.DEV)
    max_len = bt.shape[1] * W.BLOCK
    qp = np.zeros((b, hq, pd), np.float16)
    qp[:, :, :hd] = c["q"]
    d = dict(
        case=c, cache=cache, pd=pd, hd=hd, hkv=hkv, max_len=max_len, qp=qp,
        q=torch.from_numpy(qp).to(G.DEV),
        indices=bt.reshape(-1).contiguous(),
        indptr=(torch.arange(b + 1, dtype=torch.int32, device=G.DEV) * bt.shape[1]),
        last=torch.zeros(b, dtype=torch.int32, device=G.DEV),
        seq=torch.tensor(lens, dtype=torch.int32, device=G.DEV),
        signs=hadamard_signs(pd, G.DEV), scale=1.0 / np.sqrt(hd))
    qb, dc = pd // 2, pd // 64
    d["ws"] = dict(
        k_quant=torch.empty((b, hkv, max_len, qb), dtype=torch.uint8, device=G.DEV),
        v_quant=torch.empty((b, hkv, max_len, qb), dtype=torch.uint8, device=G.DEV),
        k_norms=torch.empty((b, hkv, max_len, dc), dtype=torch.float16, device=G.DEV),
        v_norms=torch.empty((b, hkv, max_len, dc), dtype=torch.float16, device=G.DEV),
        o=torch.empty((b, hq, pd), dtype=torch.float16, device=G.DEV))
    return d


def _ws_call(d):
    w = d["ws"]
    pd = d["pd"]
    return torch.ops.turboquant_v5.decode_v5_from_cache_ws(
        d["q"], d["cache"], d["indices"], d["indptr"], d["last"], d["seq"], d["hkv"], W.BLOCK,
        d["hd"], pd, float(d["scale"]), d["signs"], pd // 2, 2 * (pd // 64), w["k_quant"],
        w["v_quant"], w["k_norms"], w["v_norms"], w["o"], d["max_len"])


def _oracle(d):
    return G.oracle_decode(d["case"], d["cache"].cpu().numpy(), d["qp"], d["pd"], d["scale"])


@pytest.mark.parametrize("lens,hq,hkv,hd", [([64, 17, 1], 32, 8, 128),
                                            ([1024, 300], 32, 8, 128),
                                            ([4096, 2000, 33], 16, 4, 64),
                                            ([700], 16, 2, 256)])
def test_from_cache_ws_matches_oracle(lens, hq, hkv, hd):
    print(f"case: from_cache_ws lens={lens} {hq}/{hkv}/{hd}", flush=True)
    ops.register_ops()
    d = _inputs(lens, hq, hkv, hd)
    out = _ws_call(d)
    torch.cuda.synchronize()
    assert out.data_ptr() == d["ws"]["o"].data_ptr()
    G.assert_close(out.float().cpu().numpy(), _oracle(d), "from_cache_ws")


@pytest.mark.parametrize("seq_len", [64, 256, 1024])
def test_from_cache_ws_graph_replays_match_eager(seq_len):
    print(f"case: from_cache_ws graph seq_len={seq_len}", flush=True)
    ops.register_ops()
    d = _inputs([seq_len, seq_len // 2 + 1])
    ref = _ws_call(d).clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            _ws_call(d)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _ws_call(d)
    for i in range(5):
        d["ws"]["o"].zero_()
        d["ws"]["k_quant"].fill_(0x5A)  # the partials scratch starts dirty on every replay
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(d["ws"]["o"], ref), f"replay {i}"


def test_from_cache_splitkv_ws_equals_paged_op():
    print("case: from_cache_splitkv_ws", flush=True)
    ops.register_ops()
    d = _inputs([2048, 999, 16])
    b, hq, pd = d["q"].shape
    S = 8
    po = torch.empty((b * S, hq, pd), dtype=torch.float32, device=G.DEV)
    pl = torch.empty((b * S, hq), dtype=torch.float32, device=G.DEV)
    ar = torch.arange(b * S, dtype=torch.int32, device=G.DEV)
    extra = (po, pl, ar // S, ar % S, torch.arange(b + 1, dtype=torch.int32, device=G.DEV) * S,
             torch.tensor([-(-d["max_len"] // S)], dtype=torch.int32, device=G.DEV), S)
    w = d["ws"]
    common = (d["q"], d["cache"], d["indices"], d["indptr"], d["last"], d["seq"], d["hkv"],
              W.BLOCK, d["hd"], pd, float(d["scale"]), d["signs"], pd // 2, 2 * (pd // 64))
    o1 = torch.ops.turboquant_v5.decode_v5_from_cache_splitkv_ws(
        *common, w["k_quant"], w["v_quant"], w["k_norms"], w["v_norms"], w["o"],
        d["max_len"], *extra).clone()
    o2 = torch.empty_like(o1)
    torch.ops.turboquant_v5.decode_v5_from_cache_paged_splitkv_ws(
        *common, o2, d["max_len"], *extra)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    G.assert_close(o1.float().cpu().numpy(), _oracle(d), "splitkv_ws")


def test_from_cache_eager_matches_oracle():
    print("case: decode_v5_from_cache eager", flush=True)
    d = _inputs([1500, 3])
    pd = d["pd"]
    o = ops.decode_v5_from_cache(d["q"], d["cache"], d["indices"], d["indptr"], d["last"],
                                 d["seq"], d["hkv"], W.BLOCK, d["hd"], pd, float(d["scale"]),
                                 d["signs"], pd // 2, 2 * (pd // 64))
    torch.cuda.synchronize()
    G.assert_close(o.float().cpu().numpy(), _oracle(d), "from_cache eager")


def test_from_cache_ws_rejects_wrong_workspace():
    ops.register_ops()
    d = _inputs([100])
    d["ws"]["k_quant"] = d["ws"]["k_quant"][:, :, :-1]
    with pytest.raises(RuntimeError, match="k_quant_ws shape mismatch"):
        _ws_call(d)


def test_from_cache_eager_csr_indptr_longer_later_sequence():
    """A CSR page table (indices = each sequence's pages back to back) whose
    later sequence has more pages than the first: the eager op sizes its
    splits from seq_lens.max() (reference decode_v5_tc_binding.cu:350), so
    the longer sequence is read in full."""
    print("case: decode_v5_from_cache eager, CSR indptr", flush=True)
    import oracle
    lens = [100, 3000, 17]
    c = W.decode_case(93, 3, lens, 32, 8, 128)
    cache, pd = G.build_cache(c)
    bt = c["block_table"]
    npg = [-(-n // W.BLOCK) for n in lens]
    ind = np.concatenate([bt[i, :npg[i]] for i in range(3)]).astype(np.int32)
    ip = np.concatenate([[0], np.cumsum(npg)]).astype(np.int32)
    qp = np.zeros((3, 32, pd), np.float16)
    qp[:, :, :128] = c["q"]
    dev = G.DEV
    seq = torch.tensor(lens, dtype=torch.int32, device=dev)
    o = ops.decode_v5_from_cache(torch.from_numpy(qp).to(dev), cache,
                                 torch.from_numpy(ind).to(dev), torch.from_numpy(ip).to(dev),
                                 seq, seq, 8, W.BLOCK, 128, pd, 1.0 / np.sqrt(128),
                                 hadamard_signs(pd, dev), pd // 2, 2 * (pd // 64))
    torch.cuda.synchronize()
    ref = oracle.decode(qp, cache.cpu().numpy(), ind, ip, np.array(lens, np.int32), 8, pd,
                        1.0 / np.sqrt(128), hadamard_signs(pd).numpy())
    G.assert_close(o.float().cpu().numpy(), ref, "from_cache eager CSR")
