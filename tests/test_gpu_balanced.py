"""GPU parity of the balanced-plan decode (split plan made on the device from
seq_lens) against the fp64 dequantize-then-attend oracle (max-abs 2e-3 /
rel 1e-2): configs[3] ragged batches at BASELINE's B=64 for head sizes
64/128/256, edge lengths, batches larger than the grid, and graph replays
whose seq_lens change between replays."""
import numpy as np
import pytest
import torch

from tests import gpu_cases as G
from turboquant_amd import workloads as W
from turboquant_amd import ops
from turboquant_amd.geometry import hadamard_signs

pytestmark = pytest.mark.gpu


def _check_plan(split, lens, rows_max):
    """The row table: rows of sequence b are r * ceil(L_b / U) consecutive
    rows (r = 1, or 2 when the units are block pairs), U a multiple of 32."""
    b = len(lens)
    u = int(split[b + 1])
    assert u > 0 and u % 32 == 0, u
    assert split[0] == 0 and split[b] <= rows_max
    d = np.diff(split[:b + 1]).astype(np.int64)
    n = -(-np.maximum(np.asarray(lens, np.int64), 0) // u)
    assert any(np.array_equal(d, r * n) for r in (1, 2)), (d[:8], n[:8], u)
    return u


def _check(case, cache, pd, what):
    b, hq = case["q"].shape[:2]
    rows = ops.balanced_rows(b, hq, case["num_kv_heads"], pd)
    got, qp, scale, split = G.run_balanced(case, cache, pd, rows=rows)
    _check_plan(split, case["seq_lens"], rows)
    ref = G.oracle_decode(case, cache.cpu().numpy(), qp, pd, scale)
    G.assert_close(got, ref, what)
    return got, ref


@pytest.mark.parametrize("hd", [128, 64, 256])
def test_cfg4_ragged_b64(hd):
    """B=64, L ~ U[1024, 32768] (seed 4), K Student-t(3), V N(0,1)."""
    hq, hkv = {64: (16, 4), 128: (32, 8), 256: (16, 2)}[hd]
    lens = np.random.default_rng(4).integers(1024, 32768 + 1, size=64)
    print(f"case: balanced cfg4 hd={hd} B=64 {hq}/{hkv} tokens={int(lens.sum())}", flush=True)
    case, cache, pd = G.device_case(4 + 1000 * hd, lens, hq, hkv, hd, k_dist="t3")
    _check(case, cache, pd, f"balanced cfg4 hd{hd}")


def test_cfg3_uniform_matches_static_layout():
    """Equal lengths: the plan is the static layout (8 x 32768 at 512 units
    of 512 tokens) and the output matches the oracle."""
    print("case: balanced cfg3 B=8 L=32768", flush=True)
    case, cache, pd = G.device_case(3, [32768] * 8, 32, 8, 128)
    _check(case, cache, pd, "balanced cfg3")


@pytest.mark.parametrize("b,length", [(3, 1000), (64, 4096), (5, 1), (17, 33)])
def test_uniform_lengths_closed_form_plan(b, length):
    """Equal lengths take the plan's closed form (no search): the row table
    is b equal blocks, the unit size the smallest that fits, and the output
    matches the oracle."""
    print(f"case: balanced uniform B={b} L={length}", flush=True)
    c = W.decode_case(97 + b, b, [length] * b, 32, 8, 128)
    cache, pd = G.build_cache(c)
    _, _ = _check(c, cache, pd, f"balanced uniform B={b} L={length}")
    _, _, _, split = G.run_balanced(c, cache, pd)
    d = np.diff(split[:b + 1])
    assert np.all(d == d[0]) and d[0] > 0, split[:b + 1]
    u = int(split[b + 1])
    # rows per sequence = rowmul * ceil(L / U); a smaller U (by 32) would need more
    # units per sequence than U does
    assert u >= 32 and u % 32 == 0 and (u == 32 or -(-length // (u - 32)) > -(-length // u)), u


@pytest.mark.parametrize("hq,hkv,hd", [(32, 8, 128), (16, 2, 128), (16, 16, 64), (16, 4, 256),
                                       (16, 1, 128), (16, 2, 256), (12, 2, 256)])
def test_edge_lengths(hq, hkv, hd):
    """Lengths 0, 1, 15, 16, 17, 31, 32, 33 beside long ones, GQA 1..16."""
    lens = [0, 1, 15, 16, 17, 31, 32, 33, 5000, 0, 777]
    print(f"case: balanced edges {hq}/{hkv}/{hd}", flush=True)
    c = W.decode_case(71 + hq + hd, len(lens), lens, hq, hkv, hd)
    cache, pd = G.build_cache(c)
    got, _ = _check(c, cache, pd, f"balanced edges {hq}/{hkv}/{hd}")
    assert np.all(got[0] == 0) and np.all(got[9] == 0)  # empty sequences -> zeros


def test_all_empty_batch():
    print("case: balanced all-empty batch", flush=True)
    c = W.decode_case(81, 3, [0, 0, 0], 32, 8, 128)
    cache, pd = G.build_cache(c)
    got, _, _, split = G.run_balanced(c, cache, pd)
    assert np.all(got == 0) and np.all(split[:4] == 0)


def test_batch_larger_than_grid():
    """More sequences than resident workgroup slots: one unit per sequence
    at least, several rounds of workgroups."""
    rng = np.random.default_rng(91)
    lens = rng.integers(1, 200, size=700)
    print(f"case: balanced B=700 tokens={int(lens.sum())}", flush=True)
    c = W.decode_case(91, len(lens), lens, 32, 8, 128)
    cache, pd = G.build_cache(c)
    _check(c, cache, pd, "balanced B=700")


def test_small_workspace_is_refused_or_used():
    """A workspace with fewer rows than the batch is refused; one with just
    the batch's rows gives the same result as the full one."""
    print("case: balanced small workspace", flush=True)
    c = W.decode_case(93, 5, [3000, 10, 700, 0, 64], 32, 8, 128)
    cache, pd = G.build_cache(c)
    with pytest.raises(RuntimeError, match="fewer than the batch"):
        G.run_balanced(c, cache, pd, rows=4)
    got, qp, scale, split = G.run_balanced(c, cache, pd, rows=5)
    _check_plan(split, c["seq_lens"], 5)
    ref = G.oracle_decode(c, cache.cpu().numpy(), qp, pd, scale)
    G.assert_close(got, ref, "balanced rows=5")


def test_graph_replay_with_changing_seq_lens():
    """One captured graph replayed with different seq_lens each time (the
    plan is remade on the device): every replay equals the eager call with
    the same lengths, and the oracle."""
    print("case: balanced graph replay, changing seq_lens", flush=True)
    full = [3000, 1500, 64, 2000]
    c = W.decode_case(95, 4, full, 32, 8, 128)
    cache, pd = G.build_cache(c)
    d = G.decode_inputs(c, pd)
    rows = ops.balanced_rows(4, 32, 8, pd)
    dev = G.DEV
    o = torch.empty((4, 32, pd), dtype=torch.float16, device=dev)
    po = torch.empty((rows, 32, pd), dtype=torch.float32, device=dev)
    pl = torch.empty((rows, 32), dtype=torch.float32, device=dev)
    split = torch.zeros(6, dtype=torch.int32, device=dev)
    s = hadamard_signs(pd, dev)
    scale = 1.0 / np.sqrt(128)
    seq = d["seq"].clone()

    def call():
        ops.decode_paged_balanced(d["q"], cache, d["indices"], d["indptr"], seq, 8, 128, pd,
                                  scale, s, o, po, pl, split)

    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        call()
    for i, lens in enumerate(([3000, 1500, 64, 2000], [17, 2999, 0, 1024], [1, 1, 1, 1],
                              [3000, 1500, 64, 2000])):
        seq.copy_(torch.tensor(lens, dtype=torch.int32))
        torch.cuda.synchronize()
        call()
        torch.cuda.synchronize()
        eager = o.float().cpu().numpy().copy()
        o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = o.float().cpu().numpy()
        assert np.array_equal(got, eager), f"replay {i}"
        c2 = dict(c)
        c2["seq_lens"] = np.array(lens, np.int32)
        ref = G.oracle_decode(c2, cache.cpu().numpy(), d["qp"], pd, scale)
        G.assert_close(got, ref, f"replay {i} vs oracle")


def test_sequence_longer_than_2_pow_24_tokens():
    """A sequence of 2^24 + 777 tokens beside a short one (1 kv head, head
    size 64): the plan's unit counts take the integer division past 2^24
    tokens (a float estimate alone could be off by more than one there), the
    row table covers every token, and the output matches the oracle."""
    lens = [(1 << 24) + 777, 3000]
    print(f"case: balanced B=2 lens={lens} 4/1/64", flush=True)
    case, cache, pd = G.device_case(61, lens, 4, 1, 64, chunk_tokens=1 << 20)
    _check(case, cache, pd, "balanced 2^24+ tokens")
