"""Prefill attention kernel (tq_prefill_attention) against a float64 reference
of causal GQA attention with the queries aligned to the end of the keys."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def ref_attention(q, k, v, scale):
    """float64 softmax(q k^T * scale) v per head, query i of Lq seeing keys
    j <= Lk - Lq + i; q [Lq, Hq, D], k/v [Lk, Hkv, D]."""
    lq, hq, d = q.shape
    lk, hkv, _ = k.shape
    r = hq // hkv
    qd, kd, vd = q.double(), k.double(), v.double()
    kk = kd.repeat_interleave(r, dim=1)
    vv = vd.repeat_interleave(r, dim=1)
    s = torch.einsum("ihd,jhd->hij", qd, kk) * scale
    i = torch.arange(lq, device=q.device)[:, None]
    j = torch.arange(lk, device=q.device)[None, :]
    s = s.masked_fill(j > (lk - lq) + i, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("hij,jhd->ihd", p, vv)


CASES = [
    # (Lq, Lk, Hq, Hkv)
    (1, 1, 32, 8),
    (17, 17, 32, 8),
    (128, 128, 32, 8),
    (129, 129, 8, 8),
    (200, 1000, 32, 8),
    (1000, 1000, 16, 2),
    (64, 4096, 32, 8),
    (1, 777, 32, 4),
    (300, 300, 32, 32),
    # 256-row workgroups (q heads x 256-row blocks >= the CU count)
    (2085, 3000, 32, 8),
    (2048, 2048, 128, 16),
    # short chunks over long contexts: keys split over workgroups, then merged
    (256, 20000, 32, 8),
    (17, 9000, 8, 2),
]
# head size 64 (the configs[3] geometry: 16 q / 4 kv heads), both shapes
CASES64 = [
    (1, 1, 16, 4),
    (129, 400, 16, 4),
    (1000, 1000, 16, 4),
    (4100, 4500, 16, 4),
    # 256-row blocks of four waves x two row blocks (heads x blocks >= CUs):
    # GQA 8 with a ragged last block, and GQA 1
    (2500, 3001, 32, 4),
    (4097, 4097, 16, 16),
    # short chunk over a long context: keys split over workgroups, then merged
    (256, 8000, 16, 4),
]


# head size 256 (the configs[3] geometry: 16 q / 2 kv heads): one shape, split
# and unsplit
CASES256 = [
    (1, 1, 16, 2),
    (129, 400, 16, 2),
    (1000, 1000, 16, 2),
    (2100, 2500, 16, 2),
    (256, 8000, 16, 2),
    (17, 9000, 8, 2),
]


@pytest.mark.parametrize("lq,lk,hq,hkv,d", [c + (128,) for c in CASES] +
                         [c + (64,) for c in CASES64] + [c + (256,) for c in CASES256])
def test_prefill_matches_float64(lq, lk, hq, hkv, d):
    print(f"case: prefill lq={lq} lk={lk} hq={hq} hkv={hkv} d={d}", flush=True)
    from turboquant_amd import ops
    g = torch.Generator(device=DEV).manual_seed(lq * 7919 + lk + d)
    q = torch.randn((lq, hq, d), generator=g, device=DEV).half()
    k = torch.randn((lk, hkv, d), generator=g, device=DEV).half()
    v = torch.randn((lk, hkv, d), generator=g, device=DEV).half()
    scale = 1.0 / math.sqrt(d)
    o = torch.full((lq, hq, d), float("nan"), dtype=torch.float16, device=DEV)
    ops.prefill_attention(q, k, v, o, scale)
    torch.cuda.synchronize()
    ref = ref_attention(q, k, v, scale)
    err = (o.double() - ref).abs()
    tol = 2e-3 + 1e-2 * ref.abs()
    assert torch.isfinite(o).all()
    assert (err <= tol).all(), f"max err {err.max().item():.3e}"


@pytest.mark.parametrize("lq,lk", [(300, 700), (2100, 2500)])
def test_prefill_strided_rows_and_heavy_tails(lq, lk):
    """Rows of q/k/v/o taken from wider packed tensors (as the backend's
    qkv projection slices them), Student-t keys with a few large scores; a
    128-row and a 256-row workgroup shape."""
    print(f"case: prefill strided rows, t3 keys lq={lq} lk={lk}", flush=True)
    from turboquant_amd import ops
    g = torch.Generator(device=DEV).manual_seed(5)
    hq, hkv, d = 32, 8, 128
    qkv = torch.randn((lk, (hq + 2 * hkv) * d), generator=g, device=DEV).half()
    t = torch.distributions.StudentT(3.0).sample((lk, hkv * d)).to(DEV).half()
    qkv[:, hq * d:(hq + hkv) * d] = t
    q = qkv[lk - lq:, :hq * d].view(lq, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(lk, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(lk, hkv, d)
    big = torch.empty((lq, hq * d * 2), dtype=torch.float16, device=DEV)
    o = big[:, :hq * d].view(lq, hq, d)
    scale = 1.0 / math.sqrt(d)
    ops.prefill_attention(q, k, v, o, scale)
    torch.cuda.synchronize()
    ref = ref_attention(q, k, v, scale)
    err = (o.double() - ref).abs()
    assert (err <= 2e-3 + 1e-2 * ref.abs()).all(), f"max err {err.max().item():.3e}"


def test_prefill_split_plan_and_agreement():
    """The split-KV plan engages for a short chunk over a long context (the
    workspace query is positive) and gives what the unsplit kernel gives
    (tq_prefill_attention without a workspace), within fp16 rounding of the
    merged outputs; both within the float64 tolerance."""
    print("case: prefill split vs unsplit lq=300 lk=16384", flush=True)
    from turboquant_amd import _lib, ops
    lib = _lib.load()
    lq, lk, hq, hkv, d = 300, 16384, 32, 8, 128
    assert lib.tq_prefill_workspace_bytes(lq, lk, hq, hkv, d) > 0
    assert lib.tq_prefill_workspace_bytes(8192, 8192, hq, hkv, d) == 0  # full grid: no split
    g = torch.Generator(device=DEV).manual_seed(21)
    q = torch.randn((lq, hq, d), generator=g, device=DEV).half()
    k = torch.randn((lk, hkv, d), generator=g, device=DEV).half()
    v = torch.randn((lk, hkv, d), generator=g, device=DEV).half()
    split = torch.empty_like(q)
    ops.prefill_attention(q, k, v, split, 0.088)
    whole = torch.empty_like(q)
    rc = lib.tq_prefill_attention(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                                  k.stride(0), k.stride(1), v.data_ptr(), v.stride(0),
                                  v.stride(1), whole.data_ptr(), whole.stride(0), whole.stride(1),
                                  lq, lk, hq, hkv, d, 0.088,
                                  torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "prefill_attention")
    torch.cuda.synchronize()
    assert (split.float() - whole.float()).abs().max().item() <= 2e-3
    ref = ref_attention(q, k, v, 0.088)
    for o in (split, whole):
        assert ((o.double() - ref).abs() <= 2e-3 + 1e-2 * ref.abs()).all()


@pytest.mark.parametrize("lq,lk", [(256, 512), (2048, 2300), (256, 8192)])
def test_prefill_graph_replay_matches_eager(lq, lk):
    print(f"case: prefill graph replay lq={lq} lk={lk}", flush=True)
    from turboquant_amd import ops
    g = torch.Generator(device=DEV).manual_seed(9)
    hq, hkv, d = 32, 8, 128
    q = torch.randn((lq, hq, d), generator=g, device=DEV).half()
    k = torch.randn((lk, hkv, d), generator=g, device=DEV).half()
    v = torch.randn((lk, hkv, d), generator=g, device=DEV).half()
    eager = torch.empty((lq, hq, d), dtype=torch.float16, device=DEV)
    ops.prefill_attention(q, k, v, eager, 0.088)
    o = torch.empty_like(eager)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        ops.prefill_attention(q, k, v, o, 0.088)
    for _ in range(3):
        o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, eager)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_prefill_split_workspace_rows_without_visible_keys(d):
    """Split mode, where a split's tiles can lie wholly beyond a query row's
    last key: such rows must leave a finite workspace entry (O = 0, row sum
    0, max -inf) rather than NaN, and the merged output stays within the
    float64 tolerance.  The workspace is the caller's, so it is read back."""
    print(f"case: prefill split workspace, masked splits d={d}", flush=True)
    from turboquant_amd import _lib
    lib = _lib.load()
    # 2 q heads: 8 query blocks of 128 rows, 65 key tiles split 8 ways (9
    # tiles each); the keys start 3088 = 16 mod 32 before the chunk, so the
    # split starting at key 3456 begins inside the 32 rows of one wave (rows
    # 352..367 see none of its keys, rows 368..383 do)
    lq, lk, hq, hkv = 1024, 4112, 2, 1
    nbytes = int(lib.tq_prefill_workspace_bytes(lq, lk, hq, hkv, d))
    assert nbytes > 0
    g = torch.Generator(device=DEV).manual_seed(31 + d)
    q = torch.randn((lq, hq, d), generator=g, device=DEV).half()
    k = torch.randn((lk, hkv, d), generator=g, device=DEV).half()
    v = torch.randn((lk, hkv, d), generator=g, device=DEV).half()
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=DEV)  # NaN pattern
    o = torch.empty((lq, hq, d), dtype=torch.float16, device=DEV)
    rc = lib.tq_prefill_attention_ws(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                                     k.stride(0), k.stride(1), v.data_ptr(), v.stride(0),
                                     v.stride(1), o.data_ptr(), o.stride(0), o.stride(1),
                                     lq, lk, hq, hkv, d, 0.05, ws.data_ptr(), nbytes,
                                     torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "prefill_attention_ws")
    torch.cuda.synchronize()
    per_split = lq * hq * (2 * d + 8)
    nsplit = nbytes // per_split
    assert nsplit * per_split == nbytes and nsplit >= 2
    wo = ws[:nsplit * lq * hq * d * 2].view(torch.float16).view(nsplit, lq, hq, d)
    ml = ws[nsplit * lq * hq * d * 2:].view(torch.float32).view(nsplit, lq, hq, 2)
    assert torch.isfinite(wo).all()
    masked = ml[..., 0] == float("-inf")
    assert masked.any(), "no split without visible keys: the case does not test it"
    assert (ml[..., 1][masked] == 0).all()
    assert (wo[masked] == 0).all()
    assert torch.isfinite(ml[..., 1]).all()
    ref = ref_attention(q, k, v, 0.05)
    assert ((o.double() - ref).abs() <= 2e-3 + 1e-2 * ref.abs()).all()
