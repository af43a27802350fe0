"""The algorithm library on the GPU: the same quantizers on cuda:0 agree with
their CPU results (codes and reconstructions), and the reference's bounds
hold there too."""
import math

import pytest
import torch

from turboquant_amd import algorithm as A

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_mse_gpu_matches_cpu(bits):
    print(f"case: algorithm MSE {bits} bits on cuda", flush=True)
    x = torch.randn(300, 128, generator=torch.Generator().manual_seed(bits))
    qc = A.TurboQuantMSE(128, bits, device="cpu")
    qg = A.TurboQuantMSE(128, bits, device="cuda:0")
    pc, nc = qc.quantize(x)
    pg, ng = qg.quantize(x.cuda())
    agree = (A.unpack_bits(pg.cpu(), bits, 128) == A.unpack_bits(pc, bits, 128)).float().mean()
    assert agree > 0.9999  # reduction order of the norm may move a boundary case
    assert torch.allclose(ng.cpu(), nc, rtol=1e-6)
    xg = qg.dequantize(pg, ng)
    mse = ((x.cuda() - xg).pow(2).sum(-1) / x.cuda().pow(2).sum(-1)).mean().item()
    assert mse <= math.sqrt(3) * math.pi / 2 * 4.0 ** (-bits)


def test_prod_gpu_inner_products():
    print("case: algorithm Prod on cuda", flush=True)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(64, 128, generator=g)
    y = torch.randn(64, 128, generator=g)
    q = A.TurboQuantProd(128, 3, device="cuda:0", seed=5)
    xh = q.dequantize(*q.quantize(x.cuda()))
    est = (xh * y.cuda()).sum(-1).cpu()
    true = (x * y).sum(-1)
    # unbiased with variance O(|x|^2 |y|^2 / d): the mean error over 64 pairs is small
    assert abs((est - true).mean().item()) < 0.15 * true.abs().mean().item() + 0.5


CASES = [(64, 4), (96, 4), (128, 1), (128, 2), (128, 3), (128, 4), (200, 3), (256, 4),
         (256, 2), (1024, 4), (1000, 1)]


@pytest.mark.parametrize("dim,bits", CASES)
def test_mse_hip_kernels_against_the_torch_path(dim, bits):
    """The HIP quantize / dequantize (tq_mse_quantize / tq_mse_dequantize)
    against the same quantizer's torch ops on the CPU: codes agree but for
    coordinates the norm's summation order moves across a boundary, norms
    within 1e-6; dequantization of the same packed codes and norms is the
    same fp32 arithmetic in the same order, so bit-identical; the
    reference's MSE bound holds (quantizer distortion <= sqrt(3) pi / 2 4^-b,
    arXiv:2504.19874 Theorem 1)."""
    print(f"case: algorithm MSE HIP dim={dim} bits={bits}", flush=True)
    from turboquant_amd import ops
    g = torch.Generator().manual_seed(dim * 10 + bits)
    x = torch.randn(2000, dim, generator=g) * 3.0
    x[5] = 0.0  # the 1e-8 norm clamp
    qc = A.TurboQuantMSE(dim, bits, device="cpu")
    qg = A.TurboQuantMSE(dim, bits, device="cuda:0")
    assert qg._hip(x.cuda())
    pd = qg.rotation.padded_dim
    pg, ng = qg.quantize(x.cuda())
    pc, nc = qc.quantize(x)
    assert pg.shape == pc.shape and pg.dtype == torch.uint8 and ng.dtype == torch.float32
    cg = A.unpack_bits(pg.cpu(), bits, pd)
    cc = A.unpack_bits(pc, bits, pd)
    agree = (cg == cc).float().mean().item()
    print(f"  code agreement with the torch path {agree:.7f}", flush=True)
    assert agree >= 0.9999
    assert torch.allclose(ng.cpu(), nc, rtol=1e-6, atol=0)
    # the same codes and norms back through both paths: identical bits
    xg = qg.dequantize(pc.cuda(), nc.cuda()).cpu()
    xc = qc.dequantize(pc, nc)
    assert xg.shape == (2000, dim)
    assert torch.equal(xg, xc), (xg - xc).abs().max().item()
    # the reference's bound on the GPU's own round trip
    xr = qg.dequantize(pg, ng)
    xx = x.cuda()
    keep = xx.pow(2).sum(-1) > 0
    mse = ((xx - xr).pow(2).sum(-1)[keep] / xx.pow(2).sum(-1)[keep]).mean().item()
    assert mse <= math.sqrt(3) * math.pi / 2 * 4.0 ** (-bits)
    assert ops is not None


def test_mse_hip_nonfinite_rows_and_empty_batch():
    """A NaN row: norm NaN, every code the top index (torch.bucketize of
    NaN), as on the torch path; an empty batch returns empty tensors."""
    print("case: algorithm MSE HIP non-finite and empty", flush=True)
    x = torch.randn(8, 128)
    x[3, 7] = float("nan")
    qc = A.TurboQuantMSE(128, 4, device="cpu")
    qg = A.TurboQuantMSE(128, 4, device="cuda:0")
    pg, ng = qg.quantize(x.cuda())
    pc, nc = qc.quantize(x)
    assert torch.isnan(ng[3]).item() and torch.isnan(nc[3]).item()
    assert torch.equal(pg[3].cpu(), pc[3])
    pe, ne = qg.quantize(torch.empty(0, 128, device="cuda:0"))
    assert pe.shape == (0, 64) and ne.shape == (0,)
    assert qg.dequantize(pe, ne).shape == (0, 128)


PROD_CASES = [(64, 2), (64, 5), (96, 3), (97, 3), (100, 4), (128, 2), (128, 3), (128, 4), (128, 5),
              (200, 4), (256, 3), (1000, 2)]


@pytest.mark.parametrize("dim,bits", PROD_CASES)
def test_prod_hip_kernels_against_the_torch_path(dim, bits):
    """TurboQuantProd through tq_prod_quantize / tq_prod_dequantize against
    the same quantizer's torch ops.  Codes and norms as the MSE test; the
    kernel's residual norm and unit residual against torch's x - x_hat, norm
    and division on the kernel's own codes (the read-back is bit-identical,
    only the norm's summation order differs); QJL signs against the CPU path
    where the codes agree; the dequantize epilogue against torch's
    x_mse + (z S) * (sqrt(pi/2) / d * gamma) on the same GEMM output, bit
    for bit."""
    print(f"case: algorithm Prod HIP dim={dim} bits={bits}", flush=True)
    from turboquant_amd import ops
    g = torch.Generator().manual_seed(dim * 7 + bits)
    x = torch.randn(1500, dim, generator=g) * 2.0
    x[9] = 0.0
    qc = A.TurboQuantProd(dim, bits, device="cpu", seed=11)
    qg = A.TurboQuantProd(dim, bits, device="cuda:0", seed=11)
    pd = qg.mse.rotation.padded_dim
    xg = x.cuda()
    bnd, cen = qg.mse._host_tables()
    pk, nm, ru, rn = ops.prod_quantize(xg, pd, bits - 1, qg.mse.rotation.signs, bnd, cen)
    pm, nmm = qg.mse.quantize(xg)
    assert torch.equal(pk, pm) and torch.equal(nm, nmm)  # the MSE kernel's outputs
    r = xg - qg.mse.dequantize(pk, nm)
    rn_t = torch.linalg.vector_norm(r, dim=-1).clamp_min(1e-8)
    assert torch.allclose(rn, rn_t, rtol=2e-6, atol=0), (rn - rn_t).abs().max().item()
    ru_t = r / rn_t.unsqueeze(-1)
    err = (ru - ru_t).abs().max().item()
    print(f"  unit residual max |diff| {err:.3e}", flush=True)
    assert err <= 2e-6
    # unit length, but for x = 0, whose residual (the centroids read back at the
    # clamped norm 1e-8) is shorter than the 1e-8 clamp of its own norm
    lens = ru.norm(dim=-1)
    lens[9] = 1.0
    assert rn[9].item() == 1e-8 or abs(rn[9].item() - 1e-8) < 1e-15
    assert torch.allclose(lens, torch.ones_like(rn), atol=1e-5)
    # the public API against the CPU path (fused QJL product up to pd 128)
    pg, ng, zg, rg = qg.quantize(xg)
    assert torch.equal(pg, pk) and torch.equal(ng, nm) and torch.equal(rg, rn)
    pc, nc, zc, rc = qc.quantize(x)
    cg = A.unpack_bits(pg.cpu(), bits - 1, pd)
    cc = A.unpack_bits(pc, bits - 1, pd)
    same = (cg == cc).all(-1)
    assert same.float().mean().item() >= 0.99
    assert zg.dtype == torch.int8 and set(zg.unique().tolist()) <= {-1, 1}
    # signs against an fp32 GEMM of the kernel's own unit residual: any
    # difference sits where that product is within rounding of 0
    proj = ru @ qg.qjl.S.t()
    want_z = torch.where(proj >= 0, 1, -1).to(torch.int8)
    diff = zg != want_z
    print(f"  QJL signs differing from the fp32 GEMM: {int(diff.sum())} of {diff.numel()}, "
          f"max |proj| there {proj[diff].abs().max().item() if diff.any() else 0:.2e}",
          flush=True)
    assert diff.float().mean().item() <= 1e-4
    if diff.any():
        assert proj[diff].abs().max().item() < 1e-4
    sign_agree = (zg.cpu()[same] == zc[same]).float().mean().item()
    print(f"  QJL sign agreement with the CPU path {sign_agree:.6f} on {int(same.sum())} rows",
          flush=True)
    assert sign_agree >= 0.999
    assert torch.allclose(rg.cpu()[same], rc[same], rtol=1e-5, atol=0)
    # dequantize: the BLAS-path epilogue equals torch's expression on the same
    # GEMM bit for bit; the fused path forms z S itself (fp16 halves of S, fp32
    # accumulation), within 1e-5 of it
    term = zg.float() @ qg.qjl.S
    want = qg.mse.dequantize(pg, ng) + term * (qg.qjl.dequant_scale * rg.unsqueeze(-1))
    got = ops.prod_dequantize(pg, ng, term, rg, dim, pd, bits - 1, qg.mse.rotation.signs, cen)
    assert torch.equal(got, want), (got - want).abs().max().item()
    xh = qg.dequantize(pg, ng, zg, rg)
    if pd <= 128:
        _, _, th, tl = qg.qjl.halves(pd)
        fused = ops.prod_dequantize_qjl(pg, ng, zg, rg, dim, pd, bits - 1,
                                        qg.mse.rotation.signs, cen, th, tl)
        assert torch.equal(xh, fused)
        # the signs at an odd address (a view one byte into a buffer): the op
        # copies them to an aligned tensor, same result
        buf = torch.empty(zg.numel() + 1, dtype=torch.int8, device=zg.device)
        zodd = buf[1:].view(zg.shape)
        zodd.copy_(zg)
        assert zodd.data_ptr() % 8 != 0
        assert torch.equal(xh, ops.prod_dequantize_qjl(pg, ng, zodd, rg, dim, pd, bits - 1,
                                                       qg.mse.rotation.signs, cen, th, tl))
        err = (xh - want).abs().max().item()
        print(f"  fused dequantize max |diff| from the fp32 GEMM expression {err:.2e}", flush=True)
        assert torch.allclose(xh, want, rtol=1e-5, atol=1e-5 * want.abs().max().item())
    else:
        assert torch.equal(xh, want)
    # and against the CPU dequantize of the CPU's own outputs, within GEMM rounding
    xc = qc.dequantize(pc, nc, zc, rc)
    ok = same & (zg.cpu() == zc).all(-1)
    assert torch.allclose(xh.cpu()[ok], xc[ok], rtol=1e-4, atol=1e-4)


def test_prod_hip_unbiased_inner_products():
    """The reference's unbiasedness check (tests/test_algorithm.py:120-138):
    over many random pairs the mean error of <x_hat, y> is near 0 and far
    below the MSE-only estimator's bias, on the HIP path."""
    print("case: algorithm Prod HIP unbiasedness", flush=True)
    g = torch.Generator().manual_seed(3)
    d = 128
    x = torch.randn(4000, d, generator=g)
    x = x / x.norm(dim=-1, keepdim=True)
    y = torch.randn(4000, d, generator=g)
    y = y / y.norm(dim=-1, keepdim=True)
    q = A.TurboQuantProd(d, 2, device="cuda:0")
    xh = q.dequantize(*q.quantize(x.cuda())).cpu()
    err = ((xh * y).sum(-1) - (x * y).sum(-1))
    # |mean| within 4 standard errors; the variance bound is pi / (2 d) per pair
    se = math.sqrt(math.pi / (2 * d) / x.shape[0])
    assert abs(err.mean().item()) < 4 * se + 1e-3


@pytest.mark.parametrize("pd,bits", [(64, 1), (64, 4), (128, 2), (128, 3), (128, 4), (256, 4),
                                     (1024, 3)])
def test_bin_table_codes_equal_the_search(pd, bits):
    """The quantize kernels' one-lookup bucketize (bin table of the symmetric
    codebook) against their binary search on the same inputs: identical
    codes, norms and residuals.  The inputs put many rotated coordinates
    within a few ulps of a boundary, exactly on 0, and at +-inf / NaN rows."""
    print(f"case: algorithm bin-table bucketize pd={pd} bits={bits}", flush=True)
    from turboquant_amd import _lib, ops
    lib = _lib.load()
    q = A.TurboQuantMSE(pd, bits, device="cuda:0")
    s = q.rotation.signs.double().cpu()
    b = q.codebook.boundaries.double().cpu()
    g = torch.Generator().manual_seed(pd + bits)
    n = 3000
    # rotated targets near the boundaries (and exact zeros), mapped back to
    # x = s * FWHT(y) / sqrt(pd) in float64, so the kernel's y lands within
    # rounding of them
    pick = torch.randint(0, len(b), (n, pd), generator=g)
    y = b[pick] * (1 + 1e-7 * torch.randn(n, pd, generator=g, dtype=torch.float64))
    y[torch.rand(n, pd, generator=g) < 0.05] = 0.0
    h = y.clone()
    step = 1
    while step < pd:  # unnormalised FWHT
        h = h.view(n, -1, 2, step)
        h = torch.stack((h[:, :, 0] + h[:, :, 1], h[:, :, 0] - h[:, :, 1]), dim=2)
        step *= 2
    x = (h.reshape(n, pd) * s / math.sqrt(pd)).float()
    x[0] = 0.0
    x[1, 3] = float("inf")
    x[2, 5] = float("nan")
    xg = x.cuda()
    bnd, cen = q._host_tables()
    try:
        pb, nb = ops.mse_quantize(xg, pd, bits, q.rotation.signs, bnd)
        lib.tq_diag_mse_bucketize(1)
        ps, ns = ops.mse_quantize(xg, pd, bits, q.rotation.signs, bnd)
    finally:
        lib.tq_diag_mse_bucketize(0)
    assert torch.equal(nb.isnan(), ns.isnan())
    assert torch.equal(nb[~nb.isnan()], ns[~ns.isnan()])
    diff = (A.unpack_bits(pb.cpu(), bits, pd) != A.unpack_bits(ps.cpu(), bits, pd)).sum().item()
    print(f"  codes differing: {diff}", flush=True)
    assert torch.equal(pb, ps)
    if bits >= 2 and pd <= 128:  # the fused Prod kernel's MSE stage the same way
        pq = A.TurboQuantProd(pd, bits + 1, device="cuda:0")
        bq, cq = pq.mse._host_tables()
        sh, sl, _, _ = pq.qjl.halves(pd)
        try:
            r1 = ops.prod_quantize_qjl(xg, pd, bits, pq.mse.rotation.signs, bq, cq, sh, sl)
            lib.tq_diag_mse_bucketize(1)
            r2 = ops.prod_quantize_qjl(xg, pd, bits, pq.mse.rotation.signs, bq, cq, sh, sl)
        finally:
            lib.tq_diag_mse_bucketize(0)
        assert torch.equal(r1[0], r2[0])
        assert torch.equal(r1[2], r2[2])
