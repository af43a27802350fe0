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
