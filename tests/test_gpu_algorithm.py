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
