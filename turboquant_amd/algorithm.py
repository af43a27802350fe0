"""TurboQuant vector quantizers (Zandieh et al., arXiv:2504.19874) as a torch
library: the public algorithm API of the reference package
(turboquant/__init__.py:9-22), device-agnostic, for experiments and offline
compression.  The serving path (the paged 4-bit cache) is the HIP kernels in
``turboquant_amd.ops``; this module is the algorithm they specialise.

* ``fwht`` / ``RandomHadamardRotation`` — normalised Walsh-Hadamard transform
  and the sign-randomised rotation (reference turboquant/hadamard.py:20-78).
  The butterflies run in ascending stride, as the reference's, so results
  carry the same fp32 bits.
* ``Codebook`` — Lloyd-Max centroids of N(0, 1) for 1-4 bits, scaled by
  1/sqrt(dim); indices by ``torch.bucketize`` (a value equal to a boundary
  takes the lower bucket), as turboquant/codebook.py:65-103.
* ``QJL`` — 1-bit quantized Johnson-Lindenstrauss transform
  (turboquant/qjl.py:15-56).
* ``TurboQuantMSE`` (Algorithm 1) and ``TurboQuantProd`` (Algorithm 2)
  (turboquant/quantizer.py:63-158), with bit-packing low bits first
  (quantizer.py:17-60).  On a GPU, fp32 vectors of padded size 64..1024 are
  quantized and dequantized by this package's HIP kernels
  (ops.mse_quantize / ops.mse_dequantize, tq_mse.hip); TurboQuantProd's MSE
  stage goes through them too, its QJL stage is a GEMM.

Random tensors (signs, QJL matrix) come from seeded CPU torch generators, so
the same seeds give the reference's values.
"""
from __future__ import annotations

import math

import torch

__all__ = ["TurboQuantMSE", "TurboQuantProd", "RandomHadamardRotation", "Codebook", "QJL",
           "fwht", "next_power_of_2", "pack_bits", "unpack_bits"]

# Lloyd-Max quantizer centroids for N(0, 1) (the reference's table,
# turboquant/codebook.py:16-56); the 4-bit row is the cache codebook.
CENTROIDS_N01 = {
    1: (0.7978845608028654,),
    2: (0.4527800398860679, 1.5104176088887660),
    3: (0.2451209601065855, 0.7560052489261838, 1.3439709227384000, 2.1519775207392190),
    4: (0.1284153814744918, 0.3880823046410021, 0.6567591430551046, 0.9423683558764893,
        1.2562490887894980, 1.6180344937899930, 2.0693470280837980, 2.7326368237440100),
}


def _levels(bit_width: int) -> list[float]:
    pos = list(CENTROIDS_N01[bit_width])
    return [-c for c in reversed(pos)] + pos


def next_power_of_2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


@torch.no_grad()
def fwht_unnormalized(x: torch.Tensor) -> torch.Tensor:
    """y = H x along the last dim (d a power of two, H the Sylvester
    Hadamard matrix of +-1 entries); stride-1 butterflies first, each stage
    (a + b, a - b) on pairs (i, i + h)."""
    d = x.shape[-1]
    if d <= 0 or d & (d - 1):
        raise AssertionError(f"last dim must be a power of 2, got {d}")
    lead = x.shape[:-1]
    y = x.reshape(-1, d)
    h = 1
    while h < d:
        z = y.view(-1, d // (2 * h), 2, h)
        a, b = z[:, :, 0, :], z[:, :, 1, :]
        y = torch.stack((a + b, a - b), dim=2).view(-1, d)
        h *= 2
    return y.view(*lead, d)


def fwht(x: torch.Tensor) -> torch.Tensor:
    """y = H x / sqrt(d) along the last dim (d a power of two)."""
    return fwht_unnormalized(x) * (1.0 / math.sqrt(x.shape[-1]))


def _seeded_signs(n: int, seed: int) -> torch.Tensor:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    s = torch.sign(torch.randn(n, generator=g))
    return torch.where(s == 0, torch.ones_like(s), s)


class RandomHadamardRotation:
    """y = FWHT(s * pad(x)), x = unpad(s * FWHT(y)); s = sign(randn) from a
    CPU generator seeded with `seed` (0 -> +1)."""

    def __init__(self, dim: int, device="cuda", seed: int = 42):
        self.orig_dim = dim
        self.padded_dim = next_power_of_2(dim)
        self.signs = _seeded_signs(self.padded_dim, seed).to(device)

    @torch.no_grad()
    def rotate(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] < self.padded_dim:
            x = torch.nn.functional.pad(x, (0, self.padded_dim - x.shape[-1]))
        return fwht(x * self.signs)

    @torch.no_grad()
    def inverse_rotate(self, y: torch.Tensor) -> torch.Tensor:
        return (fwht(y) * self.signs)[..., :self.orig_dim]


class Codebook:
    """Scalar Lloyd-Max quantizer for the coordinates of a rotated unit vector
    of dimension `dim` (each close to N(0, 1/dim))."""

    def __init__(self, dim: int, bit_width: int, device="cuda"):
        if not 1 <= bit_width <= 4:
            raise AssertionError(f"supported bit widths: 1-4, got {bit_width}")
        self.dim = dim
        self.bit_width = bit_width
        self.num_levels = 1 << bit_width
        self.scale = 1.0 / math.sqrt(dim)
        lv = _levels(bit_width)
        mids = [(lv[i] + lv[i + 1]) / 2.0 for i in range(len(lv) - 1)]
        # products in float64, then one rounding to fp32
        self.centroids = torch.tensor([c * self.scale for c in lv], dtype=torch.float32,
                                      device=device)
        self.boundaries = torch.tensor([m * self.scale for m in mids], dtype=torch.float32,
                                       device=device)

    @torch.no_grad()
    def quantize(self, x: torch.Tensor) -> torch.Tensor:
        return torch.bucketize(x, self.boundaries).to(torch.uint8)

    @torch.no_grad()
    def dequantize(self, indices: torch.Tensor) -> torch.Tensor:
        return self.centroids[indices.long()]


def pack_bits(indices: torch.Tensor, bit_width: int) -> torch.Tensor:
    """Pack b-bit indices 8 // b per byte, index i of a byte at bits
    [i*b, (i+1)*b) (3-bit packs two per byte); the last dim is zero padded
    to a whole byte."""
    per = 8 // bit_width
    d = indices.shape[-1]
    nbytes = -(-d // per)
    if nbytes * per > d:
        indices = torch.nn.functional.pad(indices, (0, nbytes * per - d))
    grp = indices.to(torch.int32).view(*indices.shape[:-1], nbytes, per)
    shifts = torch.arange(per, device=indices.device, dtype=torch.int32) * bit_width
    return (grp << shifts).sum(dim=-1).to(torch.uint8)


def unpack_bits(packed: torch.Tensor, bit_width: int, orig_dim: int) -> torch.Tensor:
    per = 8 // bit_width
    shifts = torch.arange(per, device=packed.device, dtype=torch.int32) * bit_width
    vals = (packed.to(torch.int32).unsqueeze(-1) >> shifts) & ((1 << bit_width) - 1)
    return vals.flatten(-2)[..., :orig_dim].to(torch.uint8)


class QJL:
    """1-bit quantized JL transform: Q(x) = sign(S x), and the unbiased
    inner-product dequantization sqrt(pi/2)/d * gamma * S^T z, S a d x d
    Gaussian matrix from a CPU generator seeded with `seed`."""

    def __init__(self, dim: int, device="cuda", seed: int = 1042):
        self.dim = dim
        self.dequant_scale = math.sqrt(math.pi / 2.0) / dim
        g = torch.Generator(device="cpu")
        g.manual_seed(seed)
        self.S = torch.randn(dim, dim, generator=g).to(device)

    def halves(self, padded_dim: int):
        """(S_hi, S_lo, S^T_hi, S^T_lo): fp16 halves with S = hi + lo (to 22
        bits), zero-padded to [padded_dim, padded_dim], for the fused kernels
        (made once per padded size and device)."""
        cache = self.__dict__.setdefault("_halves", {})
        key = (padded_dim, str(self.S.device))
        if key not in cache:
            out = []
            for m in (self.S, self.S.t()):
                hi = m.half()
                lo = (m - hi.float()).half()
                for h in (hi, lo):
                    pad = torch.zeros((padded_dim, padded_dim), dtype=torch.float16,
                                      device=self.S.device)
                    pad[:self.dim, :self.dim] = h
                    out.append(pad)
            cache[key] = (out[0], out[1], out[2], out[3])
        return cache[key]

    @torch.no_grad()
    def quantize(self, x: torch.Tensor) -> torch.Tensor:
        proj = x.float() @ self.S.t()
        # sign() with 0 -> +1, without an int64 intermediate
        return (proj >= 0).to(torch.int8).mul_(2).sub_(1)

    @torch.no_grad()
    def dequantize_inner_product(self, signs: torch.Tensor,
                                 residual_norm: torch.Tensor) -> torch.Tensor:
        return (signs.float() @ self.S) * (self.dequant_scale * residual_norm.unsqueeze(-1))


class TurboQuantMSE:
    """Algorithm 1: norm, normalise, rotate, scalar-quantize, bit-pack; the
    inverse looks the centroids up, rotates back and rescales."""

    def __init__(self, dim: int, bit_width: int, device="cuda", seed: int = 42):
        self.dim = dim
        self.bit_width = bit_width
        self.device = device
        self.rotation = RandomHadamardRotation(dim, device=device, seed=seed)
        self.codebook = Codebook(self.rotation.padded_dim, bit_width, device=device)

    def _hip(self, t: torch.Tensor) -> bool:
        """The HIP kernels serve fp32 vectors on a GPU with padded size 64..1024
        (tq_mse_quantize / tq_mse_dequantize); anything else runs as torch
        ops on its own device."""
        pd = self.rotation.padded_dim
        return t.is_cuda and 64 <= pd <= 1024 and self.rotation.signs.is_cuda

    def _host_tables(self):
        if getattr(self, "_tables", None) is None:
            self._tables = (self.codebook.boundaries.cpu().tolist(),
                            self.codebook.centroids.cpu().tolist())
        return self._tables

    @torch.no_grad()
    def quantize(self, x: torch.Tensor):
        """x [..., dim] -> (packed uint8 [..., ceil(pd / (8 // b))], norms [...])."""
        if x.dtype == torch.float32 and self._hip(x):
            from . import ops
            return ops.mse_quantize(x, self.rotation.padded_dim, self.bit_width,
                                    self.rotation.signs, self._host_tables()[0])
        norms = torch.linalg.vector_norm(x, dim=-1, keepdim=True).clamp_min(1e-8)
        idx = self.codebook.quantize(self.rotation.rotate(x / norms))
        return pack_bits(idx, self.bit_width), norms.squeeze(-1)

    @torch.no_grad()
    def dequantize(self, packed: torch.Tensor, norms: torch.Tensor) -> torch.Tensor:
        if self._hip(packed) and norms.dtype == torch.float32:
            from . import ops
            return ops.mse_dequantize(packed, norms, self.dim, self.rotation.padded_dim,
                                      self.bit_width, self.rotation.signs,
                                      self._host_tables()[1])
        idx = unpack_bits(packed, self.bit_width, self.rotation.padded_dim)
        return self.rotation.inverse_rotate(self.codebook.dequantize(idx)) * norms.unsqueeze(-1)


class TurboQuantProd:
    """Algorithm 2: TurboQuantMSE at b - 1 bits, then QJL on the unit residual,
    so that inner products are unbiased."""

    def __init__(self, dim: int, bit_width: int, device="cuda", seed: int = 42):
        if bit_width < 2:
            raise AssertionError("the inner-product quantizer needs bit_width >= 2")
        self.dim = dim
        self.bit_width = bit_width
        self.device = device
        self.mse = TurboQuantMSE(dim, bit_width - 1, device=device, seed=seed)
        self.qjl = QJL(dim, device=device, seed=seed + 10000)

    @torch.no_grad()
    def quantize(self, x: torch.Tensor):
        """-> (mse_packed, mse_norms, qjl_signs int8 {-1, +1}, residual_norms).
        fp32 vectors on a GPU take one HIP kernel: up to padded size 128 the
        whole algorithm with the QJL product on the matrix cores
        (tq_prod_quantize_qjl), above it the MSE stage, its read-back and the
        unit residual (tq_prod_quantize) followed by the QJL GEMM."""
        if x.dtype == torch.float32 and self.mse._hip(x):
            from . import ops
            bnd, cen = self.mse._host_tables()
            pd = self.mse.rotation.padded_dim
            if pd <= 128:  # QJL product fused on the matrix cores
                sh, sl, _, _ = self.qjl.halves(pd)
                return ops.prod_quantize_qjl(x, pd, self.mse.bit_width, self.mse.rotation.signs,
                                             bnd, cen, sh, sl)
            packed, norms, ru, rn = ops.prod_quantize(x, self.mse.rotation.padded_dim,
                                                      self.mse.bit_width,
                                                      self.mse.rotation.signs, bnd, cen)
            return packed, norms, self.qjl.quantize(ru), rn
        packed, norms = self.mse.quantize(x)
        r = x - self.mse.dequantize(packed, norms)
        rn = torch.linalg.vector_norm(r, dim=-1).clamp_min(1e-8)
        return packed, norms, self.qjl.quantize(r / rn.unsqueeze(-1)), rn

    @torch.no_grad()
    def dequantize(self, mse_packed, mse_norms, qjl_signs, residual_norms) -> torch.Tensor:
        if self.mse._hip(mse_packed) and mse_norms.dtype == torch.float32:
            from . import ops
            pd = self.mse.rotation.padded_dim
            if pd <= 128 and qjl_signs.dtype == torch.int8:
                _, _, th, tl = self.qjl.halves(pd)
                return ops.prod_dequantize_qjl(mse_packed, mse_norms, qjl_signs, residual_norms,
                                               self.dim, pd, self.mse.bit_width,
                                               self.mse.rotation.signs,
                                               self.mse._host_tables()[1], th, tl)
            return ops.prod_dequantize(mse_packed, mse_norms, qjl_signs.float() @ self.qjl.S,
                                       residual_norms, self.dim, self.mse.rotation.padded_dim,
                                       self.mse.bit_width, self.mse.rotation.signs,
                                       self.mse._host_tables()[1])
        return (self.mse.dequantize(mse_packed, mse_norms)
                + self.qjl.dequantize_inner_product(qjl_signs, residual_norms))
