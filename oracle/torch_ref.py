"""Vectorised torch-CPU restatement of the reference's PyTorch path, fp32.

TEST INFRASTRUCTURE ONLY (the CPU baseline of bench.py and a cross-check in
tests/): the product never imports it.  It is what a user of the reference
without a GPU kernel runs: the write as whole-tensor torch ops in the order of
quantize_write_kernel.cuh:332-431 (norm, normalise, sign flip, butterflies
h = 1, 2, 4, ..., scale, bucketize with ties going up, high-nibble pack,
fp16 norm copies), and the decode as turboquant/triton_decode_ref.py:89-131,
264-299 computes it: dequantize c[code] * norm / sqrt(pd) in the rotated
domain, rotate q, GQA softmax attention per (sequence, kv head), inverse
rotation of the output.  Chunked per (sequence, kv head) so a 32k-token
sequence dequantizes ~17 MB at a time.

Differences from the C oracle (oracle/tq_oracle.c): the sum of squares is
torch's reduction (not the reference's lane tree) and the decode accumulates
in fp32, so codes may differ within a few ulp of a boundary and outputs by
fp32 rounding; tests/test_oracle.py bounds both.
"""
from __future__ import annotations

import math

import torch

CODEBOOK = torch.tensor([
    -2.7326368, -2.0693470, -1.6180345, -1.2562491, -0.9423684, -0.6567591, -0.3880823,
    -0.1284154, 0.1284154, 0.3880823, 0.6567591, 0.9423684, 1.2562491, 1.6180345, 2.0693470,
    2.7326368], dtype=torch.float32)
BOUNDARIES = torch.tensor([
    -2.4009919259139040, -1.8436907609368955, -1.4371417912897455, -1.0993087223329937,
    -0.7995637494657970, -0.5224207238480534, -0.2582488430577470, 0.0, 0.2582488430577470,
    0.5224207238480534, 0.7995637494657970, 1.0993087223329937, 1.4371417912897455,
    1.8436907609368955, 2.4009919259139040], dtype=torch.float32)


def fwht(x: torch.Tensor) -> torch.Tensor:
    """Unnormalised butterflies (a + b, a - b), h = 1, 2, 4, ... on the last dim."""
    n = x.shape[-1]
    lead = x.shape[:-1]
    h = 1
    while h < n:
        y = x.reshape(*lead, n // (2 * h), 2, h)
        a, b = y[..., 0, :], y[..., 1, :]
        x = torch.stack((a + b, a - b), dim=-2).reshape(*lead, n)
        h *= 2
    return x


def quantize(x: torch.Tensor, pd: int, signs: torch.Tensor) -> torch.Tensor:
    """Rows x [..., head_dim] (any float) -> entry bytes uint8 [..., pd/2 + 2*pd/64]."""
    xf = x.float()
    if xf.shape[-1] < pd:
        xf = torch.nn.functional.pad(xf, (0, pd - xf.shape[-1]))
    l2 = torch.sqrt((xf * xf).sum(-1, keepdim=True))
    inv = torch.where(l2 > 1e-8, 1.0 / l2, torch.zeros_like(l2))
    v = fwht(xf * inv * signs[:pd]) * (1.0 / math.sqrt(pd))
    code = torch.searchsorted(BOUNDARIES * (1.0 / math.sqrt(pd)), v.contiguous(), right=True)
    code = code.to(torch.uint8)
    packed = (code[..., 0::2] << 4) | code[..., 1::2]
    nb = l2.to(torch.float16).view(torch.uint8).reshape(*l2.shape[:-1], 2)
    return torch.cat([packed, nb.repeat(*([1] * (nb.dim() - 1)), pd // 64)], dim=-1)


def write_kv_cache(kv_cache: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   signs: torch.Tensor, slot_mapping: torch.Tensor, pd: int) -> None:
    """Scatter-quantize K/V [N, H, head_dim] into kv_cache uint8 [2, nb, bs, H, ebs]."""
    _, nb, bs, h, ebs = kv_cache.shape
    ok = (slot_mapping >= 0) & (slot_mapping < nb * bs)
    slots = slot_mapping[ok].long()
    n = pd // 2 + 2 * (pd // 64)
    flat = kv_cache.view(2, nb * bs, h, ebs)
    for i, src in enumerate((key, value)):
        flat[i, slots, :, :n] = quantize(src[ok], pd, signs)


def dequant(entries: torch.Tensor, pd: int) -> torch.Tensor:
    """Entry bytes [..., ebs] -> rotated-domain fp32 [..., pd] =
    c[code] * norm / sqrt(pd)."""
    codes = entries[..., :pd // 2]
    idx = torch.stack(((codes >> 4), (codes & 15)), dim=-1).reshape(*codes.shape[:-1], pd)
    norms = entries[..., pd // 2:pd // 2 + 2 * (pd // 64)].contiguous().view(torch.float16)
    norm = norms.float().repeat_interleave(64, dim=-1)
    return CODEBOOK[idx.long()] * norm * (1.0 / math.sqrt(pd))


def decode(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
           seq_lens: torch.Tensor, num_kv_heads: int, pd: int, sm_scale: float,
           signs: torch.Tensor | None) -> torch.Tensor:
    """q [B, Hq, pd] -> attention output fp32 [B, Hq, pd] in the original domain."""
    b, hq, _ = q.shape
    ratio = hq // num_kv_heads
    _, nb, bs, hk, ebs = kv_cache.shape
    out = torch.zeros((b, hq, pd), dtype=torch.float32)
    isq = 1.0 / math.sqrt(pd)
    qf = q.float()
    if signs is not None:
        qf = fwht(qf * signs[:pd]) * isq
    for i in range(b):
        L = int(seq_lens[i])
        if L <= 0:
            continue
        pages = block_table[i, :(L + bs - 1) // bs].long()
        for h in range(num_kv_heads):
            kk = dequant(kv_cache[0, pages, :, h].reshape(-1, ebs)[:L], pd)
            vv = dequant(kv_cache[1, pages, :, h].reshape(-1, ebs)[:L], pd)
            qq = qf[i, h * ratio:(h + 1) * ratio]
            p = torch.softmax((qq @ kk.T) * sm_scale, dim=-1)
            out[i, h * ratio:(h + 1) * ratio] = p @ vv
    if signs is not None:
        out = fwht(out) * isq * signs[:pd]
    return out
