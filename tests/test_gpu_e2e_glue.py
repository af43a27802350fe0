"""The end-to-end harness's layer glue kernels (tq_e2e.hip) against their
torch definitions: residual add + RMSNorm, per-head q/k RMSNorm + RoPE from a
fused QKV row, SiLU(g) * u.  fp32 arithmetic inside, one fp16 rounding per
output (torch rounds between its ops), so outputs agree within a few fp16
ulps."""
import math

import pytest
import torch
import torch.nn.functional as F

from turboquant_amd import e2e

pytestmark = pytest.mark.gpu


def _close(got, want, what, ulps=4):
    err = (got.float() - want.float()).abs()
    tol = ulps * torch.finfo(torch.float16).eps * want.float().abs().clamp_min(1e-2)
    bad = (err > tol).sum().item()
    print(f"  {what}: max |diff| {err.max().item():.3e}, beyond {ulps} ulp: {bad}", flush=True)
    assert bad == 0


@pytest.mark.parametrize("rows,hidden", [(1, 4096), (37, 4096), (300, 512), (8, 8192), (5, 40)])
def test_add_rms_norm(rows, hidden):
    print(f"case: e2e add_rms_norm rows={rows} hidden={hidden}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + hidden)
    x = torch.randn((rows, hidden), generator=g, device="cuda").half()
    y = torch.randn((rows, hidden), generator=g, device="cuda").half()
    w = (1 + 0.1 * torch.randn(hidden, generator=g, device="cuda")).half()
    h = torch.empty_like(x)
    x0 = x.clone()
    e2e.add_rms_norm(x, y, w, h, 1e-6)
    assert torch.equal(x, x0 + y)  # the fp16 add, rounded once
    _close(h, e2e.rms_norm(x.float(), w.float(), 1e-6), "norm of the sum")
    # norm alone (no y), add alone (no h)
    h2 = torch.empty_like(x)
    e2e.add_rms_norm(x, None, w, h2, 1e-6)
    assert torch.equal(h2, h)
    x1 = x.clone()
    e2e.add_rms_norm(x, y, None, None, 1e-6)
    assert torch.equal(x, x1 + y)


@pytest.mark.parametrize("tokens,hq,hkv,d", [(1, 32, 8, 128), (8, 32, 8, 128), (513, 32, 8, 128),
                                             (17, 16, 4, 64), (9, 16, 2, 256),
                                             (11, 8, 2, 96), (5, 4, 1, 40)])
def test_qk_norm_rope(tokens, hq, hkv, d):
    print(f"case: e2e qk_norm_rope tokens={tokens} {hq}/{hkv}/{d}", flush=True)
    s = e2e.ModelShape(layers=1, heads=hq, kv_heads=hkv, head_dim=d)
    g = torch.Generator(device="cuda").manual_seed(tokens * 7 + d)
    width = (hq + 2 * hkv) * d
    qkv = torch.randn((tokens, width), generator=g, device="cuda").half() * 3
    qw = (1 + 0.2 * torch.randn(d, generator=g, device="cuda")).half()
    kw = (1 + 0.2 * torch.randn(d, generator=g, device="cuda")).half()
    cos, sin = e2e.rope_tables(40000, d, 1.0e6, "cuda")
    pos = torch.randint(0, 40000, (tokens,), generator=g, device="cuda")
    q, k = e2e.qk_norm_rope(qkv, s, qw, kw, cos, sin, pos)
    qn = e2e.rms_norm(qkv[:, :hq * d].reshape(tokens, hq, d).float(), qw.float(), s.eps).half()
    kn = e2e.rms_norm(qkv[:, hq * d:(hq + hkv) * d].reshape(tokens, hkv, d).float(), kw.float(),
                      s.eps).half()
    c, sn = cos[pos].float(), sin[pos].float()
    want_q = qn.float() * c[:, None] + torch.roll(qn.float(), d // 2, -1) * sn[:, None]
    want_k = kn.float() * c[:, None] + torch.roll(kn.float(), d // 2, -1) * sn[:, None]
    # the normed value is rounded to fp16 on both sides; RoPE adds one rounding
    err_q = (q.float() - want_q).abs().max().item()
    err_k = (k.float() - want_k).abs().max().item()
    print(f"  max |diff| q {err_q:.3e}, k {err_k:.3e}", flush=True)
    assert err_q < 8e-3 and err_k < 8e-3
    assert torch.allclose(q.float(), want_q, rtol=4e-3, atol=4e-3)
    assert torch.allclose(k.float(), want_k, rtol=4e-3, atol=4e-3)
    # a position past the tables (or negative) gives NaN rows for that token
    # only, and no read outside the tables
    if tokens > 2:
        bad = pos.clone()
        bad[0], bad[2] = 40000, -1
        q2, k2 = e2e.qk_norm_rope(qkv, s, qw, kw, cos, sin, bad)
        for t in (0, 2):
            assert torch.isnan(q2[t]).all() and torch.isnan(k2[t]).all()
        keep = torch.ones(tokens, dtype=torch.bool, device="cuda")
        keep[0] = keep[2] = False
        assert torch.equal(q2[keep], q[keep]) and torch.equal(k2[keep], k[keep])


@pytest.mark.parametrize("rows,inter", [(1, 12288), (33, 12288), (100, 1024), (3, 8)])
def test_silu_mul(rows, inter):
    print(f"case: e2e silu_mul rows={rows} inter={inter}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + inter)
    gu = (torch.randn((rows, 2 * inter), generator=g, device="cuda") * 4).half()
    out = e2e.silu_mul(gu)
    gg, uu = gu.float().chunk(2, dim=-1)
    _close(out, F.silu(gg) * uu, "silu * u")


def test_layers_match_the_torch_definitions():
    """One tiny model's prefill logits with the glue kernels against the
    same model written with torch ops (rms_norm, rope, silu * u, fp16 SDPA
    over the prompt): the glue changes only fp16 roundings."""
    print("case: e2e tiny model glue against torch layers", flush=True)
    shape = e2e.ModelShape.tiny(layers=2)
    dev = torch.device("cuda:0")
    r = e2e.Runner(shape, 1, 64 + 8, dev, seed=3)
    tok = torch.randint(0, shape.vocab, (64,), generator=torch.Generator().manual_seed(5)).to(dev)
    first = r.prefill(0, tok)
    W = r.weights
    s = shape
    pos = torch.arange(64, device=dev)
    cos, sin = r.cos[pos], r.sin[pos]
    x = F.embedding(tok, W["embed"]).float()
    for lw in W["layers"]:
        h = e2e.rms_norm(x, lw["ln1"].float(), s.eps)
        qkv = h @ lw["qkv"].float().t()
        q, k, v = qkv.split([s.heads * s.head_dim, s.kv_heads * s.head_dim,
                             s.kv_heads * s.head_dim], -1)
        q = e2e.rms_norm(q.reshape(64, s.heads, s.head_dim), lw["q_norm"].float(), s.eps)
        k = e2e.rms_norm(k.reshape(64, s.kv_heads, s.head_dim), lw["k_norm"].float(), s.eps)
        q = q * cos[:, None].float() + torch.roll(q, s.head_dim // 2, -1) * sin[:, None].float()
        k = k * cos[:, None].float() + torch.roll(k, s.head_dim // 2, -1) * sin[:, None].float()
        o = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1),
                                           v.reshape(64, s.kv_heads, s.head_dim).transpose(0, 1),
                                           is_causal=True, scale=1 / math.sqrt(s.head_dim),
                                           enable_gqa=True).transpose(0, 1).reshape(64, -1)
        x = x + o @ lw["o"].float().t()
        h = e2e.rms_norm(x, lw["ln2"].float(), s.eps)
        gg, uu = (h @ lw["gate_up"].float().t()).chunk(2, -1)
        x = x + (F.silu(gg) * uu) @ lw["down"].float().t()
    logits = e2e.rms_norm(x[-1:], W["norm"].float(), s.eps) @ W["lm_head"].float().t()
    top5 = logits[0].topk(5).indices.tolist()
    print(f"  glue first token {first}, fp32 torch top-5 {top5}", flush=True)
    assert first in top5
