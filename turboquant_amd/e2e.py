"""End-to-end decode through the TurboQuant backend on one GPU.

The reference measures end-to-end output tokens/s by serving a model with
vLLM and its CUSTOM attention backend (reference tests/bench_vllm_serve.py:48-70,
docs/BENCHMARKS.md:60,71: Qwen3-8B, 32768 input and 256 output tokens,
concurrency 8).  vLLM is not part of this build, so this module is the
serving loop itself, in torch: a random-init decoder of the Qwen3-8B
architecture (36 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, MLP
12288, vocab 151936, RMSNorm with per-head q/k norms, RoPE theta 1e6, SwiGLU,
fp16 weights) whose every attention goes through the vLLM-facing
``TurboQuantFusedImpl`` exactly as vLLM drives it:

* ``do_kv_cache_update`` writes each step's K/V into the layer's quantized
  cache (the write kernel), then
* ``forward`` runs attention: a prompt through the prefill path, a decode
  batch through the balanced split-KV decode over the quantized cache.

Metadata objects carry the FlashAttentionMetadata fields the backend reads
(max_query_len, num_actual_tokens, block_table, seq_lens, query_start_loc,
slot_mapping).  Prompts are prefilled one at a time (each a fresh 32k-token
chunk); the decode step of the whole batch (embedding, 36 layers, final norm,
LM head, greedy argmax, position advance) is captured once in a HIP graph
and replayed once per output token.

Optionally (``keep_fp16_kv``) the runner also keeps an fp16 copy of every
layer's K/V and can decode the same model with plain fp16-KV SDPA attention,
so the greedy tokens of the two runs can be compared.
"""
from __future__ import annotations

import argparse
import json
import math
import time
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from . import ops
from .vllm_backend_fused import TurboQuantBackend, TurboQuantFusedImpl

BLOCK = 16


@dataclass(frozen=True)
class ModelShape:
    layers: int = 36
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 12288
    vocab: int = 151936
    rope_theta: float = 1.0e6
    eps: float = 1.0e-6

    @staticmethod
    def qwen3_8b() -> "ModelShape":
        return ModelShape()

    @staticmethod
    def tiny(layers: int = 2) -> "ModelShape":
        """Same attention geometry (32/8/128), small everything else."""
        return ModelShape(layers=layers, hidden=512, intermediate=1024, vocab=4096)


@dataclass
class Meta:
    """The FlashAttentionMetadata fields TurboQuantFusedImpl reads."""
    max_query_len: int
    num_actual_tokens: int
    block_table: torch.Tensor | None
    seq_lens: torch.Tensor | None
    query_start_loc: torch.Tensor
    slot_mapping: torch.Tensor | None


def build_weights(shape: ModelShape, seed: int, device) -> dict:
    """Random-init fp16 weights (normal, std 0.02; norm weights 1)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    h, d = shape.hidden, shape.head_dim
    qkv_out = (shape.heads + 2 * shape.kv_heads) * d

    def lin(o, i):
        return (torch.randn((o, i), generator=g, device=device, dtype=torch.float16) * 0.02)

    w = {"embed": lin(shape.vocab, h), "lm_head": lin(shape.vocab, h),
         "norm": torch.ones(h, dtype=torch.float16, device=device), "layers": []}
    for _ in range(shape.layers):
        w["layers"].append({
            "ln1": torch.ones(h, dtype=torch.float16, device=device),
            "ln2": torch.ones(h, dtype=torch.float16, device=device),
            "q_norm": torch.ones(d, dtype=torch.float16, device=device),
            "k_norm": torch.ones(d, dtype=torch.float16, device=device),
            "qkv": lin(qkv_out, h),
            "o": lin(h, shape.heads * d),
            "gate_up": lin(2 * shape.intermediate, h),
            "down": lin(h, shape.intermediate),
        })
    return w


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dim in torch (the definition the fused glue
    kernels below are tested against)."""
    return F.rms_norm(x, (x.shape[-1],), w, eps)


# ---------------------------------------------------------------- layer glue
# The model's elementwise work between the GEMMs runs as three fused HIP
# kernels (tq_e2e.hip): residual add + RMSNorm, per-head q/k RMSNorm + RoPE
# straight from the QKV GEMM's output, and SiLU(g) * u.

def add_rms_norm(x: torch.Tensor, y: torch.Tensor | None, w: torch.Tensor | None,
                 h: torch.Tensor | None, eps: float) -> None:
    """x += y (when y is given), then h = RMSNorm(x) * w (when h is given);
    x, y, h fp16 [T, H] contiguous, updated in place."""
    from . import _lib
    assert x.is_contiguous() and x.dtype == torch.float16
    rc = _lib.load().tq_e2e_add_rms_norm(
        x.data_ptr(), y.data_ptr() if y is not None else None,
        w.data_ptr() if w is not None else None, h.data_ptr() if h is not None else None,
        x.shape[0], x.shape[1], float(eps), ops._stream_ptr(x.device))
    _lib.check(rc, "e2e_add_rms_norm")


def qk_norm_rope(qkv: torch.Tensor, shape: "ModelShape", q_w: torch.Tensor, k_w: torch.Tensor,
                 cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor):
    """q [T, Hq, D] and k [T, Hkv, D] of a fused QKV GEMM output [T, *]:
    per-head RMSNorm, then rotate-half RoPE at positions pos (int64 [T])."""
    from . import _lib
    s = shape
    t = qkv.shape[0]
    q = torch.empty((t, s.heads, s.head_dim), dtype=torch.float16, device=qkv.device)
    k = torch.empty((t, s.kv_heads, s.head_dim), dtype=torch.float16, device=qkv.device)
    assert qkv.stride(1) == 1 and pos.dtype == torch.int64 and pos.is_contiguous()
    assert cos.shape == sin.shape and cos.shape[-1] == s.head_dim
    assert cos.is_contiguous() and sin.is_contiguous()
    rc = _lib.load().tq_e2e_qk_norm_rope(
        qkv.data_ptr(), qkv.stride(0), q_w.data_ptr(), k_w.data_ptr(), cos.data_ptr(),
        sin.data_ptr(), cos.shape[0], pos.data_ptr(), t, s.heads, s.kv_heads, s.head_dim, float(s.eps),
        q.data_ptr(), k.data_ptr(), ops._stream_ptr(qkv.device))
    _lib.check(rc, "e2e_qk_norm_rope")
    return q, k


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """SiLU(gu[:, :I]) * gu[:, I:] of the gate/up GEMM output [T, 2I]."""
    from . import _lib
    assert gu.is_contiguous()
    t, i2 = gu.shape
    out = torch.empty((t, i2 // 2), dtype=gu.dtype, device=gu.device)
    rc = _lib.load().tq_e2e_silu_mul(gu.data_ptr(), out.data_ptr(), t, i2 // 2,
                                     ops._stream_ptr(gu.device))
    _lib.check(rc, "e2e_silu_mul")
    return out


def rope_tables(n: int, d: int, theta: float, device) -> tuple[torch.Tensor, torch.Tensor]:
    """fp16 cos and signed-sin tables [n, d] of rotate-half RoPE (angles in
    fp32): x' = x * cos + roll(x, d/2) * sin_signed, sin_signed = (-sin, sin)."""
    inv = theta ** (-torch.arange(0, d, 2, device=device, dtype=torch.float32) / d)
    ang = torch.arange(n, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    cos = torch.cat((ang.cos(), ang.cos()), -1).half()
    sin = torch.cat((-ang.sin(), ang.sin()), -1).half()
    return cos, sin


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of x [T, H, D] with the table rows of its positions."""
    return torch.addcmul(x * cos[:, None, :], torch.roll(x, x.shape[-1] // 2, dims=-1),
                         sin[:, None, :])


def greedy(logits: torch.Tensor) -> torch.Tensor:
    """argmax over the vocabulary in two in-block stages (a group maximum,
    then the best group), int64 [B]."""
    b, v = logits.shape
    grp = 128 if v % 128 == 0 else 1
    vals, idx = logits.view(b, v // grp, grp).max(dim=2)
    j = vals.argmax(dim=1)
    return j * grp + idx.gather(1, j[:, None]).squeeze(1)


@dataclass
class Runner:
    """The model, its per-layer quantized caches and the decode state."""
    shape: ModelShape
    batch: int
    max_tokens: int               # per sequence (prompt + output)
    device: torch.device
    seed: int = 0
    keep_fp16_kv: bool = False
    weights: dict = field(default=None, repr=False)

    def __post_init__(self):
        s = self.shape
        dev = self.device
        if self.weights is None:
            self.weights = build_weights(s, self.seed, dev)
        self.pages_per_seq = math.ceil(self.max_tokens / BLOCK)
        nblocks = self.batch * self.pages_per_seq
        g = torch.Generator(device="cpu")
        g.manual_seed(self.seed + 1)
        # page ids: a seeded permutation of the pool, one table for all layers
        perm = torch.randperm(nblocks, generator=g).to(torch.int32)
        self.block_table = perm.view(self.batch, self.pages_per_seq).to(dev)
        shape5 = TurboQuantBackend.get_kv_cache_shape(nblocks, BLOCK, s.kv_heads, s.head_dim,
                                                      "fp8")
        self.caches = [torch.zeros(shape5, dtype=torch.uint8, device=dev)
                       for _ in range(s.layers)]
        self.impls = [TurboQuantFusedImpl(s.heads, s.head_dim, 1.0 / math.sqrt(s.head_dim),
                                          s.kv_heads, None, None, "fp8")
                      for _ in range(s.layers)]
        self.cos, self.sin = rope_tables(self.max_tokens, s.head_dim, s.rope_theta, dev)
        self.kv16 = None
        if self.keep_fp16_kv:
            self.kv16 = [torch.zeros((2, self.batch, s.kv_heads, self.max_tokens, s.head_dim),
                                     dtype=torch.float16, device=dev)
                         for _ in range(s.layers)]
        # decode state (fixed buffers, updated inside the captured step)
        self.pos = torch.zeros(self.batch, dtype=torch.int64, device=dev)
        self.tok = torch.zeros(self.batch, dtype=torch.int64, device=dev)
        self.seq_lens = torch.zeros(self.batch, dtype=torch.int32, device=dev)
        self.slots = torch.zeros(self.batch, dtype=torch.int32, device=dev)
        self.qsl = torch.arange(self.batch + 1, dtype=torch.int32, device=dev)
        self.out_buf = None
        self.step_idx = torch.zeros(1, dtype=torch.int64, device=dev)
        self.graph = None
        # list collecting (layer, q, k, v, out) of decode attention, eager only
        self.probe = None

    # ------------------------------------------------------------ layers
    def _qkv(self, lw, h, pos):
        """q, k (normed, rotated), v of the normed tokens h at positions pos."""
        s = self.shape
        t = h.shape[0]
        qkv = F.linear(h, lw["qkv"])
        q, k = qk_norm_rope(qkv, s, lw["q_norm"], lw["k_norm"], self.cos, self.sin, pos)
        v = qkv[:, (s.heads + s.kv_heads) * s.head_dim:].view(t, s.kv_heads, s.head_dim)
        return q, k, v

    def _layers(self, x, pos, attend):
        """Every layer over the residual stream x [T, hidden] (fp16,
        contiguous, updated in place): x += o_proj(attend(li, lw, q, k, v));
        x += MLP(x).  attend returns the attention output [T, Hq * D]."""
        s = self.shape
        layers = self.weights["layers"]
        h = torch.empty_like(x)
        add_rms_norm(x, None, layers[0]["ln1"], h, s.eps)
        for li, lw in enumerate(layers):
            q, k, v = self._qkv(lw, h, pos)
            o = attend(li, lw, q, k, v)
            add_rms_norm(x, F.linear(o, lw["o"]), lw["ln2"], h, s.eps)
            y = F.linear(silu_mul(F.linear(h, lw["gate_up"])), lw["down"])
            if li + 1 < len(layers):
                add_rms_norm(x, y, layers[li + 1]["ln1"], h, s.eps)
            else:
                add_rms_norm(x, y, None, None, s.eps)
        return x

    def _logits(self, x_rows):
        h = torch.empty_like(x_rows)
        add_rms_norm(x_rows, None, self.weights["norm"], h, self.shape.eps)
        return F.linear(h, self.weights["lm_head"])

    # ------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, b: int, tokens: torch.Tensor) -> int:
        """Prefill sequence b with `tokens` (int64 [L], a fresh prompt);
        returns the greedy first output token and sets the decode state."""
        s = self.shape
        dev = self.device
        L = tokens.numel()
        pos = torch.arange(L, device=dev)
        pages = self.block_table[b]
        slots = (pages[pos // BLOCK].to(torch.int64) * BLOCK + pos % BLOCK).to(torch.int32)
        meta = Meta(L, L, pages[None, :], torch.tensor([L], dtype=torch.int32, device=dev),
                    torch.tensor([0, L], dtype=torch.int32, device=dev), slots)
        x = F.embedding(tokens, self.weights["embed"])

        def attend(li, lw, q, k, v):
            impl = self.impls[li]
            impl.do_kv_cache_update(None, k, v, self.caches[li], slots)
            if self.kv16 is not None:
                self.kv16[li][0, b, :, :L] = k.transpose(0, 1)
                self.kv16[li][1, b, :, :L] = v.transpose(0, 1)
            return impl.forward(None, q.reshape(L, -1), k.reshape(L, -1), v.reshape(L, -1),
                                self.caches[li], meta)
        x = self._layers(x, pos, attend)
        first = greedy(self._logits(x[-1:]))
        self.pos[b] = L
        self.tok[b] = first[0]
        self.first_pos = self.pos.clone()
        self.first_tok = self.tok.clone()
        return int(first[0])

    # ------------------------------------------------------------ decode
    def _decode_body(self):
        """One decode step of the batch from (tok, pos); advances them."""
        s = self.shape
        pos = self.pos
        bt = self.block_table
        page = bt.gather(1, (pos // BLOCK)[:, None]).squeeze(1).to(torch.int64)
        self.slots.copy_((page * BLOCK + pos % BLOCK).to(torch.int32))
        self.seq_lens.copy_((pos + 1).to(torch.int32))
        meta = Meta(1, self.batch, bt, self.seq_lens, self.qsl, self.slots)
        x = F.embedding(self.tok, self.weights["embed"])

        def attend(li, lw, q, k, v):
            impl = self.impls[li]
            impl.do_kv_cache_update(None, k, v, self.caches[li], self.slots)
            o = impl.forward(None, q.reshape(self.batch, -1), k.reshape(self.batch, -1),
                             v.reshape(self.batch, -1), self.caches[li], meta)
            if self.probe is not None:
                self.probe.append((li, q.clone(), k.clone(), v.clone(), o.clone()))
            return o
        x = self._layers(x, pos, attend)
        nxt = greedy(self._logits(x))
        self.tok.copy_(nxt)
        self.out_buf.index_copy_(0, self.step_idx, nxt[None, :])
        self.pos.add_(1)
        self.step_idx.add_(1)

    def _start_decode(self, steps: int):
        self.out_buf = torch.zeros((steps, self.batch), dtype=torch.int64, device=self.device)
        self.step_idx.zero_()

    @torch.no_grad()
    def decode_eager(self, steps: int) -> torch.Tensor:
        self._start_decode(steps)
        for _ in range(steps):
            self._decode_body()
        return self.out_buf

    @torch.no_grad()
    def capture(self, steps: int):
        """Capture one decode step into a HIP graph that can be replayed up
        to `steps` times.  One eager warm-up step runs first (it sizes every
        workspace and loads the kernels); the state (pos, tok) is restored
        afterwards, so decoding continues from where the caller was.  The
        warm-up's cache writes land in the slots the first replay rewrites."""
        saved = (self.pos.clone(), self.tok.clone())
        self._start_decode(steps)
        self._decode_body()
        torch.cuda.synchronize()
        self.pos.copy_(saved[0])
        self.tok.copy_(saved[1])
        self.step_idx.zero_()
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            self._decode_body()
        torch.cuda.synchronize()
        self.pos.copy_(saved[0])
        self.tok.copy_(saved[1])
        self.step_idx.zero_()
        self.graph = g
        self.graph_steps = steps
        return g

    @torch.no_grad()
    def decode_graph(self, steps: int) -> torch.Tensor:
        """`steps` replays of the captured step from the current state;
        returns the tokens [steps, B]."""
        assert self.graph is not None and steps <= self.graph_steps
        self.step_idx.zero_()
        for _ in range(steps):
            self.graph.replay()
        return self.out_buf[:steps]

    # ------------------------------------------------------- fp16 reference
    @torch.no_grad()
    def fp16_attention(self, li: int, q: torch.Tensor, k: torch.Tensor,
                       v: torch.Tensor) -> torch.Tensor:
        """Decode attention of layer li over fp16 K/V (no quantization): q
        [B, Hq, D] of one decode step whose new token's k, v [B, Hkv, D] sit
        at position pos - 1 (after the step), the earlier tokens from the
        fp16 copies the prefill kept.  Equal sequence lengths only.
        Returns [B, Hq, D] fp16."""
        assert self.kv16 is not None
        p = int(self.pos[0]) - 1
        assert bool((self.pos == p + 1).all()), "fp16_attention needs equal lengths"
        kvl = self.kv16[li]
        kk = torch.cat([kvl[0, :, :, :p], k[:, :, None, :]], dim=2)
        vv = torch.cat([kvl[1, :, :, :p], v[:, :, None, :]], dim=2)
        o = F.scaled_dot_product_attention(q[:, :, None, :], kk, vv,
                                           scale=1.0 / math.sqrt(self.shape.head_dim),
                                           enable_gqa=True)
        return o[:, :, 0, :]

    @torch.no_grad()
    def decode_fp16_reference(self, steps: int, forced: torch.Tensor | None = None,
                              kv: str = "fp16"):
        """The same model decoded from the state the prefill left, with
        attention in torch SDPA over

        * kv="fp16": the fp16 K/V copies (no quantization);
        * kv="dequant": the quantized cache read back as fp16 rows in the
          original domain (tq_dequant_paged), the new token's K/V written
          into the cache first: the reference's dequantize-then-attend
          semantics (triton_decode_ref.py:264-299), so the difference from
          the fused decode is the fused kernel's arithmetic alone.  It
          rewrites the cache entries of the positions it decodes (the same
          slots the fused decode writes).

        forced None: greedy free run; returns its tokens [steps, B].
        forced [steps, B] (another run's tokens): teacher forcing, each step
        fed the forced history; returns (top-1 tokens, rank of the forced
        token among this run's logits), both [steps, B]."""
        assert kv in ("fp16", "dequant")
        assert kv == "dequant" or self.kv16 is not None
        s = self.shape
        out = torch.zeros((steps, self.batch), dtype=torch.int64, device=self.device)
        rank = torch.zeros((steps, self.batch), dtype=torch.int64, device=self.device)
        pos = self.first_pos.clone()
        tok = self.first_tok.clone()
        scale = 1.0 / math.sqrt(s.head_dim)
        p0 = int(pos[0])
        assert bool((pos == p0).all()), "the reference decode needs equal lengths"
        if kv == "dequant":
            kd = torch.empty((2, self.batch, self.max_tokens, s.kv_heads, s.head_dim),
                             dtype=torch.float16, device=self.device)
        bt = self.block_table
        for step in range(steps):
            p = p0 + step
            x = F.embedding(tok, self.weights["embed"])
            if kv == "dequant":
                page = bt.gather(1, (pos // BLOCK)[:, None]).squeeze(1).to(torch.int64)
                slots = (page * BLOCK + pos % BLOCK).to(torch.int32)

            def attend(li, lw, q, k, v):
                if kv == "fp16":
                    kvl = self.kv16[li]
                    kvl[0, :, :, p] = k
                    kvl[1, :, :, p] = v
                    kk, vv = kvl[0, :, :, :p + 1], kvl[1, :, :, :p + 1]
                else:
                    impl = self.impls[li]
                    impl.do_kv_cache_update(None, k, v, self.caches[li], slots)
                    for b in range(self.batch):
                        ops.dequant_paged(self.caches[li], bt[b], p + 1, s.kv_heads, s.head_dim,
                                          impl._pd, impl._signs, kd[0, b], kd[1, b])
                    kk = kd[0, :, :p + 1].transpose(1, 2)
                    vv = kd[1, :, :p + 1].transpose(1, 2)
                o = F.scaled_dot_product_attention(q[:, :, None, :], kk, vv, scale=scale,
                                                   enable_gqa=True)
                return o.reshape(self.batch, -1)
            x = self._layers(x, pos, attend)
            logits = self._logits(x)
            top = greedy(logits)
            out[step] = top
            if forced is not None:
                f = forced[step]
                lf = logits.gather(1, f[:, None])
                rank[step] = (logits > lf).sum(1)
                tok = f
            else:
                tok = top
            pos = pos + 1
        return out if forced is None else (out, rank)

@torch.no_grad()
def attention_vs_fp16(r: Runner) -> dict:
    """The quantization error where it enters the model: one eager decode
    step from the prefill's state, every layer's decode attention output
    (fused kernel over the quantized cache) against attention over the fp16
    K/V of the same step (Runner.fp16_attention); per (sequence, q head) row
    the cosine similarity and the relative L2 error.  The decode state is
    restored afterwards."""
    pos0, tok0 = r.pos.clone(), r.tok.clone()
    r.probe = []
    r.decode_eager(1)
    probe, r.probe = r.probe, None
    cos, rel = [], []
    for li, q, k, v, o in probe:
        ref = r.fp16_attention(li, q, k, v).float().flatten(0, 1)
        got = o.float().reshape(ref.shape)
        cos.append(F.cosine_similarity(got, ref, dim=-1))
        rel.append((got - ref).norm(dim=-1) / ref.norm(dim=-1).clamp_min(1e-30))
    r.pos.copy_(pos0)
    r.tok.copy_(tok0)
    cos = torch.stack(cos)
    rel = torch.stack(rel)
    return {"layers": len(probe), "rows_per_layer": int(cos.shape[1]),
            "cosine_min": round(cos.min().item(), 6), "cosine_mean": round(cos.mean().item(), 6),
            "rel_l2_err_mean": round(rel.mean().item(), 6),
            "rel_l2_err_max": round(rel.max().item(), 6),
            "reference": "same step's attention over fp16 K/V (torch SDPA), no quantization"}


def run(shape: ModelShape, batch: int = 8, prompt_len: int = 32768, new_tokens: int = 256,
        seed: int = 0, compare_steps: int = 0, device: str = "cuda:0", log=None) -> dict:
    """Prefill `batch` random prompts of `prompt_len` tokens one after another,
    then decode `new_tokens` - 1 more tokens for the whole batch with graph
    replays (the first output token comes from the prefill).  Returns the
    serving figures:

    * output_tok_s: batch * new_tokens / (prefill + decode wall time), the
      output-token throughput a serving benchmark reports;
    * decode_tok_s, tpot_ms: the decode phase alone (time per output token
      after the first);
    * ttft_s: mean time to first token with the prompts prefilled in turn;
    * with compare_steps > 0, the greedy-token agreement with the same model
      decoded over fp16 K/V for that many steps from the same prefill.
    Graph capture (a one-time setup, as a server does at start-up) is timed
    separately and not counted."""
    dev = torch.device(device)
    say = log or (lambda *a: None)
    r = Runner(shape, batch, prompt_len + new_tokens, dev, seed,
               keep_fp16_kv=compare_steps > 0)
    g = torch.Generator(device="cpu")
    g.manual_seed(seed + 2)
    prompts = torch.randint(0, shape.vocab, (batch, prompt_len), generator=g)
    # one short throwaway prefill so that library initialisation (GEMM
    # heuristics, kernel loading) is not charged to the first request
    warm = Runner(shape, 1, 64, dev, seed, weights=r.weights)
    warm.prefill(0, prompts[0, :48].to(dev))
    del warm
    torch.cuda.synchronize()
    ttft = []
    t0 = time.perf_counter()
    for b in range(batch):
        r.prefill(b, prompts[b].to(dev))
        torch.cuda.synchronize()
        ttft.append(time.perf_counter() - t0)
        say(f"[e2e] prefill {b + 1}/{batch}: {ttft[-1]:.2f} s")
    t_prefill = time.perf_counter() - t0
    first = r.tok.clone()
    res = {}
    if compare_steps > 0:
        res["attention_vs_fp16"] = attention_vs_fp16(r)
        free = r.decode_fp16_reference(compare_steps)
        free_dq = r.decode_fp16_reference(compare_steps, kv="dequant")
        torch.cuda.synchronize()
    steps = new_tokens - 1
    tc = time.perf_counter()
    r.capture(steps)
    torch.cuda.synchronize()
    t_capture = time.perf_counter() - tc
    t1 = time.perf_counter()
    toks = r.decode_graph(steps)
    torch.cuda.synchronize()
    t_decode = time.perf_counter() - t1
    say(f"[e2e] decode {steps} steps: {t_decode * 1e3:.1f} ms")
    if compare_steps > 0:
        n = min(compare_steps, steps)

        def agreement(free_toks, kv, what):
            same = (toks[:n] == free_toks[:n]).cpu()
            div = [int((~same[:, b]).nonzero()[0, 0]) if (~same[:, b]).any() else n
                   for b in range(batch)]
            top, rank = r.decode_fp16_reference(n, forced=toks[:n], kv=kv)
            rank = rank.cpu()
            return {
                "steps": n,
                "reference": what,
                "free_run_token_match_rate": float(same.float().mean()),
                "free_run_first_divergence_step": div,
                "teacher_forced_top1_match_rate": float((top[:n] == toks[:n]).float().mean()),
                "teacher_forced_in_top5_rate": float((rank < 5).float().mean()),
                "teacher_forced_median_rank": float(rank.float().median()),
            }

        res["agreement"] = agreement(
            free, "fp16", "same model and prefill, attention over fp16 K/V (torch SDPA)")
        res["agreement_dequant"] = agreement(
            free_dq, "dequant", "same model, prefill and quantized cache, attention over the "
            "cache read back as fp16 rows (dequantize-then-attend, torch SDPA)")
    res.update({
        "output_tok_s": batch * new_tokens / (t_prefill + t_decode),
        "decode_tok_s": batch * steps / t_decode if steps else None,
        "tpot_ms": t_decode / steps * 1e3 if steps else None,
        "ttft_s": sum(ttft) / len(ttft),
        "prefill_s": t_prefill,
        "decode_s": t_decode,
        "capture_s": t_capture,
        "batch": batch, "prompt_len": prompt_len, "new_tokens": new_tokens,
        "layers": shape.layers,
        "first_tokens": first.tolist(),
    })
    r.tokens = toks
    return res


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--tiny", action="store_true", help="small hidden/MLP/vocab (tests)")
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=32768)
    ap.add_argument("--new", type=int, default=256)
    ap.add_argument("--compare", type=int, default=0,
                    help="greedy-agreement steps against an fp16-KV run")
    ap.add_argument("--seed", type=int, default=0)
    a = ap.parse_args(argv)
    shape = ModelShape.tiny(a.layers) if a.tiny else ModelShape(layers=a.layers)
    res = run(shape, a.batch, a.prompt, a.new, a.seed, a.compare,
              log=lambda m: print(m, flush=True))
    print(json.dumps(res))


if __name__ == "__main__":
    main()
