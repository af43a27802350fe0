"""torch-facing ops over the C ABI, registered under the reference's op names.

* ``torch.ops.turboquant_write.quantize_write_kv_cache`` — schema of
  csrc/src/quantize_write_binding.cu:285-286 (reference).
* ``torch.ops.turboquant_v5.decode_v5_from_cache_paged_splitkv_ws`` — schema of
  csrc/src/decode_v5_tc_binding.cu:966-973 (reference).
* ``torch.ops.turboquant_v5.decode_paged_balanced_ws`` — the same decode with
  the split plan made on the GPU from seq_lens (ragged batches); the
  backend's default.
* ``torch.ops.turboquant_v5.decode_v5_from_cache_ws`` and
  ``decode_v5_from_cache_splitkv_ws`` — schemas of decode_v5_tc_binding.cu:948-964,
  the non-split (graph-safe) and gather-then-split ops the reference backend
  and tests call; ``decode_v5_from_cache`` is the eager (allocating) form.

Both launch on the current torch stream, allocate nothing and never sync, so
they can be captured in a HIP graph.  They have a CUDA (= HIP on ROCm) kernel
only: CPU tensors raise.
"""
from __future__ import annotations

import torch

from . import _lib
from .geometry import entry_bytes

_DTYPES = {torch.float32: _lib.TQ_F32, torch.float16: _lib.TQ_F16, torch.bfloat16: _lib.TQ_BF16}


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(*tensors: torch.Tensor) -> None:
    """Every tensor on a GPU, and all on the same one (the kernels launch on
    the first tensor's device and read the others' addresses there)."""
    dev = None
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError("TurboQuant ops run on the GPU only; got a CPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"TurboQuant ops need all tensors on one GPU: {dev} and {t.device}")


def quantize_write_kv_cache(kv_cache: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            signs: torch.Tensor, slot_mapping: torch.Tensor, head_dim: int,
                            padded_dim: int) -> None:
    """Quantize K/V [num_tokens, H, head_dim] and scatter into kv_cache in place.

    kv_cache: uint8-addressable [2, num_blocks, block_size, H, ebs].  Mirrors
    quantize_write_kv_cache (quantize_write_binding.cu:207-269) including its
    checks; key/value may be fp32 (as the reference requires), fp16 or bf16.
    """
    if kv_cache.dim() != 5 or kv_cache.size(0) != 2:
        raise RuntimeError("kv_cache leading dim must be 2 (K,V)")
    if slot_mapping.dtype != torch.int32:
        raise RuntimeError("slot_mapping must be int32")
    if key.dtype not in _DTYPES or value.dtype != key.dtype:
        raise RuntimeError(f"key/value must share a float dtype, got {key.dtype}/{value.dtype}")
    if key.dim() != 3 or value.shape != key.shape:
        raise RuntimeError("key/value must be [num_tokens, num_heads, head_dim]")
    if key.size(2) < head_dim:
        # the kernel reads head_dim elements of every row
        raise RuntimeError(f"key/value rows hold {key.size(2)} elements, fewer than "
                           f"head_dim {head_dim}")
    _require_gpu(kv_cache, key, value, signs, slot_mapping)
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise RuntimeError("key/value last dim must be contiguous")
    ebs = kv_cache.size(-1) * kv_cache.element_size()
    if ebs % 16 != 0:
        raise RuntimeError(f"kv_cache.size(-1) must be 16-byte aligned, got {ebs}")
    if not kv_cache.is_contiguous():
        raise RuntimeError("kv_cache must be contiguous")
    if signs.dtype != torch.float32 or signs.numel() < padded_dim:
        raise RuntimeError("signs must be fp32 [padded_dim]")
    num_tokens = min(key.size(0), slot_mapping.numel())
    if num_tokens == 0:
        return
    _, nb, bs, h, _ = kv_cache.shape
    if key.size(1) != h:
        raise RuntimeError(f"key has {key.size(1)} heads, cache has {h}")
    lib = _lib.load()
    base = kv_cache.data_ptr()
    slab = nb * bs * h * ebs
    with torch.cuda.device(kv_cache.device):
        rc = lib.tq_quantize_write_kv_cache(
            base, base + slab, key.data_ptr(), value.data_ptr(), _DTYPES[key.dtype],
            key.stride(0), key.stride(1), value.stride(0), value.stride(1),
            signs.data_ptr(), slot_mapping.data_ptr(), num_tokens, h, int(head_dim),
            int(padded_dim), bs, ebs, nb, _stream_ptr(kv_cache.device))
    _lib.check(rc, "quantize_write_kv_cache")


def decode_paged_splitkv(q: torch.Tensor, kv_cache: torch.Tensor, indices: torch.Tensor,
                         indptr: torch.Tensor, seq_lens: torch.Tensor, num_kv_heads: int,
                         head_dim: int, padded_dim: int, sm_scale: float,
                         signs: torch.Tensor | None, o: torch.Tensor, partition_o: torch.Tensor,
                         partition_lse: torch.Tensor, num_splits: int,
                         kv_chunk_size: int) -> torch.Tensor:
    """Split-KV decode: q fp16 [B, Hq, pd] -> o fp16 [B, Hq, pd] (returned)."""
    _require_gpu(q, kv_cache, indices, indptr, seq_lens, o, partition_o, partition_lse)
    if q.dtype != torch.float16 or q.dim() != 3 or q.size(2) != padded_dim or q.stride(2) != 1:
        raise RuntimeError("q must be fp16 [B, Hq, padded_dim] with a contiguous last dim")
    b, hq, pd = q.shape
    for t, name in ((indices, "indices"), (indptr, "indptr"), (seq_lens, "seq_lens")):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise RuntimeError(f"{name} must be a contiguous int32 tensor")
    if seq_lens.numel() < b or indptr.numel() < b:
        raise RuntimeError("seq_lens / indptr shorter than the batch")
    if tuple(o.shape) != (b, hq, pd) or o.dtype != torch.float16 or not o.is_contiguous():
        raise RuntimeError("o_ws shape mismatch")
    if (partition_o.dtype != torch.float32 or partition_o.numel() < b * num_splits * hq * pd
            or not partition_o.is_contiguous()):
        raise RuntimeError("partition_o_ws shape/dtype mismatch")
    if (partition_lse.dtype != torch.float32 or partition_lse.numel() < b * num_splits * hq
            or not partition_lse.is_contiguous()):
        raise RuntimeError("partition_lse_ws shape/dtype mismatch")
    if kv_cache.dim() != 5 or kv_cache.size(0) != 2 or not kv_cache.is_contiguous():
        raise RuntimeError("kv_cache must be contiguous [2, num_blocks, block_size, H, ebs]")
    _, nb, bs, hk, _ = kv_cache.shape
    if hk != num_kv_heads:
        raise RuntimeError(f"kv_cache has {hk} kv heads, num_kv_heads={num_kv_heads}")
    ebs = kv_cache.size(-1) * kv_cache.element_size()
    sp = 0
    if signs is not None and signs.numel() > 0:
        if signs.dtype != torch.float32 or signs.numel() < pd:
            raise RuntimeError("hadamard_signs must be fp32 [padded_dim]")
        _require_gpu(q, signs)
        sp = signs.data_ptr()
    lib = _lib.load()
    base = kv_cache.data_ptr()
    slab = nb * bs * hk * ebs
    with torch.cuda.device(q.device):
        rc = lib.tq_decode_paged_splitkv(
            q.data_ptr(), q.stride(0), q.stride(1), base, base + slab, indices.data_ptr(),
            indptr.data_ptr(), seq_lens.data_ptr(), b, hq, int(num_kv_heads), int(head_dim),
            int(padded_dim), bs, ebs, nb, float(sm_scale), sp, int(num_splits),
            int(kv_chunk_size), partition_o.data_ptr(), partition_lse.data_ptr(), o.data_ptr(),
            _stream_ptr(q.device))
    _lib.check(rc, "decode_paged_splitkv")
    return o


def balanced_rows(batch: int, num_qo_heads: int, num_kv_heads: int, padded_dim: int,
                  device: torch.device | None = None) -> int:
    """Partial rows a balanced decode of this geometry may use on `device`
    (the resident workgroup slots of the partials kernel, at least one per
    sequence): size partition_o [rows, Hq, pd] and partition_lse [rows, Hq]."""
    lib = _lib.load()
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        rows = lib.tq_decode_balanced_rows(int(batch), int(num_qo_heads), int(num_kv_heads),
                                           int(padded_dim))
    if rows < 0:
        _lib.check(rows, "decode_balanced_rows")
    return rows


def decode_paged_balanced(q: torch.Tensor, kv_cache: torch.Tensor, indices: torch.Tensor,
                          indptr: torch.Tensor, seq_lens: torch.Tensor, num_kv_heads: int,
                          head_dim: int, padded_dim: int, sm_scale: float,
                          signs: torch.Tensor | None, o: torch.Tensor,
                          partition_o: torch.Tensor, partition_lse: torch.Tensor,
                          split_indptr: torch.Tensor) -> torch.Tensor:
    """Split-KV decode with the split plan made on the GPU from seq_lens:
    every work unit covers about the same number of tokens whatever the
    length mix of the batch (the reference sizes splits from max_len,
    vllm_backend_fused.py:128-156).  split_indptr int32 [B + 2] receives the
    partial-row table (sequence b owns rows split_indptr[b] ..
    split_indptr[b + 1]) and, last, the unit size in tokens.  No host read,
    so it can be captured in a HIP graph whose seq_lens change per replay."""
    _require_gpu(q, kv_cache, indices, indptr, seq_lens, o, partition_o, partition_lse,
                 split_indptr)
    if q.dtype != torch.float16 or q.dim() != 3 or q.size(2) != padded_dim or q.stride(2) != 1:
        raise RuntimeError("q must be fp16 [B, Hq, padded_dim] with a contiguous last dim")
    b, hq, pd = q.shape
    for t, name in ((indices, "indices"), (indptr, "indptr"), (seq_lens, "seq_lens"),
                    (split_indptr, "split_indptr")):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise RuntimeError(f"{name} must be a contiguous int32 tensor")
    if seq_lens.numel() < b or indptr.numel() < b:
        raise RuntimeError("seq_lens / indptr shorter than the batch")
    if split_indptr.numel() < b + 2:
        raise RuntimeError("split_indptr must hold batch + 2 entries")
    if tuple(o.shape) != (b, hq, pd) or o.dtype != torch.float16 or not o.is_contiguous():
        raise RuntimeError("o_ws shape mismatch")
    if (partition_o.dtype != torch.float32 or partition_o.dim() != 3
            or tuple(partition_o.shape[1:]) != (hq, pd) or not partition_o.is_contiguous()):
        raise RuntimeError("partition_o_ws must be fp32 [rows, Hq, padded_dim]")
    rows = partition_o.size(0)
    if (partition_lse.dtype != torch.float32 or partition_lse.numel() < rows * hq
            or not partition_lse.is_contiguous()):
        raise RuntimeError("partition_lse_ws must be fp32 [rows, Hq]")
    if kv_cache.dim() != 5 or kv_cache.size(0) != 2 or not kv_cache.is_contiguous():
        raise RuntimeError("kv_cache must be contiguous [2, num_blocks, block_size, H, ebs]")
    _, nb, bs, hk, _ = kv_cache.shape
    if hk != num_kv_heads:
        raise RuntimeError(f"kv_cache has {hk} kv heads, num_kv_heads={num_kv_heads}")
    ebs = kv_cache.size(-1) * kv_cache.element_size()
    sp = 0
    if signs is not None and signs.numel() > 0:
        if signs.dtype != torch.float32 or signs.numel() < pd:
            raise RuntimeError("hadamard_signs must be fp32 [padded_dim]")
        _require_gpu(q, signs)
        sp = signs.data_ptr()
    lib = _lib.load()
    base = kv_cache.data_ptr()
    slab = nb * bs * hk * ebs
    with torch.cuda.device(q.device):
        rc = lib.tq_decode_paged_balanced(
            q.data_ptr(), q.stride(0), q.stride(1), base, base + slab, indices.data_ptr(),
            indptr.data_ptr(), seq_lens.data_ptr(), b, hq, int(num_kv_heads), int(head_dim),
            int(padded_dim), bs, ebs, nb, float(sm_scale), sp, rows, partition_o.data_ptr(),
            partition_lse.data_ptr(), split_indptr.data_ptr(), o.data_ptr(),
            _stream_ptr(q.device))
    _lib.check(rc, "decode_paged_balanced")
    return o


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                      sm_scale: float) -> torch.Tensor:
    """Causal GQA attention of q [Lq, Hq, D] over k, v [Lk, Hkv, D] (fp16,
    D = 64, 128 or 256, Lq <= Lk), the queries aligned to the end of the keys
    (query i sees keys <= Lk - Lq + i), written into o [Lq, Hq, D] fp16.
    Heads and dims of every tensor contiguous; token strides free (multiples
    of 8)."""
    _require_gpu(q, k, v, o)
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (o, "o")):
        if t.dtype != torch.float16 or t.dim() != 3 or t.stride(2) != 1:
            raise RuntimeError(f"{name} must be fp16 [tokens, heads, head_dim] with contiguous dims")
    lq, hq, d = q.shape
    lk, hkv, dk = k.shape
    if tuple(v.shape) != (lk, hkv, dk) or dk != d or tuple(o.shape) != (lq, hq, d):
        raise RuntimeError("prefill_attention: q/k/v/o shapes disagree")
    lib = _lib.load()
    with torch.cuda.device(q.device):
        # a short chunk over a long context splits its keys over workgroups;
        # the split's workspace comes from torch's allocator (graph-safe)
        nbytes = int(lib.tq_prefill_workspace_bytes(int(lq), int(lk), int(hq), int(hkv), int(d)))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes > 0 else None
        rc = lib.tq_prefill_attention_ws(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                                         k.stride(0), k.stride(1), v.data_ptr(), v.stride(0),
                                         v.stride(1), o.data_ptr(), o.stride(0), o.stride(1),
                                         int(lq), int(lk), int(hq), int(hkv), int(d),
                                         float(sm_scale),
                                         ws.data_ptr() if ws is not None else None, nbytes,
                                         _stream_ptr(q.device))
    _lib.check(rc, "prefill_attention")
    return o


def dequant_paged(kv_cache: torch.Tensor, pages: torch.Tensor, num_tokens: int,
                  num_kv_heads: int, head_dim: int, padded_dim: int,
                  signs: torch.Tensor | None, out_k: torch.Tensor, out_v: torch.Tensor) -> None:
    """Cached K/V of tokens [0, num_tokens) of one sequence (its page-table
    row `pages`) as fp16 rows [num_tokens, H_kv, head_dim] in the original
    domain, written into out_k / out_v (rows may be strided, heads and dims
    contiguous)."""
    _require_gpu(kv_cache, pages, out_k, out_v)
    if kv_cache.dim() != 5 or kv_cache.size(0) != 2 or not kv_cache.is_contiguous():
        raise RuntimeError("kv_cache must be contiguous [2, num_blocks, block_size, H, ebs]")
    _, nb, bs, hk, _ = kv_cache.shape
    if hk != num_kv_heads:
        raise RuntimeError(f"kv_cache has {hk} kv heads, num_kv_heads={num_kv_heads}")
    if pages.dtype != torch.int32 or not pages.is_contiguous():
        raise RuntimeError("pages must be a contiguous int32 tensor")
    if num_tokens > pages.numel() * bs:
        raise RuntimeError("pages do not cover num_tokens")
    for t in (out_k, out_v):
        if (t.dtype != torch.float16 or t.dim() != 3 or t.size(0) < num_tokens
                or t.size(1) != num_kv_heads or t.size(2) != head_dim or t.stride(2) != 1
                or t.stride(1) != head_dim or t.stride(0) != out_k.stride(0)):
            raise RuntimeError("out_k / out_v must be fp16 [>= num_tokens, H_kv, head_dim] "
                               "with contiguous heads and one row stride")
    if num_tokens == 0:
        return
    ebs = kv_cache.size(-1) * kv_cache.element_size()
    sp = 0
    if signs is not None and signs.numel() > 0:
        if signs.dtype != torch.float32 or signs.numel() < padded_dim:
            raise RuntimeError("signs must be fp32 [padded_dim]")
        _require_gpu(kv_cache, signs)
        sp = signs.data_ptr()
    lib = _lib.load()
    base = kv_cache.data_ptr()
    slab = nb * bs * hk * ebs
    with torch.cuda.device(kv_cache.device):
        rc = lib.tq_dequant_paged(base, base + slab, pages.data_ptr(), int(num_tokens),
                                  int(num_kv_heads), int(head_dim), int(padded_dim), bs, ebs, nb,
                                  sp, out_k.data_ptr(), out_v.data_ptr(), out_k.stride(0),
                                  _stream_ptr(kv_cache.device))
    _lib.check(rc, "dequant_paged")


def _host_f32(values) -> "ctypes.Array":
    import ctypes
    vals = [float(v) for v in values]
    return (ctypes.c_float * max(1, len(vals)))(*vals)


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    """t contiguous at a 16-byte aligned address (the kernels read it in
    16-byte pieces); a copy when it is not."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def mse_quantize(x: torch.Tensor, padded_dim: int, bit_width: int, signs: torch.Tensor,
                 boundaries) -> tuple[torch.Tensor, torch.Tensor]:
    """TurboQuantMSE.quantize on the GPU (tq_mse_quantize): x fp32
    [..., dim] -> (packed uint8 [..., padded_dim / per], norms fp32 [...]).
    `boundaries` are the codebook's 2^b - 1 scaled boundaries as host
    floats."""
    _require_gpu(x, signs)
    if x.dtype != torch.float32:
        raise RuntimeError("mse_quantize: x must be fp32")
    if signs.dtype != torch.float32 or signs.numel() < padded_dim:
        raise RuntimeError("mse_quantize: signs must be fp32 [padded_dim]")
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()  # the kernel reads whole rows as float4
    dim = x.shape[-1]
    lead = x.shape[:-1]
    n = x.numel() // dim if dim else 0
    per = 2 if bit_width == 3 else 8 // bit_width
    packed = torch.empty((*lead, padded_dim // per), dtype=torch.uint8, device=x.device)
    norms = torch.empty(lead, dtype=torch.float32, device=x.device)
    signs = _aligned16(signs)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.tq_mse_quantize(x.data_ptr(), n, dim, int(padded_dim), int(bit_width),
                                 signs.data_ptr(), _host_f32(boundaries), packed.data_ptr(),
                                 norms.data_ptr(), _stream_ptr(x.device))
    _lib.check(rc, "mse_quantize")
    return packed, norms


def mse_dequantize(packed: torch.Tensor, norms: torch.Tensor, dim: int, padded_dim: int,
                   bit_width: int, signs: torch.Tensor, centroids) -> torch.Tensor:
    """TurboQuantMSE.dequantize on the GPU (tq_mse_dequantize): packed uint8
    [..., padded_dim / per] and norms [...] -> fp32 [..., dim].  `centroids`
    are the codebook's 2^b scaled levels as host floats."""
    _require_gpu(packed, norms, signs)
    per = 2 if bit_width == 3 else 8 // bit_width
    if packed.dtype != torch.uint8 or packed.shape[-1] != padded_dim // per:
        raise RuntimeError("mse_dequantize: packed must be uint8 [..., padded_dim / per]")
    if tuple(norms.shape) != tuple(packed.shape[:-1]):
        raise RuntimeError("mse_dequantize: norms must match packed's leading dims")
    packed = packed.contiguous()
    if packed.data_ptr() % 16:
        packed = packed.clone()  # the kernel reads a lane's codes as dwords
    nf = norms.to(torch.float32).contiguous()
    lead = packed.shape[:-1]
    n = nf.numel()
    out = torch.empty((*lead, dim), dtype=torch.float32, device=packed.device)
    signs = _aligned16(signs)
    lib = _lib.load()
    with torch.cuda.device(packed.device):
        rc = lib.tq_mse_dequantize(packed.data_ptr(), nf.data_ptr(), n, int(dim),
                                   int(padded_dim), int(bit_width), signs.data_ptr(),
                                   _host_f32(centroids), out.data_ptr(),
                                   _stream_ptr(packed.device))
    _lib.check(rc, "mse_dequantize")
    return out


def prod_quantize(x: torch.Tensor, padded_dim: int, mse_bit_width: int, signs: torch.Tensor,
                  boundaries, centroids):
    """TurboQuantProd's MSE stage and residual on the GPU (tq_prod_quantize):
    x fp32 [..., dim] -> (packed, norms, residual_unit fp32 [..., dim],
    residual_norms fp32 [...]); packed and norms are mse_quantize's."""
    _require_gpu(x, signs)
    if x.dtype != torch.float32:
        raise RuntimeError("prod_quantize: x must be fp32")
    if signs.dtype != torch.float32 or signs.numel() < padded_dim:
        raise RuntimeError("prod_quantize: signs must be fp32 [padded_dim]")
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    dim = x.shape[-1]
    lead = x.shape[:-1]
    n = x.numel() // dim if dim else 0
    per = 2 if mse_bit_width == 3 else 8 // mse_bit_width
    packed = torch.empty((*lead, padded_dim // per), dtype=torch.uint8, device=x.device)
    norms = torch.empty(lead, dtype=torch.float32, device=x.device)
    resid = torch.empty((*lead, dim), dtype=torch.float32, device=x.device)
    rnorm = torch.empty(lead, dtype=torch.float32, device=x.device)
    signs = _aligned16(signs)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.tq_prod_quantize(x.data_ptr(), n, dim, int(padded_dim), int(mse_bit_width),
                                  signs.data_ptr(), _host_f32(boundaries), _host_f32(centroids),
                                  packed.data_ptr(), norms.data_ptr(), resid.data_ptr(),
                                  rnorm.data_ptr(), _stream_ptr(x.device))
    _lib.check(rc, "prod_quantize")
    return packed, norms, resid, rnorm


def prod_dequantize(packed: torch.Tensor, norms: torch.Tensor, qjl_term: torch.Tensor,
                    residual_norms: torch.Tensor, dim: int, padded_dim: int, mse_bit_width: int,
                    signs: torch.Tensor, centroids) -> torch.Tensor:
    """TurboQuantProd.dequantize on the GPU (tq_prod_dequantize): the MSE
    read-back plus qjl_term * (sqrt(pi/2) / dim * residual_norms), qjl_term
    being z S (fp32 [..., dim])."""
    _require_gpu(packed, norms, qjl_term, residual_norms, signs)
    per = 2 if mse_bit_width == 3 else 8 // mse_bit_width
    if packed.dtype != torch.uint8 or packed.shape[-1] != padded_dim // per:
        raise RuntimeError("prod_dequantize: packed must be uint8 [..., padded_dim / per]")
    lead = tuple(packed.shape[:-1])
    if tuple(norms.shape) != lead or tuple(residual_norms.shape) != lead:
        raise RuntimeError("prod_dequantize: norms must match packed's leading dims")
    if tuple(qjl_term.shape) != (*lead, dim):
        raise RuntimeError("prod_dequantize: qjl_term must be [..., dim]")
    packed = packed.contiguous()
    if packed.data_ptr() % 16:
        packed = packed.clone()
    nf = norms.to(torch.float32).contiguous()
    rn = residual_norms.to(torch.float32).contiguous()
    qt = qjl_term.to(torch.float32).contiguous()
    out = torch.empty((*lead, dim), dtype=torch.float32, device=packed.device)
    signs = _aligned16(signs)
    lib = _lib.load()
    with torch.cuda.device(packed.device):
        rc = lib.tq_prod_dequantize(packed.data_ptr(), nf.data_ptr(), qt.data_ptr(),
                                    rn.data_ptr(), nf.numel(), int(dim), int(padded_dim),
                                    int(mse_bit_width), signs.data_ptr(), _host_f32(centroids),
                                    out.data_ptr(), _stream_ptr(packed.device))
    _lib.check(rc, "prod_dequantize")
    return out


def prod_quantize_qjl(x: torch.Tensor, padded_dim: int, mse_bit_width: int,
                      signs: torch.Tensor, boundaries, centroids, s_hi: torch.Tensor,
                      s_lo: torch.Tensor):
    """TurboQuantProd.quantize with the QJL product fused (tq_prod_quantize_qjl,
    padded_dim 64 or 128): x fp32 [..., dim] -> (packed, norms, qjl_signs int8
    [..., dim], residual_norms).  s_hi / s_lo: fp16 [padded_dim, padded_dim]
    halves of the QJL matrix."""
    _require_gpu(x, signs, s_hi, s_lo)
    if x.dtype != torch.float32:
        raise RuntimeError("prod_quantize_qjl: x must be fp32")
    for t in (s_hi, s_lo):
        if t.dtype != torch.float16 or tuple(t.shape) != (padded_dim, padded_dim) \
                or not t.is_contiguous() or t.data_ptr() % 16:
            raise RuntimeError("prod_quantize_qjl: S halves must be contiguous aligned fp16 "
                               "[padded_dim, padded_dim]")
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    dim = x.shape[-1]
    lead = x.shape[:-1]
    n = x.numel() // dim if dim else 0
    per = 2 if mse_bit_width == 3 else 8 // mse_bit_width
    packed = torch.empty((*lead, padded_dim // per), dtype=torch.uint8, device=x.device)
    norms = torch.empty(lead, dtype=torch.float32, device=x.device)
    z = torch.empty((*lead, dim), dtype=torch.int8, device=x.device)
    rnorm = torch.empty(lead, dtype=torch.float32, device=x.device)
    signs = _aligned16(signs)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.tq_prod_quantize_qjl(x.data_ptr(), n, dim, int(padded_dim), int(mse_bit_width),
                                      signs.data_ptr(), _host_f32(boundaries),
                                      _host_f32(centroids), s_hi.data_ptr(), s_lo.data_ptr(),
                                      packed.data_ptr(), norms.data_ptr(), z.data_ptr(),
                                      rnorm.data_ptr(), _stream_ptr(x.device))
    _lib.check(rc, "prod_quantize_qjl")
    return packed, norms, z, rnorm


def prod_dequantize_qjl(packed: torch.Tensor, norms: torch.Tensor, qjl_signs: torch.Tensor,
                        residual_norms: torch.Tensor, dim: int, padded_dim: int,
                        mse_bit_width: int, signs: torch.Tensor, centroids,
                        st_hi: torch.Tensor, st_lo: torch.Tensor) -> torch.Tensor:
    """TurboQuantProd.dequantize with z S formed in-kernel
    (tq_prod_dequantize_qjl, padded_dim 64 or 128).  st_hi / st_lo: fp16
    halves of S^T."""
    _require_gpu(packed, norms, qjl_signs, residual_norms, signs, st_hi, st_lo)
    per = 2 if mse_bit_width == 3 else 8 // mse_bit_width
    if packed.dtype != torch.uint8 or packed.shape[-1] != padded_dim // per:
        raise RuntimeError("prod_dequantize_qjl: packed must be uint8 [..., padded_dim / per]")
    lead = tuple(packed.shape[:-1])
    if tuple(norms.shape) != lead or tuple(residual_norms.shape) != lead:
        raise RuntimeError("prod_dequantize_qjl: norms must match packed's leading dims")
    if qjl_signs.dtype != torch.int8 or tuple(qjl_signs.shape) != (*lead, dim):
        raise RuntimeError("prod_dequantize_qjl: qjl_signs must be int8 [..., dim]")
    for t in (st_hi, st_lo):
        if t.dtype != torch.float16 or tuple(t.shape) != (padded_dim, padded_dim) \
                or not t.is_contiguous() or t.data_ptr() % 16:
            raise RuntimeError("prod_dequantize_qjl: S^T halves must be contiguous aligned "
                               "fp16 [padded_dim, padded_dim]")
    packed = packed.contiguous()
    if packed.data_ptr() % 16:
        packed = packed.clone()
    nf = norms.to(torch.float32).contiguous()
    rn = residual_norms.to(torch.float32).contiguous()
    z = _aligned16(qjl_signs)
    out = torch.empty((*lead, dim), dtype=torch.float32, device=packed.device)
    signs = _aligned16(signs)
    lib = _lib.load()
    with torch.cuda.device(packed.device):
        rc = lib.tq_prod_dequantize_qjl(packed.data_ptr(), nf.data_ptr(), z.data_ptr(),
                                        rn.data_ptr(), nf.numel(), int(dim), int(padded_dim),
                                        int(mse_bit_width), signs.data_ptr(),
                                        _host_f32(centroids), st_hi.data_ptr(),
                                        st_lo.data_ptr(), out.data_ptr(),
                                        _stream_ptr(packed.device))
    _lib.check(rc, "prod_dequantize_qjl")
    return out


# --------------------------------------------------------------------------
# torch.library registration under the reference's namespaces and schemas
# --------------------------------------------------------------------------
_registered = False
_libs = []


def _reference_paged_splitkv(q, kv_cache, indices, indptr, last_page_len, seq_lens,
                             num_kv_heads, page_size, head_dim, padded_dim, sm_scale,
                             hadamard_signs, qbytes, nbytes, o_ws, max_len, partition_o_ws,
                             partition_lse_ws, request_indices, kv_tile_indices, split_indptr,
                             kv_chunk_size_t, num_splits):
    """Argument adapter for decode_v5_from_cache_paged_splitkv_ws.

    The chunk size is recomputed on the host as ceil(max_len / num_splits),
    the value the reference backend stores in kv_chunk_size_t
    (vllm_backend_fused.py:210-213), so no device tensor is read.
    request_indices / kv_tile_indices / split_indptr are implied by
    (batch, num_splits); last_page_len and nbytes are unused, as in the
    reference op.
    """
    if int(padded_dim) != q.size(-1):
        raise RuntimeError("padded_dim does not match q")
    exp_q, _, _ = entry_bytes(int(head_dim))
    if int(qbytes) != exp_q:
        raise RuntimeError(f"qbytes {qbytes} does not match head_dim {head_dim}")
    if int(max_len) <= 0:
        raise RuntimeError("max_len must be positive")
    if int(num_splits) < 1:
        raise RuntimeError("num_splits must be >= 1")
    cs = -(-int(max_len) // int(num_splits))
    return decode_paged_splitkv(q, kv_cache, indices, indptr, seq_lens, int(num_kv_heads),
                                int(head_dim), int(padded_dim), float(sm_scale), hadamard_signs,
                                o_ws, partition_o_ws, partition_lse_ws, int(num_splits), cs)


def _check_gather_ws(q, num_kv_heads, max_len, qbytes, padded_dim, k_quant_ws, v_quant_ws,
                     k_norms_ws, v_norms_ws, o_ws):
    """The workspace checks of decode_v5_from_cache_ws
    (decode_v5_tc_binding.cu:466-478), kept so that callers sized for the
    reference are accepted or refused alike."""
    b, hq = q.size(0), q.size(1)
    dc = int(padded_dim) // 64
    if int(max_len) <= 0:
        raise RuntimeError("max_len must be positive")
    if tuple(k_quant_ws.shape) != (b, int(num_kv_heads), int(max_len), int(qbytes)):
        raise RuntimeError("k_quant_ws shape mismatch")
    if tuple(v_quant_ws.shape) != tuple(k_quant_ws.shape):
        raise RuntimeError("v_quant_ws shape mismatch")
    if tuple(k_norms_ws.shape) != (b, int(num_kv_heads), int(max_len), dc):
        raise RuntimeError("k_norms_ws shape mismatch")
    if tuple(v_norms_ws.shape) != tuple(k_norms_ws.shape):
        raise RuntimeError("v_norms_ws shape mismatch")
    if tuple(o_ws.shape) != (b, hq, int(padded_dim)):
        raise RuntimeError("o_ws shape mismatch")


def _scratch_f32(t: torch.Tensor, n: int):
    """n fp32 elements at the start of a contiguous caller-owned buffer, or None."""
    if not t.is_contiguous() or t.numel() * t.element_size() < 4 * n or t.data_ptr() % 16:
        return None
    return t.view(-1).view(torch.uint8)[:4 * n].view(torch.float32)


def _from_cache_ws(q, kv_cache, indices, indptr, last_page_len, seq_lens, num_kv_heads,
                   page_size, head_dim, padded_dim, sm_scale, hadamard_signs, qbytes, nbytes,
                   k_quant_ws, v_quant_ws, k_norms_ws, v_norms_ws, o_ws, max_len):
    """decode_v5_from_cache_ws (decode_v5_tc_binding.cu:439-551): the reference
    gathers the pages into contiguous K/V workspaces and runs one unsplit
    kernel.  Here the paged kernel reads the pages directly, so the gather
    workspaces are free; they hold the split partials instead (the op owns
    their contents during the call, as the reference's gather does), which
    keeps the split-KV layout without any allocation.  Tokens are read up to
    min(seq_lens[b], num_splits * kv_chunk_size) with num_splits *
    kv_chunk_size >= max_len."""
    from .geometry import CHUNK_ALIGN, choose_splits
    _check_gather_ws(q, num_kv_heads, max_len, qbytes, padded_dim, k_quant_ws, v_quant_ws,
                     k_norms_ws, v_norms_ws, o_ws)
    b, hq, pd = q.size(0), q.size(1), int(padded_dim)
    splits, chunk = choose_splits(b, int(max_len), int(num_kv_heads), hq, pd)
    while True:
        po = _scratch_f32(k_quant_ws, b * splits * hq * pd)
        pl = _scratch_f32(v_quant_ws, b * splits * hq)
        if (po is not None and pl is not None) or splits == 1:
            break
        splits = max(1, splits // 2)
        chunk = -(-int(max_len) // splits)
        chunk = (chunk + CHUNK_ALIGN - 1) // CHUNK_ALIGN * CHUNK_ALIGN
        splits = -(-int(max_len) // chunk)
    if po is None or pl is None:
        raise RuntimeError("decode_v5_from_cache_ws: workspaces too small for the partials")
    return decode_paged_splitkv(q, kv_cache, indices, indptr, seq_lens, int(num_kv_heads),
                                int(head_dim), pd, float(sm_scale), hadamard_signs, o_ws, po,
                                pl, splits, chunk)


def _from_cache_splitkv_ws(q, kv_cache, indices, indptr, last_page_len, seq_lens, num_kv_heads,
                           page_size, head_dim, padded_dim, sm_scale, hadamard_signs, qbytes,
                           nbytes, k_quant_ws, v_quant_ws, k_norms_ws, v_norms_ws, o_ws, max_len,
                           partition_o_ws, partition_lse_ws, request_indices, kv_tile_indices,
                           split_indptr, kv_chunk_size_t, num_splits):
    """decode_v5_from_cache_splitkv_ws (decode_v5_tc_binding.cu:586-752): the
    gather-then-split variant.  The paged kernel needs no gather, so this is
    the paged split op with the caller's partition workspaces."""
    _check_gather_ws(q, num_kv_heads, max_len, qbytes, padded_dim, k_quant_ws, v_quant_ws,
                     k_norms_ws, v_norms_ws, o_ws)
    return _reference_paged_splitkv(q, kv_cache, indices, indptr, last_page_len, seq_lens,
                                    num_kv_heads, page_size, head_dim, padded_dim, sm_scale,
                                    hadamard_signs, qbytes, nbytes, o_ws, max_len, partition_o_ws,
                                    partition_lse_ws, request_indices, kv_tile_indices,
                                    split_indptr, kv_chunk_size_t, num_splits)


def decode_v5_from_cache(q, kv_cache, indices, indptr, last_page_len, seq_lens, num_kv_heads,
                         page_size, head_dim, padded_dim, sm_scale, hadamard_signs, qbytes,
                         nbytes):
    """The eager decode_v5_from_cache (decode_v5_tc_binding.cu:324-423): it
    allocates its own output and workspaces (not graph-capturable, as in the
    reference).  max_len is seq_lens.max(), as the reference computes it
    (decode_v5_tc_binding.cu:350); the op is eager, so this host read is
    allowed.  A CSR indptr whose later rows are longer than the first is
    covered."""
    from .geometry import choose_splits
    b, hq, pd = q.size(0), q.size(1), int(padded_dim)
    max_len = int(seq_lens[:b].max()) if b else 0
    max_len = max(max_len, int(page_size))
    splits, chunk = choose_splits(b, max_len, int(num_kv_heads), hq, pd)
    o = torch.empty((b, hq, pd), dtype=torch.float16, device=q.device)
    po = torch.empty((b * splits, hq, pd), dtype=torch.float32, device=q.device)
    pl = torch.empty((b * splits, hq), dtype=torch.float32, device=q.device)
    return decode_paged_splitkv(q, kv_cache, indices, indptr, seq_lens, int(num_kv_heads),
                                int(head_dim), pd, float(sm_scale), hadamard_signs, o, po, pl,
                                splits, chunk)


def _balanced_ws(q, kv_cache, indices, indptr, seq_lens, num_kv_heads, head_dim, padded_dim,
                 sm_scale, hadamard_signs, o_ws, partition_o_ws, partition_lse_ws,
                 split_indptr) -> None:
    """turboquant_v5::decode_paged_balanced_ws: decode_paged_balanced, its
    result in o_ws (the schema returns nothing)."""
    decode_paged_balanced(q, kv_cache, indices, indptr, seq_lens, num_kv_heads, head_dim,
                          padded_dim, sm_scale, hadamard_signs, o_ws, partition_o_ws,
                          partition_lse_ws, split_indptr)


def _register_fakes() -> None:
    """Meta ("fake") kernels, so that torch.compile and vLLM's graph capture
    can trace the ops without running them: the write mutates its cache
    argument and returns nothing; the reference's decode ops return a tensor
    shaped like o_ws (fp16 [B, Hq, padded_dim]); the balanced op writes
    o_ws, which its schema marks, and returns nothing."""
    from torch.library import register_fake

    @register_fake("turboquant_write::quantize_write_kv_cache", lib=_libs[0])
    def _write_fake(kv_cache, key, value, signs, slot_mapping, head_dim, padded_dim):
        return None

    def _decode_fake(q, kv_cache, *args):
        return q.new_empty((q.size(0), q.size(1), q.size(2)), dtype=torch.float16)

    for name in ("decode_v5_from_cache_paged_splitkv_ws", "decode_v5_from_cache_ws",
                 "decode_v5_from_cache_splitkv_ws"):
        register_fake(f"turboquant_v5::{name}", _decode_fake, lib=_libs[1])

    @register_fake("turboquant_v5::decode_paged_balanced_ws", lib=_libs[1])
    def _balanced_fake(q, kv_cache, indices, indptr, seq_lens, num_kv_heads, head_dim,
                       padded_dim, sm_scale, hadamard_signs, o_ws, partition_o_ws,
                       partition_lse_ws, split_indptr):
        return None


def register_ops() -> None:
    """Define turboquant_write::* and turboquant_v5::* with the reference
    schemas and bind the HIP implementations to the CUDA dispatch key."""
    global _registered
    if _registered:
        return
    from torch.library import Library
    w = Library("turboquant_write", "DEF")
    w.define("quantize_write_kv_cache(Tensor(a!) kv_cache, Tensor key, Tensor value, "
             "Tensor signs, Tensor slot_mapping, int head_dim, int padded_dim) -> ()")
    w.impl("quantize_write_kv_cache", quantize_write_kv_cache, "CUDA")
    d = Library("turboquant_v5", "DEF")
    d.define("decode_v5_from_cache_paged_splitkv_ws(Tensor q, Tensor kv_cache, "
             "Tensor indices, Tensor indptr, Tensor last_page_len, Tensor seq_lens, "
             "int num_kv_heads, int page_size, int head_dim, int padded_dim, "
             "float sm_scale, Tensor hadamard_signs, int qbytes, int nbytes, "
             "Tensor o_ws, int max_len, "
             "Tensor partition_o_ws, Tensor partition_lse_ws, "
             "Tensor request_indices, Tensor kv_tile_indices, "
             "Tensor split_indptr, Tensor kv_chunk_size_t, int num_splits) -> Tensor")
    d.impl("decode_v5_from_cache_paged_splitkv_ws", _reference_paged_splitkv, "CUDA")
    d.define("decode_v5_from_cache_ws(Tensor q, Tensor kv_cache, Tensor indices, "
             "Tensor indptr, Tensor last_page_len, Tensor seq_lens, "
             "int num_kv_heads, int page_size, int head_dim, int padded_dim, "
             "float sm_scale, Tensor hadamard_signs, int qbytes, int nbytes, "
             "Tensor k_quant_ws, Tensor v_quant_ws, Tensor k_norms_ws, "
             "Tensor v_norms_ws, Tensor o_ws, int max_len) -> Tensor")
    d.impl("decode_v5_from_cache_ws", _from_cache_ws, "CUDA")
    d.define("decode_v5_from_cache_splitkv_ws(Tensor q, Tensor kv_cache, Tensor indices, "
             "Tensor indptr, Tensor last_page_len, Tensor seq_lens, "
             "int num_kv_heads, int page_size, int head_dim, int padded_dim, "
             "float sm_scale, Tensor hadamard_signs, int qbytes, int nbytes, "
             "Tensor k_quant_ws, Tensor v_quant_ws, Tensor k_norms_ws, "
             "Tensor v_norms_ws, Tensor o_ws, int max_len, "
             "Tensor partition_o_ws, Tensor partition_lse_ws, "
             "Tensor request_indices, Tensor kv_tile_indices, "
             "Tensor split_indptr, Tensor kv_chunk_size_t, int num_splits) -> Tensor")
    d.impl("decode_v5_from_cache_splitkv_ws", _from_cache_splitkv_ws, "CUDA")
    # this build's balanced-split decode (no reference counterpart: the
    # reference plans splits on the host from max_len)
    # it writes its result into o_ws, and the partial rows, LSEs and row table
    # into the other workspaces, and says so in its schema (returning
    # nothing: functionalization refuses aliased outputs of custom ops), so
    # functionalization and torch.compile keep the call and its writes
    d.define("decode_paged_balanced_ws(Tensor q, Tensor kv_cache, Tensor indices, "
             "Tensor indptr, Tensor seq_lens, int num_kv_heads, int head_dim, "
             "int padded_dim, float sm_scale, Tensor hadamard_signs, Tensor(a!) o_ws, "
             "Tensor(b!) partition_o_ws, Tensor(c!) partition_lse_ws, "
             "Tensor(d!) split_indptr) -> ()")
    d.impl("decode_paged_balanced_ws", _balanced_ws, "CUDA")
    _libs.extend([w, d])
    _register_fakes()
    _registered = True
