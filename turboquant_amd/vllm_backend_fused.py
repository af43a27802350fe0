"""TurboQuant vLLM attention backend on the MI355X HIP kernels.

Drop-in for reference turboquant/vllm_backend_fused.py:32-468: same classes,
static/class methods, constructor and forward signatures, cache shape and
page-size hook; the kernels behind them are libtq_hip.so.

    LLM(..., attention_backend="CUSTOM", kv_cache_dtype="fp8")

fp8 selects a 1-byte allocation that this backend views as packed 4-bit codes
plus fp16 norms, [2, num_blocks, block_size, num_kv_heads, ebs].

vLLM is imported lazily-optional: when it is absent (unit tests, the CPU
container) minimal stand-in base classes keep the module importable so the
backend can be driven with a metadata object carrying the fields vLLM's
FlashAttentionMetadata provides (max_query_len, num_actual_tokens,
block_table, seq_lens, query_start_loc, slot_mapping).
"""
from __future__ import annotations

import math
import sys
import traceback

import torch
import torch.nn.functional as F

from .decoder_dispatch import KERNEL_NAME, STATIC_KERNEL_NAME
from .decoder_dispatch import _op as _dispatch_op
from .geometry import (BALANCED_MAX_BATCH, QUANT_BYTES_PER_CHUNK, TILE_DIMS, choose_splits,
                       entry_bytes, hadamard_signs, padded_dim)

try:  # pragma: no cover - exercised only where vLLM is installed
    from vllm.v1.attention.backends.flash_attn import (FlashAttentionBackend,
                                                       FlashAttentionImpl,
                                                       FlashAttentionMetadataBuilder)
    HAVE_VLLM = True
except Exception:  # vLLM absent: stand-ins with the pieces this module uses
    HAVE_VLLM = False

    class FlashAttentionBackend:  # type: ignore[no-redef]
        accept_output_buffer = True

        @staticmethod
        def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size,
                               cache_dtype_str="auto"):
            if block_size % 16 != 0:
                raise ValueError("Block size must be a multiple of 16.")
            return (2, num_blocks, block_size, num_kv_heads, head_size)

        @classmethod
        def supports_kv_cache_dtype(cls, kv_cache_dtype) -> bool:
            return kv_cache_dtype in (None, "auto")

    class FlashAttentionImpl:  # type: ignore[no-redef]
        def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes,
                     sliding_window, kv_cache_dtype, *args, **kwargs):
            self.num_heads = num_heads
            self.head_size = head_size
            self.scale = float(scale)
            self.num_kv_heads = num_kv_heads
            self.alibi_slopes = alibi_slopes
            self.sliding_window = sliding_window
            self.kv_cache_dtype = kv_cache_dtype
            self.num_queries_per_kv = num_heads // num_kv_heads

        def forward(self, *args, **kwargs):
            raise NotImplementedError("fp16 KV cache path needs vLLM's FlashAttention")

    class FlashAttentionMetadataBuilder:  # type: ignore[no-redef]
        pass


_FP8 = ("fp8", "fp8_e4m3")


def _next_pow2(n):
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


class TurboQuantBackend(FlashAttentionBackend):
    """Backend "CUSTOM" (vllm_backend_fused.py:32-86)."""

    # vLLM calls do_kv_cache_update separately from forward
    forward_includes_kv_cache_update = False

    @staticmethod
    def get_name():
        return "CUSTOM"

    @staticmethod
    def get_impl_cls():
        return TurboQuantFusedImpl

    @staticmethod
    def get_builder_cls():
        return TurboQuantMetadataBuilder

    @classmethod
    def supports_kv_cache_dtype(cls, kv_cache_dtype) -> bool:
        if kv_cache_dtype in _FP8:
            return True
        return super().supports_kv_cache_dtype(kv_cache_dtype)

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int,
                           head_size: int, cache_dtype_str: str = "auto") -> tuple[int, ...]:
        if cache_dtype_str in _FP8:
            _, _, ebs = entry_bytes(head_size)
            return (2, num_blocks, block_size, num_kv_heads, ebs)
        return FlashAttentionBackend.get_kv_cache_shape(num_blocks, block_size, num_kv_heads,
                                                        head_size, cache_dtype_str)

    @classmethod
    def get_kv_cache_page_size(cls, block_size, num_kv_heads, head_size, dtype,
                               cache_dtype_str="auto"):
        """Bytes of one cache block for vLLM's page-size hook
        (docker/vllm_patches/v1/attention/backend.py:94-113 in the reference)."""
        if cache_dtype_str in _FP8:
            _, _, ebs = entry_bytes(head_size)
            return 2 * block_size * num_kv_heads * ebs
        return None


class TurboQuantMetadataBuilder(FlashAttentionMetadataBuilder):
    pass


class TurboQuantFusedImpl(FlashAttentionImpl):
    """Quantized KV cache with the HIP kernels (vllm_backend_fused.py:93-468).

    Write: do_kv_cache_update -> turboquant_write::quantize_write_kv_cache.
    Decode: forward (max_query_len == 1) -> turboquant_v5::decode_paged_balanced_ws
            (split plan made on the GPU from seq_lens), or the reference's
            turboquant_v5::decode_v5_from_cache_paged_splitkv_ws with
            TQ_FORCE_KERNEL=gfx950_static.
    Prefill / mixed batches: _prefill_mixed (decode rows through the decode
    kernel, chunks with cached context over the dequantized context plus the
    fresh chunk, fresh prompts as in the reference, vllm_backend_fused.py:335-371).
    """

    def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes,
                 sliding_window, kv_cache_dtype, *args, **kwargs):
        self._real_cache_dtype = kv_cache_dtype
        parent_dtype = "auto" if kv_cache_dtype in _FP8 else kv_cache_dtype
        super().__init__(num_heads, head_size, scale, num_kv_heads, alibi_slopes,
                         sliding_window, parent_dtype, *args, **kwargs)
        self.kv_cache_dtype = self._real_cache_dtype
        self._pd = padded_dim(self.head_size)
        self._dc = self._pd // TILE_DIMS
        self._qbytes = self._dc * QUANT_BYTES_PER_CHUNK
        self._nbytes = self._dc * 2
        self._signs = None
        self._is_fp8 = kv_cache_dtype in _FP8
        # (batch_size, max_pages_per_seq) -> workspace tensors
        self._v5_ws_cache: dict[tuple[int, int], dict] = {}
        self._decode_op = None
        self._decode_op_name = None
        self._write_op = None

    # ---------------------------------------------------------------- setup
    @staticmethod
    def _choose_num_splits(batch_size: int, max_len: int, num_kv_heads: int,
                           device: torch.device | None = None) -> int:
        return choose_splits(batch_size, max_len, num_kv_heads)[0]

    def _get_v5_ws(self, batch_size: int, max_pages: int, block_size: int,
                   device: torch.device, op_name: str | None = None):
        """Workspace keyed by (batch_size, max_pages) as in the reference
        (vllm_backend_fused.py:158-215): allocated on the first call of a
        shape bucket (vLLM warm-up), reused by graph replays.  op_name: the
        op the workspace is for (default: the dispatched one).
        Returns (ws, max_len, num_splits)."""
        op_name = op_name or self._decode_op_name
        key = (batch_size, max_pages, op_name)
        max_len = max_pages * block_size
        ws = self._v5_ws_cache.get(key)
        if ws is None and op_name == KERNEL_NAME:
            # balanced plan: rows for the resident workgroup slots, the row
            # table written by the kernel
            from .ops import balanced_rows
            rows = balanced_rows(batch_size, self.num_heads, self.num_kv_heads, self._pd,
                                 device)
            ws = {
                "o": torch.empty((batch_size, self.num_heads, self._pd), dtype=torch.float16,
                                 device=device),
                "num_splits": 0,
                "partition_o": torch.empty((rows, self.num_heads, self._pd),
                                           dtype=torch.float32, device=device),
                "partition_lse": torch.empty((rows, self.num_heads), dtype=torch.float32,
                                             device=device),
                "split_indptr": torch.zeros(batch_size + 2, dtype=torch.int32, device=device),
            }
            self._v5_ws_cache[key] = ws
        if ws is None:
            num_splits, chunk = choose_splits(batch_size, max_len, self.num_kv_heads,
                                             self.num_heads, self._pd)
            padded_batch = batch_size * num_splits
            arange = torch.arange(padded_batch, dtype=torch.int32, device=device)
            ws = {
                "o": torch.empty((batch_size, self.num_heads, self._pd), dtype=torch.float16,
                                 device=device),
                "num_splits": num_splits,
                "partition_o": torch.empty((padded_batch, self.num_heads, self._pd),
                                           dtype=torch.float32, device=device),
                "partition_lse": torch.empty((padded_batch, self.num_heads),
                                             dtype=torch.float32, device=device),
                "request_indices": (arange // num_splits).to(torch.int32),
                "kv_tile_indices": (arange % num_splits).to(torch.int32),
                "split_indptr": torch.arange(batch_size + 1, dtype=torch.int32,
                                             device=device) * num_splits,
                # ceil(max_len / num_splits); the op recomputes it on the host
                "kv_chunk_size": torch.tensor([-(-max_len // num_splits)], dtype=torch.int32,
                                              device=device),
            }
            self._v5_ws_cache[key] = ws
        return ws, max_len, ws["num_splits"]

    def _ensure(self, dev):
        if self._signs is not None:
            return
        self._signs = hadamard_signs(self._pd, device=dev)

    # torch forms of the rotation the kernels apply (the reference keeps the
    # same helpers on its impl, vllm_backend_fused.py:227-252; its forward
    # does not call them either)
    @staticmethod
    def _fwht(x):
        """Unnormalised Walsh-Hadamard transform along the last dim."""
        from .algorithm import fwht_unnormalized
        return fwht_unnormalized(x)

    def _hadamard_forward(self, q):
        """q' = H (s * q) / sqrt(pd), computed in fp32, returned in q's dtype."""
        self._ensure(q.device)
        x = self._fwht(q.float() * self._signs.to(q.device))
        return (x * (1.0 / math.sqrt(x.shape[-1]))).to(q.dtype)

    def _hadamard_inverse(self, out):
        """o = s * (H o' / sqrt(pd)), the inverse of _hadamard_forward."""
        self._ensure(out.device)
        x = self._fwht(out.float()) * (1.0 / math.sqrt(out.shape[-1]))
        return (x * self._signs.to(out.device)).to(out.dtype)

    def _ensure_kernels_loaded(self):
        if self._decode_op is None or self._write_op is None:
            from . import ops
            from .decoder_dispatch import pick_decode_op
            ops.register_ops()
            self._write_op = torch.ops.turboquant_write.quantize_write_kv_cache
            self._decode_op, self._decode_op_name = pick_decode_op()

    # ---------------------------------------------------------------- write
    def _write_to_cache(self, key, value, kv_cache, slot_mapping):
        num_tokens = slot_mapping.shape[0]
        self._ensure_kernels_loaded()
        sm = slot_mapping if slot_mapping.dtype == torch.int32 else slot_mapping.to(torch.int32)
        # fp16/bf16/fp32 rows go in as they are (the kernel converts exactly);
        # the reference's .float() copy is not needed
        self._write_op(kv_cache, key[:num_tokens], value[:num_tokens], self._signs, sm,
                       self.head_size, self._pd)

    @torch.no_grad()
    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        self._ensure(key.device)
        if self._is_fp8:
            self._write_to_cache(key, value, kv_cache, slot_mapping)
        else:  # pragma: no cover - needs vLLM
            from vllm.v1.attention.backends.fa_utils import reshape_and_cache_flash
            num_tokens = slot_mapping.shape[0]
            key_cache, value_cache = kv_cache.unbind(0)
            reshape_and_cache_flash(key[:num_tokens], value[:num_tokens], key_cache,
                                    value_cache, slot_mapping, self.kv_cache_dtype,
                                    layer._k_scale, layer._v_scale)

    # -------------------------------------------------------------- forward
    @staticmethod
    def _host_boundaries(attn_metadata):
        """query_start_loc and seq_lens as host lists: the metadata's own CPU
        copies when it carries them (vLLM's query_start_loc_cpu /
        seq_lens_cpu), else one device-to-host copy of both together."""
        qsl = getattr(attn_metadata, "query_start_loc_cpu", None)
        seq = getattr(attn_metadata, "seq_lens_cpu", None)
        if qsl is not None and (seq is not None or attn_metadata.seq_lens is None):
            return qsl.tolist(), (seq.tolist() if seq is not None else None)
        dq = attn_metadata.query_start_loc
        if attn_metadata.seq_lens is None:
            return dq.cpu().tolist(), None
        n = dq.numel()
        both = torch.cat([dq.to(torch.int64), attn_metadata.seq_lens.to(torch.int64)]).cpu()
        return both[:n].tolist(), both[n:].tolist()

    def _attend(self, q, k, v, ctx, out=None):
        """q [ql, Hq, D] over k, v [ctx + ql, Hkv, D] (fp16), causal with the
        queries at the end of the keys (lower-right alignment), in this
        library's prefill kernel (tq_prefill_attention).  Head sizes 64, 128
        and 256 run as they are, written into `out` when given (fp16
        [ql, Hq, D]); a head size below its padded size (96, 80, ...) runs
        zero-padded to it: zero dims add nothing to q.k and give zero output
        dims, which are dropped.  The reference runs flash-attn here for
        every head size (vllm_backend_fused.py:335-371)."""
        from . import ops
        d, pd = self.head_size, self._pd
        if pd > 256:
            raise RuntimeError(f"prefill: head_size {d} unsupported (padded size {pd} > 256)")
        if d == pd:
            if out is None or out.dtype != torch.float16:
                out = torch.empty(q.shape, dtype=torch.float16, device=q.device)
            return ops.prefill_attention(q, k, v, out, self.scale)
        pad = (0, pd - d)
        qp, kp, vp = F.pad(q, pad), F.pad(k, pad), F.pad(v, pad)
        op = torch.empty(qp.shape, dtype=torch.float16, device=q.device)
        ops.prefill_attention(qp, kp, vp, op, self.scale)
        return op[:, :, :d]

    def _prefill_fresh(self, query, key, value, attn_metadata, output):
        """Causal attention of each prompt chunk over its own fresh K/V."""
        qsl, _ = self._host_boundaries(attn_metadata)
        for i in range(len(qsl) - 1):
            a, b = qsl[i], qsl[i + 1]
            if b <= a:
                continue
            dst = output[a:b]
            o = self._attend(query[a:b].to(torch.float16), key[a:b].to(torch.float16),
                             value[a:b].to(torch.float16), 0, dst)
            if o.data_ptr() != dst.data_ptr():
                dst.copy_(o)
        return output

    def _decode_ws(self, n, pages, device):
        """Balanced-decode workspace for n decode rows of a mixed batch."""
        key = ("mixed", n, pages)
        ws = self._v5_ws_cache.get(key)
        if ws is None:
            from .ops import balanced_rows
            rows = balanced_rows(n, self.num_heads, self.num_kv_heads, self._pd, device)
            ws = {
                "o": torch.empty((n, self.num_heads, self._pd), dtype=torch.float16,
                                 device=device),
                "partition_o": torch.empty((rows, self.num_heads, self._pd),
                                           dtype=torch.float32, device=device),
                "partition_lse": torch.empty((rows, self.num_heads), dtype=torch.float32,
                                             device=device),
                "split_indptr": torch.zeros(n + 2, dtype=torch.int32, device=device),
                "indptr": torch.arange(n + 1, dtype=torch.int32, device=device) * pages,
            }
            self._v5_ws_cache[key] = ws
        return ws

    def _prefill_mixed(self, query, key, value, kv_cache, attn_metadata, output):
        """A batch with max_query_len > 1 whose cache already holds every token
        of the batch (do_kv_cache_update runs first).  Per request with q_len
        new tokens and seq_len tokens in all, ctx = seq_len - q_len:

        * q_len == 1 and ctx > 0 (decode rows of a mixed batch): the balanced
          decode kernels over the cache, as in a pure decode batch;
        * ctx == 0 (a fresh prompt): causal attention over the fresh K/V,
          the reference's prefill (vllm_backend_fused.py:335-371);
        * ctx > 0 (a chunk of a longer prompt): the ctx cached tokens read back
          from the quantized cache (tq_dequant_paged) followed by the chunk's
          fresh K/V, causal with the chunk's queries at the end.  The
          reference attends the fresh chunk only and so drops the cached
          context; its decode path already attends over the dequantized
          cache, which this extends to chunks.
        Attention runs in this library's prefill kernel (head sizes 64, 128
        and 256, smaller sizes zero-padded to their padded size; short chunks
        over long contexts split their keys over workgroups).
        """
        from . import ops
        self._ensure_kernels_loaded()
        self._ensure(query.device)
        qsl, seq = self._host_boundaries(attn_metadata)
        bt = attn_metadata.block_table
        dec = []
        for i in range(len(qsl) - 1):
            a, b = qsl[i], qsl[i + 1]
            ql = b - a
            if ql <= 0:
                continue
            ctx = int(seq[i]) - ql
            if ctx < 0:
                raise RuntimeError(f"request {i}: seq_len {seq[i]} < query length {ql}")
            if ql == 1 and ctx > 0:
                dec.append(i)
                continue
            q = query[a:b].to(torch.float16)
            if ctx == 0:
                kk = key[a:b].to(torch.float16)
                vv = value[a:b].to(torch.float16)
            else:
                kk = torch.empty((ctx + ql, self.num_kv_heads, self.head_size),
                                 dtype=torch.float16, device=query.device)
                vv = torch.empty_like(kk)
                pages = bt[i].to(torch.int32).contiguous()
                ops.dequant_paged(kv_cache, pages, ctx, self.num_kv_heads, self.head_size,
                                  self._pd, self._signs, kk, vv)
                kk[ctx:] = key[a:b]
                vv[ctx:] = value[a:b]
            dst = output[a:b]
            o = self._attend(q, kk, vv, ctx, dst)
            if o.data_ptr() != dst.data_ptr():
                dst.copy_(o)
        for c0 in range(0, len(dec), BALANCED_MAX_BATCH):  # a plan takes <= 1024 rows
            self._decode_rows(dec[c0:c0 + BALANCED_MAX_BATCH], qsl, query, kv_cache, bt,
                              attn_metadata, output)
        return output

    def _decode_rows(self, dec, qsl, query, kv_cache, bt, attn_metadata, output):
        """The decode rows `dec` (request indices, q_len 1) of a mixed batch
        through the balanced decode op; at most BALANCED_MAX_BATCH of them."""
        from . import ops
        if dec:
            dev = query.device
            rows = torch.tensor([qsl[i] for i in dec], dtype=torch.long, device=dev)
            idx = torch.tensor(dec, dtype=torch.long, device=dev)
            q = query.index_select(0, rows).to(torch.float16)
            if self.head_size < self._pd:
                q = F.pad(q, (0, self._pd - self.head_size))
            q = q.contiguous()
            sub_bt = bt.index_select(0, idx).to(torch.int32).contiguous()
            sl = attn_metadata.seq_lens.index_select(0, idx).to(torch.int32).contiguous()
            ws = self._decode_ws(len(dec), sub_bt.shape[1], dev)
            o = ops.decode_paged_balanced(q, kv_cache, sub_bt.reshape(-1), ws["indptr"], sl,
                                          self.num_kv_heads, self.head_size, self._pd,
                                          self.scale, self._signs, ws["o"],
                                          ws["partition_o"], ws["partition_lse"],
                                          ws["split_indptr"])
            output.index_copy_(0, rows, o[:, :, :self.head_size].to(output.dtype))
        return output

    @torch.no_grad()
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, **kwargs):
        if attn_metadata is None:
            if output is None:
                output = torch.zeros_like(query)
            return output

        is_decode = attn_metadata.max_query_len == 1
        if not is_decode:
            if self._is_fp8:
                num_tokens = attn_metadata.num_actual_tokens
                if output is None:
                    output = torch.empty_like(query[:num_tokens])
                q = query[:num_tokens].view(num_tokens, self.num_heads, self.head_size)
                k = key[:num_tokens].view(num_tokens, self.num_kv_heads, self.head_size)
                v = value[:num_tokens].view(num_tokens, self.num_kv_heads, self.head_size)
                out3 = output[:num_tokens].view(num_tokens, self.num_heads, self.head_size)
                if kv_cache is None or attn_metadata.seq_lens is None:
                    self._prefill_fresh(q, k, v, attn_metadata, out3)
                else:
                    self._prefill_mixed(q, k, v, kv_cache, attn_metadata, out3)
                return output
            return super().forward(layer, query, key, value, kv_cache, attn_metadata,
                                   output, output_scale, **kwargs)

        num_actual = attn_metadata.num_actual_tokens
        q = query[:num_actual]
        if output is None:
            output = torch.empty_like(q)
        block_table = attn_metadata.block_table
        seq_lens = attn_metadata.seq_lens
        try:
            self._ensure_kernels_loaded()
            if not self._is_fp8:
                return super().forward(layer, query, key, value, kv_cache, attn_metadata,
                                       output, output_scale, **kwargs)
            self._ensure(q.device)
            block_size = kv_cache.shape[2]
            # strided page table (indptr = b * max_pages): static shapes,
            # capturable; the indptr tensor is made once per workspace
            max_pages = block_table.shape[1]
            kv_indices = block_table.reshape(-1)
            if kv_indices.dtype != torch.int32:
                kv_indices = kv_indices.to(torch.int32)
            q3 = q.view(num_actual, self.num_heads, self.head_size)
            q_fp16 = q3.to(torch.float16)
            if self.head_size < self._pd:
                q_fp16 = F.pad(q_fp16, (0, self._pd - self.head_size))
            batch_size = q_fp16.shape[0]
            # the balanced plan takes up to BALANCED_MAX_BATCH sequences; a
            # larger decode batch takes the reference's static-split op (same
            # kernels, host-planned splits)
            balanced = (self._decode_op_name == KERNEL_NAME
                        and batch_size <= BALANCED_MAX_BATCH)
            op_name = (self._decode_op_name if balanced or self._decode_op_name != KERNEL_NAME
                       else STATIC_KERNEL_NAME)
            decode_op = (self._decode_op if op_name == self._decode_op_name
                         else _dispatch_op(STATIC_KERNEL_NAME))
            ws, max_len, num_splits = self._get_v5_ws(batch_size, max_pages, block_size,
                                                      q.device, op_name)
            kv_indptr = ws.get("indptr")
            if kv_indptr is None:
                kv_indptr = ws["indptr"] = torch.arange(
                    batch_size + 1, dtype=torch.int32, device=q.device) * max_pages
            sl = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
            out3 = output[:num_actual].view(num_actual, self.num_heads, self.head_size)
            # the kernel writes the caller's output directly when it has the
            # op's layout (fp16, contiguous, head_size == padded_dim)
            direct = (self.head_size == self._pd and out3.dtype == torch.float16
                      and out3.is_contiguous())
            o_ws = out3 if direct else ws["o"]
            if balanced:
                # the op writes o_ws (declared in its schema) and returns nothing
                decode_op(
                    q_fp16, kv_cache, kv_indices, kv_indptr, sl, self.num_kv_heads,
                    self.head_size, self._pd, self.scale, self._signs, o_ws,
                    ws["partition_o"], ws["partition_lse"], ws["split_indptr"])
                result = o_ws
            else:
                num_pages = (seq_lens + block_size - 1) // block_size
                kv_last_page_len = seq_lens - (num_pages - 1) * block_size
                result = decode_op(
                    q_fp16, kv_cache, kv_indices, kv_indptr, kv_last_page_len, sl,
                    self.num_kv_heads, block_size, self.head_size, self._pd, self.scale,
                    self._signs, self._qbytes, self._nbytes, o_ws, max_len,
                    ws["partition_o"], ws["partition_lse"], ws["request_indices"],
                    ws["kv_tile_indices"], ws["split_indptr"], ws["kv_chunk_size"], num_splits)
            # the reference's op returns its result (o_ws itself when run
            # eagerly, so no copy then; its schema declares no write)
            if direct:
                if result.data_ptr() != out3.data_ptr():
                    out3.copy_(result[:num_actual])
            else:
                if self.head_size < self._pd:
                    out3.copy_(result[:num_actual, :, :self.head_size])
                else:
                    out3.copy_(result[:num_actual])
        except Exception as e:
            print(f"[TQ] Decode kernel failed: {e}", file=sys.stderr, flush=True)
            traceback.print_exc(file=sys.stderr)
            # an fp8 (packed) cache cannot be read by anything else: re-raise
            if self._is_fp8:
                raise
            return super().forward(layer, query, key, value, kv_cache, attn_metadata, output,
                                   output_scale, **kwargs)
        return output
