"""Decode-attention throughput on the packed TurboQuant KV cache (MI355X).

Headline workload (Qwen3-8B geometry): q fp16 [8, 32, 128],
8 sequences x 32768 cached tokens, 8 KV heads, head_dim 128, 16-token pages
assigned by a seeded random permutation of a 16384-page pool, split-KV + LSE
merge.  One step = one decode-attention call (partials kernel + combine
kernel) over the resident cache, through the op the vLLM backend calls
(turboquant_v5::decode_paged_balanced_ws: split plan made on the GPU).

Also measured, as fields of the same line: configs[3] ragged batches (B=64,
L ~ U[1024, 32768], Student-t K) at head sizes 64/128/256 with the balanced
plan and with the reference's max_len-based splits; configs[4] end to end
(random-init Qwen3-8B architecture, 8 x 32768-token prompts, 256 output
tokens, through TurboQuantFusedImpl); the write kernel on configs[1]; the
context read-back kernel; the prefill attention kernel (one 32k-token
causal prompt, beside torch's flash kernel) and a chunked-prefill call
through the backend; and the CPU baseline (a torch-CPU fp32 port of the
reference's PyTorch path, oracle/torch_ref.py) on the host cores.

Prints ONE JSON line.  value = algorithmic bytes per step / step time, where
algorithmic bytes = codes + norms of every (token, kv head, K|V) + page-table
entries + q + o (285,409,280 B at this shape).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the partials kernel at configs[2] (512 rows of 512
# tokens), from rocprofv3 FETCH_SIZE (x2.0) + WRITE_SIZE (x1.0), each scale
# taken from a 256 MiB device copy (profiles/decode_partials_cfg3_hbm_traffic.md);
# keyed by (op, num_splits, kv_chunk_size) so an overridden layout reports null.
PROFILED_TRAFFIC = {("balanced", 64, 512): 342079000, ("static", 64, 512): 342252000}
TRAFFIC_SOURCE = ("profiled constant: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this kernel at "
                  "this layout, profiles/decode_partials_cfg3_hbm_traffic.md")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_decode_workload(torch, batch=8, seq_len=32768, hq=32, hkv=8, hd=128, seed=3):
    """Device-resident cfg-3 workload; K/V written by the HIP write kernel."""
    from turboquant_amd import ops
    from turboquant_amd.geometry import choose_splits, entry_bytes, hadamard_signs
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(seed)
    pd = hd
    _, _, ebs = entry_bytes(hd)
    pages_per_seq = seq_len // 16
    nb = batch * pages_per_seq
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = perm.view(batch, pages_per_seq).to(dev)
    cache = torch.zeros((2, nb, 16, hkv, ebs), dtype=torch.uint8, device=dev)
    signs = hadamard_signs(pd, dev)
    gd = torch.Generator(device=dev).manual_seed(seed)
    chunk = 8192
    t_all = torch.arange(seq_len, device=dev, dtype=torch.int32)
    for b in range(batch):
        for t0 in range(0, seq_len, chunk):
            t = t_all[t0:t0 + chunk]
            slots = (bt[b, t // 16] * 16 + t % 16).to(torch.int32)
            k = torch.randn((len(t), hkv, hd), generator=gd, device=dev).half()
            v = torch.randn((len(t), hkv, hd), generator=gd, device=dev).half()
            ops.quantize_write_kv_cache(cache, k, v, signs, slots, hd, pd)
    q = torch.randn((batch, hq, pd), generator=gd, device=dev).half()
    seq = torch.full((batch,), seq_len, dtype=torch.int32, device=dev)
    indices = bt.reshape(-1).contiguous()
    indptr = (torch.arange(batch + 1, dtype=torch.int32, device=dev) * pages_per_seq)
    splits, cs = choose_splits(batch, seq_len, hkv, hq, pd)
    torch.cuda.synchronize()
    return dict(cache=cache, q=q, seq=seq, indices=indices, indptr=indptr, bt=bt, signs=signs,
                splits=splits, cs=cs, nb=nb, ebs=ebs, pd=pd, hd=hd, hq=hq, hkv=hkv,
                batch=batch, seq_len=seq_len)


def alg_bytes(w):
    per = w["pd"] // 2 + 2 * (w["pd"] // 64)
    b, L = w["batch"], w["seq_len"]
    return b * L * w["hkv"] * 2 * per + b * math.ceil(L / 16) * 4 + 2 * b * w["hq"] * w["pd"] * 2


# The GPU leaves its idle clocks only after ~25 ms of continuous work: the
# first ~300 decode steps after an idle gap run at 68-86 us against 65 us
# settled.  Every timed leg therefore first keeps the GPU busy for SETTLE_S
# with untimed calls of the same work, on top of the --warmup steps.
SETTLE_S = 0.1


def settle(torch, fn, seconds=SETTLE_S):
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_launches(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    settle(torch, fn)
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps  # ms


def time_graph(torch, fn, steps, warmup, per_graph=10):
    """Per-call time of `fn` replayed from a captured HIP graph of `per_graph`
    calls (how vLLM runs the decode), so host launch overhead stays outside
    the timed region: HIP events on the replay stream around ceil(steps /
    per_graph) replays."""
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        for _ in range(max(1, warmup)):
            fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        for _ in range(per_graph):
            fn()
    reps = max(1, -(-steps // per_graph))
    with torch.cuda.stream(st):
        for _ in range(max(1, warmup // per_graph)):
            g.replay()
        settle(torch, g.replay)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(reps):
            g.replay()
        e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * per_graph)  # ms


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _median_time(fn, runs=5):
    fn()  # warm-up run
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(torch, w):
    """The reference's PyTorch path restated in torch on the CPU
    (oracle/torch_ref.py, fp32): decode = dequantize, rotate q, GQA softmax
    attention per (sequence, kv head), inverse rotation
    (turboquant/triton_decode_ref.py:89-131, 264-299), timed on a bounded
    sample of the configs[2] workload (one of the 8 sequences, all heads);
    write = the configs[1] write as whole-tensor torch ops.  One warm-up run,
    then the median of 5, on the host cores in this process."""
    from oracle import torch_ref
    from turboquant_amd import workloads as W
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    cache = w["cache"].cpu()
    q = w["q"][:1].cpu()
    bt = w["bt"][:1].cpu()
    signs = w["signs"].cpu()
    L = w["seq_len"]
    seq = torch.tensor([L], dtype=torch.int32)
    med, n = _median_time(lambda: torch_ref.decode(q, cache, bt, seq, w["hkv"], w["pd"],
                                                   1.0 / math.sqrt(w["hd"]), signs))
    sample = dict(w, batch=1)
    nbytes = alg_bytes(sample)
    c = W.cfg2()
    shape, pd = W.cache_bytes(c["num_blocks"], 8, 128)
    wcache = torch.zeros(shape, dtype=torch.uint8)
    k, v = torch.from_numpy(c["k"]), torch.from_numpy(c["v"])
    slots = torch.from_numpy(c["slots"])
    wmed, wn = _median_time(lambda: torch_ref.write_kv_cache(wcache, k, v, signs, slots, pd))
    wbytes = W.algorithmic_write_bytes(8192, 8, 128)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "cpu": cpu_model(),
            "sample": f"1 of the 8 configs[2] sequences ({L} tokens, 8 kv heads, 32 q heads; "
                      f"same cache, q, page table), median of {n} runs after one warm-up: "
                      f"{med * 1e3:.1f} ms; oracle/torch_ref.py fp32 torch-CPU port of the "
                      f"reference's dequantize-then-attend, {threads} threads",
            "write": {"value": round(wbytes / wmed / 1e9, 3), "unit": "GB/s",
                      "ms": round(wmed * 1e3, 2),
                      "sample": "configs[1] in full (8192 tokens x 8 heads, K+V), median of "
                                f"{wn} runs after one warm-up"}}


def bench_ragged(torch, steps, warmup):
    """B=64, L ~ U[1024, 32768] (seed 4), K Student-t(3), V N(0,1),
    at head sizes 128 (32q/8kv), 64 (16q/4kv) and 256 (16q/2kv); the balanced
    op against the reference's max_len-based static splits, same cache."""
    import numpy as np

    from turboquant_amd import workloads as W
    from turboquant_amd import ops
    from turboquant_amd.geometry import choose_splits, hadamard_signs
    out = []
    lens = np.random.default_rng(4).integers(1024, 32768 + 1, size=64)
    for hd in (128, 64, 256):
        hq, hkv = {64: (16, 4), 128: (32, 8), 256: (16, 2)}[hd]
        case, cache, pd = W.device_case(4 + 1000 * hd, lens, hq, hkv, hd, k_dist="t3")
        d = W.decode_inputs(case, pd)
        b = len(lens)
        dev = cache.device
        signs = hadamard_signs(pd, dev)
        scale = 1.0 / math.sqrt(hd)
        rows = ops.balanced_rows(b, hq, hkv, pd)
        o = torch.empty((b, hq, pd), dtype=torch.float16, device=dev)
        po = torch.empty((rows, hq, pd), dtype=torch.float32, device=dev)
        pl = torch.empty((rows, hq), dtype=torch.float32, device=dev)
        split = torch.zeros(b + 2, dtype=torch.int32, device=dev)
        ms_b = time_graph(torch, lambda: ops.decode_paged_balanced(
            d["q"], cache, d["indices"], d["indptr"], d["seq"], hkv, hd, pd, scale, signs, o,
            po, pl, split), steps, warmup)
        max_len = case["block_table"].shape[1] * W.BLOCK
        S, cs = choose_splits(b, max_len, hkv, hq, pd)
        po2 = torch.empty((b * S, hq, pd), dtype=torch.float32, device=dev)
        pl2 = torch.empty((b * S, hq), dtype=torch.float32, device=dev)
        ms_s = time_graph(torch, lambda: ops.decode_paged_splitkv(
            d["q"], cache, d["indices"], d["indptr"], d["seq"], hkv, hd, pd, scale, signs, o,
            po2, pl2, S, cs), steps, warmup)
        nbytes = W.algorithmic_decode_bytes(lens, hkv, hd, hq)
        gbs = nbytes / (ms_b * 1e-3) / 1e9
        out.append({"head_dim": hd, "batch": b, "qo_heads": hq, "kv_heads": hkv,
                    "tokens": int(lens.sum()), "alg_bytes": nbytes,
                    "balanced_us": round(ms_b * 1e3, 2), "GB/s": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4), "unit_tokens": int(split[b + 1]),
                    "static_us": round(ms_s * 1e3, 2),
                    "static_GB/s": round(nbytes / (ms_s * 1e-3) / 1e9, 1),
                    "static_splits": [S, cs]})
        log(f"ragged hd={hd}: balanced {ms_b * 1e3:.1f} us ({gbs:.0f} GB/s), static "
            f"max_len splits {ms_s * 1e3:.1f} us")
        del cache, d, po, pl, po2, pl2
        torch.cuda.empty_cache()
    return out


def bench_e2e(torch, compare_steps=16):
    """random-init Qwen3-8B architecture (fp16), 8 random prompts
    of 32768 tokens, 256 output tokens each, every attention through
    TurboQuantFusedImpl (turboquant_amd/e2e.py)."""
    from turboquant_amd import e2e
    res = e2e.run(e2e.ModelShape.qwen3_8b(), batch=8, prompt_len=32768, new_tokens=256,
                  seed=0, compare_steps=compare_steps, log=log)
    res.pop("first_tokens", None)
    res = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in res.items()}
    res["config"] = ("configs[4]: random-init Qwen3-8B architecture fp16 (36 layers, hidden "
                     "4096, 32q/8kv/128, MLP 12288, vocab 151936), 8 prompts x 32768 random "
                     "tokens, 256 output tokens, concurrency 8, prefill one prompt at a time, "
                     "decode steps replayed from one HIP graph")
    torch.cuda.empty_cache()
    return res


def bench_write(torch, steps, warmup):
    """configs[1] (8192 tokens x 8 kv heads x 128, fp16, outlier channels,
    permuted slots), then the same chunk at head size 64 (4 kv heads) and 256
    (2 kv heads); graph-timed, algorithmic bytes as in workloads."""
    import numpy as np

    from turboquant_amd import workloads as W
    from turboquant_amd import ops
    from turboquant_amd.geometry import hadamard_signs
    dev = torch.device("cuda:0")
    c = W.cfg2()
    shape, pd = W.cache_bytes(c["num_blocks"], 8, 128)
    cache = torch.zeros(shape, dtype=torch.uint8, device=dev)
    k = torch.from_numpy(c["k"]).to(dev)
    v = torch.from_numpy(c["v"]).to(dev)
    slots = torch.from_numpy(c["slots"]).to(dev)
    signs = hadamard_signs(pd, dev)
    ms = time_graph(torch, lambda: ops.quantize_write_kv_cache(cache, k, v, signs, slots,
                                                               128, pd), steps, warmup)
    nbytes = W.algorithmic_write_bytes(8192, 8, 128)
    res = {"us": round(ms * 1e3, 2), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
           "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "alg_bytes": nbytes, "config": "8192 tok x 8 heads x 128, K+V fp16, outliers x20, "
                                          "permuted slots (configs[1])"}
    del cache, k, v
    # the same chunk at the other head sizes of configs[3] (kv heads 4 at hd 64,
    # 2 at hd 256), same seeding scheme
    other = []
    for hd, h in ((64, 4), (256, 2)):
        rng = np.random.default_rng(2 + hd)
        kk, vv = W.write_inputs(rng, 8192, h, hd, outliers=True)
        sl = torch.from_numpy(rng.permutation(512 * W.BLOCK)[:8192].astype(np.int32)).to(dev)
        shape, pd = W.cache_bytes(512, h, hd)
        cache = torch.zeros(shape, dtype=torch.uint8, device=dev)
        kk = torch.from_numpy(kk).to(dev)
        vv = torch.from_numpy(vv).to(dev)
        sg = hadamard_signs(pd, dev)
        ms = time_graph(torch, lambda: ops.quantize_write_kv_cache(cache, kk, vv, sg, sl, hd, pd),
                        steps, warmup)
        nb = W.algorithmic_write_bytes(8192, h, hd)
        other.append({"head_dim": hd, "kv_heads": h, "us": round(ms * 1e3, 2),
                      "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                      "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "alg_bytes": nb})
        log(f"write hd={hd} x {h} heads: {ms * 1e3:.2f} us")
        del cache, kk, vv
    res["other_head_sizes"] = other
    return res


def bench_prefill_chunk(torch, w, steps, warmup, chunk=2048):
    """One chunked-prefill attention call through TurboQuantFusedImpl.forward:
    a chunk of `chunk` new tokens at the end of a configs[2] sequence (32768
    tokens, so 30720 cached before it; the chunk's own K/V are in the cache
    too, written first as vLLM does), Qwen3-8B geometry.  The cached context
    is read back by tq_dequant_paged and the chunk attends it plus its fresh
    K/V in tq_prefill_attention (lower-right causal, grouped kv heads).  The
    metadata carries host copies of the boundaries (as vLLM's does), so no
    device-to-host read happens; timed call by call with HIP events."""
    from types import SimpleNamespace

    from turboquant_amd.vllm_backend_fused import TurboQuantFusedImpl
    dev = w["q"].device
    L, hq, hkv, hd = w["seq_len"], w["hq"], w["hkv"], w["hd"]
    impl = TurboQuantFusedImpl(hq, hd, 1.0 / math.sqrt(hd), hkv, None, None, "fp8")
    g = torch.Generator(device=dev).manual_seed(11)
    q = torch.randn((chunk, hq * hd), generator=g, device=dev).half()
    k = torch.randn((chunk, hkv * hd), generator=g, device=dev).half()
    v = torch.randn((chunk, hkv * hd), generator=g, device=dev).half()
    out = torch.empty_like(q)
    meta = SimpleNamespace(
        max_query_len=chunk, num_actual_tokens=chunk, block_table=w["bt"][:1],
        seq_lens=torch.tensor([L], dtype=torch.int32, device=dev),
        query_start_loc=torch.tensor([0, chunk], dtype=torch.int32, device=dev),
        slot_mapping=None, query_start_loc_cpu=torch.tensor([0, chunk], dtype=torch.int32),
        seq_lens_cpu=torch.tensor([L], dtype=torch.int32))
    ms = time_launches(torch, lambda: impl.forward(None, q, k, v, w["cache"], meta, output=out),
                       max(1, min(steps, 50)), max(1, min(warmup, 5)))
    return {"us": round(ms * 1e3, 1), "chunk_tokens": chunk, "cached_tokens": L - chunk,
            "config": "Qwen3-8B geometry 32q/8kv/128, one request, context read back from "
                      "the quantized cache (tq_dequant_paged) + tq_prefill_attention "
                      "(lower-right causal, GQA)"}


MFMA_F16_PEAK_TFLOPS = 2500.0


def bench_prefill_kernel(torch, seq_len=32768):
    """tq_prefill_attention on one 32768-token prompt at the Qwen3-8B
    geometry (32 q heads, 8 kv heads, head size 128, causal), the attention
    of configs[4]'s prefill, beside torch's fused flash kernel on the same
    tensors.  Work: 4 * Hq * D * (causal query-key pairs) FLOPs (QK^T and
    PV); bound: fp16 MFMA (2.5 PFLOP/s dense)."""
    import torch.nn.functional as F

    from turboquant_amd import ops
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(12)
    hq, hkv, d, L = 32, 8, 128, seq_len
    q = torch.randn((L, hq, d), generator=g, device=dev).half()
    k = torch.randn((L, hkv, d), generator=g, device=dev).half()
    v = torch.randn((L, hkv, d), generator=g, device=dev).half()
    o = torch.empty_like(q)
    scale = 1.0 / math.sqrt(d)
    flops = 4 * hq * d * (L * (L + 1) // 2)
    ms = time_launches(torch, lambda: ops.prefill_attention(q, k, v, o, scale), 10, 2)
    qt, kt, vt = (t.transpose(0, 1).unsqueeze(0) for t in (q, k, v))
    ms_t = time_launches(torch, lambda: F.scaled_dot_product_attention(
        qt, kt, vt, is_causal=True, scale=scale, enable_gqa=True), 10, 2)
    tf = flops / (ms * 1e-3) / 1e12
    res = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1),
           "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "bound": "mfma (fp16, 2.5 PFLOP/s)",
           "flops": flops, "torch_flash_us": round(ms_t * 1e3, 1),
           "torch_flash_TFLOP/s": round(flops / (ms_t * 1e-3) / 1e12, 1),
           "config": f"one {L}-token prompt, causal, 32q/8kv/128 fp16 (configs[4] prefill "
                     "attention per layer)"}
    del q, k, v, o, qt, kt, vt
    # the same prompt at head sizes 64 and 256 (configs[3]'s 16 q / 4 kv and
    # 16 q / 2 kv geometries)
    for hq, hkv, d in ((16, 4, 64), (16, 2, 256)):
        q = torch.randn((L, hq, d), generator=g, device=dev).half()
        k = torch.randn((L, hkv, d), generator=g, device=dev).half()
        v = torch.randn((L, hkv, d), generator=g, device=dev).half()
        o = torch.empty_like(q)
        scale = 1.0 / math.sqrt(d)
        flops = 4 * hq * d * (L * (L + 1) // 2)
        ms = time_launches(torch, lambda: ops.prefill_attention(q, k, v, o, scale), 10, 2)
        qt, kt, vt = (t.transpose(0, 1).unsqueeze(0) for t in (q, k, v))
        ms_t = time_launches(torch, lambda: F.scaled_dot_product_attention(
            qt, kt, vt, is_causal=True, scale=scale, enable_gqa=True), 10, 2)
        tf = flops / (ms * 1e-3) / 1e12
        res[f"head_dim_{d}"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1),
                                "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "flops": flops,
                                "torch_flash_us": round(ms_t * 1e3, 1),
                                "config": f"one {L}-token prompt, causal, {hq}q/{hkv}kv/{d} fp16"}
        del q, k, v, o, qt, kt, vt
    # a short chunk over a long context (the keys split over workgroups),
    # beside the same kernel without the split (no workspace)
    from turboquant_amd import _lib
    lib = _lib.load()
    hq, hkv, d, lq = 32, 8, 128, 256
    q = torch.randn((lq, hq, d), generator=g, device=dev).half()
    k = torch.randn((L, hkv, d), generator=g, device=dev).half()
    v = torch.randn((L, hkv, d), generator=g, device=dev).half()
    o = torch.empty_like(q)
    scale = 1.0 / math.sqrt(d)
    flops = 4 * hq * d * (lq * L - lq * (lq - 1) // 2)
    ms = time_launches(torch, lambda: ops.prefill_attention(q, k, v, o, scale), 20, 3)

    def unsplit():
        _lib.check(lib.tq_prefill_attention(
            q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1), o.data_ptr(), o.stride(0), o.stride(1), lq, L,
            hq, hkv, d, scale, torch.cuda.current_stream().cuda_stream), "prefill_attention")
    ms_u = time_launches(torch, unsplit, 20, 3)
    tf = flops / (ms * 1e-3) / 1e12
    res["short_chunk"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1),
                          "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "flops": flops,
                          "unsplit_us": round(ms_u * 1e3, 1),
                          "workspace_bytes": int(lib.tq_prefill_workspace_bytes(lq, L, hq, hkv, d)),
                          "config": f"a {lq}-token chunk over {L} keys, causal, 32q/8kv/128 fp16, "
                                    "keys split over workgroups and merged"}
    return res


def bench_mse(torch, steps, warmup, n=1 << 20, dim=128, bits=4):
    """The algorithm library's TurboQuantMSE on the GPU (tq_mse_quantize /
    tq_mse_dequantize): n fp32 vectors of dim 128 at 4 bits.  Algorithmic
    bytes: quantize reads 4 dim and writes pd b / 8 + 4 per vector;
    dequantize the reverse."""
    from turboquant_amd import algorithm as A
    dev = torch.device("cuda:0")
    q = A.TurboQuantMSE(dim, bits, device=dev)
    x = torch.randn((n, dim), device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    packed, norms = q.quantize(x)
    pd = q.rotation.padded_dim
    code_bytes = pd * bits // 8 + 4
    ms_q = time_graph(torch, lambda: q.quantize(x), steps, warmup)
    ms_d = time_graph(torch, lambda: q.dequantize(packed, norms), steps, warmup)
    bq = n * (4 * dim + code_bytes)
    return {"quantize_us": round(ms_q * 1e3, 2),
            "quantize_GB/s": round(bq / (ms_q * 1e-3) / 1e9, 1),
            "dequantize_us": round(ms_d * 1e3, 2),
            "dequantize_GB/s": round(bq / (ms_d * 1e-3) / 1e9, 1), "alg_bytes": bq,
            "config": f"TurboQuantMSE({dim}, {bits}) on {n} fp32 vectors (algorithm library, "
                      "HIP kernels; allocation of the outputs inside the timed calls)"}


def bench_prod(torch, steps, warmup, n=1 << 20, dim=128, bits=4):
    """TurboQuantProd on the GPU: n fp32 vectors of dim 128 at 4 bits (MSE
    stage at 3), through the public API, which at this size is one kernel
    each way with the QJL products on the matrix cores
    (tq_prod_quantize_qjl / tq_prod_dequantize_qjl).  Algorithmic bytes per
    vector: quantize reads 4 dim and writes the codes, norm, dim int8 signs
    and residual norm; dequantize the reverse.  MFMA work per vector: 3 (or
    2) fp16 d x d products.  Also timed: the same with the QJL products as
    fp32 BLAS GEMMs (tq_prod_quantize / tq_prod_dequantize around them), the
    path above padded size 128."""
    from turboquant_amd import algorithm as A
    from turboquant_amd import ops
    dev = torch.device("cuda:0")
    q = A.TurboQuantProd(dim, bits, device=dev)
    x = torch.randn((n, dim), device=dev, generator=torch.Generator(device=dev).manual_seed(4))
    m = q.mse
    pd = m.rotation.padded_dim
    bnd, cen = m._host_tables()
    pk, nm, z, rn = q.quantize(x)
    per = 2 if bits - 1 == 3 else 8 // (bits - 1)
    code_bytes = pd // per + 4
    ms_q = time_graph(torch, lambda: q.quantize(x), steps, warmup)
    ms_d = time_graph(torch, lambda: q.dequantize(pk, nm, z, rn), steps, warmup)

    def blas_q():
        p2, n2, ru, r2 = ops.prod_quantize(x, pd, bits - 1, m.rotation.signs, bnd, cen)
        return q.qjl.quantize(ru)

    def blas_d():
        return ops.prod_dequantize(pk, nm, z.float() @ q.qjl.S, rn, dim, pd, bits - 1,
                                   m.rotation.signs, cen)
    ms_bq = time_graph(torch, blas_q, max(1, steps // 4), max(1, warmup // 4))
    ms_bd = time_graph(torch, blas_d, max(1, steps // 4), max(1, warmup // 4))
    bq = n * (4 * dim + code_bytes + dim + 4)
    return {"quantize_us": round(ms_q * 1e3, 2),
            "quantize_GB/s": round(bq / (ms_q * 1e-3) / 1e9, 1),
            "dequantize_us": round(ms_d * 1e3, 2),
            "dequantize_GB/s": round(bq / (ms_d * 1e-3) / 1e9, 1), "alg_bytes": bq,
            "mfma_TFLOP/s": [round(n * 6 * pd * pd / (ms_q * 1e-3) / 1e12, 1),
                             round(n * 4 * pd * pd / (ms_d * 1e-3) / 1e12, 1)],
            "blas_path_us": [round(ms_bq * 1e3, 2), round(ms_bd * 1e3, 2)],
            "config": f"TurboQuantProd({dim}, {bits}) on {n} fp32 vectors: fused HIP kernels "
                      "(QJL on MFMA); blas_path_us = the kernels around fp32 BLAS GEMMs; "
                      "output allocation inside the timed calls"}


def bench_dequant(torch, w, steps, warmup):
    """tq_dequant_paged (the read-back of cached context for a prefill chunk)
    over one configs[2] sequence: 32768 tokens x 8 heads of K and V back to
    fp16 rows.  Algorithmic bytes: the entries' codes + norms read
    (2 x 68 B per token and head) plus the fp16 rows written (2 x 256 B)."""
    from turboquant_amd import ops
    L, hkv, hd, pd = w["seq_len"], w["hkv"], w["hd"], w["pd"]
    pages = w["bt"][0].contiguous()
    ok = torch.empty((L, hkv, hd), dtype=torch.float16, device=w["q"].device)
    ov = torch.empty_like(ok)
    ms = time_graph(torch, lambda: ops.dequant_paged(w["cache"], pages, L, hkv, hd, pd,
                                                     w["signs"], ok, ov), steps, warmup)
    nbytes = L * hkv * 2 * (pd // 2 + 2 * (pd // 64)) + L * hkv * 2 * hd * 2 + (L // 16) * 4
    return {"us": round(ms * 1e3, 2), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "alg_bytes": nbytes, "config": f"{L} cached tokens x {hkv} heads x {hd}, K+V "
                                           "(one configs[2] sequence), fp16 rows out"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed steps before each timed leg (each leg also runs its "
                         "work untimed for 0.1 s first, so the GPU clocks are up)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-e2e", action="store_true", help="skip the configs[4] end-to-end leg")
    ap.add_argument("--no-ragged", action="store_true", help="skip the configs[3] legs")
    ap.add_argument("--static", action="store_true",
                    help="headline through the reference's static-split op instead of the "
                         "balanced op the backend uses")
    ap.add_argument("--splits", type=int, default=0, help="override num_splits (--static)")
    ap.add_argument("--seq-len", type=int, default=32768,
                    help="cached tokens per sequence of the headline workload (configs[2]: "
                         "32768; other lengths for the step/fixed-cost split of the kernel)")
    ap.add_argument("--copy-ref", action="store_true",
                    help="only run a plain 256 MiB device copy x5 (HBM counter scale reference)")
    ap.add_argument("--stream-ref", action="store_true",
                    help="also time the partials kernel with its math compiled out "
                         "and the bare copy ring (tq_diag_decode_stream: the data movement "
                         "alone)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the headline decode steps (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build's path runs on a single MI355X; "
              f"--gpus {args.gpus} is not supported (multi-GPU sharding is not built).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_ref:
        # FETCH_SIZE / WRITE_SIZE of a copy of known size calibrate the
        # counters used for roofline.traffic
        a = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda:0")
        c = torch.empty_like(a)
        for _ in range(5):
            c.copy_(a)
        torch.cuda.synchronize()
        log("copied 256 MiB x5")
        return

    from turboquant_amd import _lib, ops
    _lib.load()
    quick = args.decode_only
    ragged = None if (quick or args.no_ragged) else bench_ragged(torch, args.steps, args.warmup)
    e2e_res = None if (quick or args.no_e2e) else bench_e2e(torch)
    log("building cfg-3 cache on the GPU (write kernel)")
    w = make_decode_workload(torch, seq_len=args.seq_len)
    if args.splits:
        w["splits"] = args.splits
        w["cs"] = -(-w["seq_len"] // args.splits) + 15 & ~15
    b, hq, pd, S = w["batch"], w["hq"], w["pd"], w["splits"]
    dev = w["q"].device
    o = torch.empty((b, hq, pd), dtype=torch.float16, device=dev)
    po = torch.empty((b * S, hq, pd), dtype=torch.float32, device=dev)
    pl = torch.empty((b * S, hq), dtype=torch.float32, device=dev)
    rows = ops.balanced_rows(b, hq, w["hkv"], pd)
    pob = torch.empty((rows, hq, pd), dtype=torch.float32, device=dev)
    plb = torch.empty((rows, hq), dtype=torch.float32, device=dev)
    split = torch.zeros(b + 2, dtype=torch.int32, device=dev)
    scale = 1.0 / math.sqrt(w["hd"])
    lib = _lib.load()
    cache = w["cache"]

    def step_static():
        ops.decode_paged_splitkv(w["q"], cache, w["indices"], w["indptr"], w["seq"], w["hkv"],
                                 w["hd"], pd, scale, w["signs"], o, po, pl, S, w["cs"])

    def step_balanced():
        ops.decode_paged_balanced(w["q"], cache, w["indices"], w["indptr"], w["seq"], w["hkv"],
                                  w["hd"], pd, scale, w["signs"], o, pob, plb, split)

    def combine_only():
        rc = lib.tq_combine_splits(po.data_ptr(), pl.data_ptr(), b, S, hq, pd,
                                   w["signs"].data_ptr(), o.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "tq_combine_splits")

    step = step_static if args.static else step_balanced
    op_name = ("turboquant_v5::decode_v5_from_cache_paged_splitkv_ws (static splits)"
               if args.static else "turboquant_v5::decode_paged_balanced_ws (balanced plan)")
    wr = dq = pf = pk = cpu = mse = prod = None
    if not quick:
        mse = bench_mse(torch, args.steps, args.warmup)
        log(f"algorithm MSE quantize {mse['quantize_us']} us, dequantize {mse['dequantize_us']} us")
        prod = bench_prod(torch, args.steps // 2, args.warmup // 2)
        log(f"algorithm Prod quantize {prod['quantize_us']} us, dequantize "
            f"{prod['dequantize_us']} us (BLAS path {prod['blas_path_us']})")
        wr = bench_write(torch, args.steps, args.warmup)
        log(f"write kernel {wr['us']} us -> {wr['GB/s']} GB/s")
        dq = bench_dequant(torch, w, args.steps, args.warmup)
        log(f"dequant kernel {dq['us']} us -> {dq['GB/s']} GB/s")
        pf = bench_prefill_chunk(torch, w, args.steps, args.warmup)
        log(f"prefill chunk {pf['chunk_tokens']} tokens over {pf['cached_tokens']} cached: "
            f"{pf['us']} us")
        pk = bench_prefill_kernel(torch)
        log(f"prefill attention kernel {pk['us']} us ({pk['TFLOP/s']} TFLOP/s); torch flash "
            f"{pk['torch_flash_us']} us")
    log(f"timing decode ({op_name}): steps={args.steps} warmup={args.warmup}")
    ms_eager = time_launches(torch, step, args.steps, args.warmup)
    ms = time_graph(torch, step, args.steps, args.warmup)
    ms_other = time_graph(torch, step_balanced if args.static else step_static, args.steps,
                          args.warmup)
    nbytes = alg_bytes(w)
    value = nbytes / (ms * 1e-3) / 1e9
    log(f"decode step {ms * 1e3:.1f} us (graph replay; {ms_eager * 1e3:.1f} us launched one "
        f"call at a time from Python) -> {value:.0f} GB/s; the other op "
        f"{ms_other * 1e3:.1f} us")
    # the partials kernel's average duration: a HIP graph of the partials
    # kernel alone, launched back to back, timed with HIP events on the
    # replay stream (per launch: the kernel plus the graph's launch gap, no
    # host overhead); the combine likewise alone over the same 512 rows.
    # HIP events around each launch would add 3-5 us of their own to it.
    def partials_only():
        if args.static:
            rc = lib.tq_decode_partials(
                w["q"].data_ptr(), w["q"].stride(0), w["q"].stride(1), cache.data_ptr(),
                cache.data_ptr() + cache[0].numel(), w["indices"].data_ptr(),
                w["indptr"].data_ptr(), w["seq"].data_ptr(), b, hq, w["hkv"], pd, 16, w["ebs"],
                w["nb"], scale, w["signs"].data_ptr(), S, w["cs"], po.data_ptr(), pl.data_ptr(),
                torch.cuda.current_stream().cuda_stream)
        else:
            rc = lib.tq_decode_partials_balanced(
                w["q"].data_ptr(), w["q"].stride(0), w["q"].stride(1), cache.data_ptr(),
                cache.data_ptr() + cache[0].numel(), w["indices"].data_ptr(),
                w["indptr"].data_ptr(), w["seq"].data_ptr(), b, hq, w["hkv"], w["hd"], pd, 16,
                w["ebs"], w["nb"], scale, w["signs"].data_ptr(), rows, pob.data_ptr(),
                plb.data_ptr(), split.data_ptr(), torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "partials")

    ms_k = time_graph(torch, partials_only, args.steps, args.warmup)
    step_static()
    torch.cuda.synchronize()
    ms_c = time_graph(torch, combine_only, args.steps, args.warmup)
    achieved = nbytes / (ms_k * 1e-3) / 1e9
    log(f"partials kernel {ms_k * 1e3:.1f} us -> {achieved:.0f} GB/s; combine {ms_c * 1e3:.1f} us; "
        f"step - both {(ms - ms_k - ms_c) * 1e3:.1f} us of launch gaps")
    stream_ref = None
    if args.stream_ref:
        def diag(mode):
            rc = lib.tq_diag_decode_stream(
                w["q"].data_ptr(), w["q"].stride(0), w["q"].stride(1), cache.data_ptr(),
                cache.data_ptr() + cache[0].numel(), w["indices"].data_ptr(),
                w["indptr"].data_ptr(), w["seq"].data_ptr(), b, hq, w["hkv"], pd, 16, w["ebs"],
                w["nb"], scale, w["signs"].data_ptr(), S, w["cs"], po.data_ptr(), pl.data_ptr(),
                mode, torch.cuda.current_stream().cuda_stream)
            _lib.check(rc, "tq_diag_decode_stream")
        lbytes = b * w["seq_len"] * w["hkv"] * 2 * w["ebs"]
        stream_ref = {}
        for mode, key, what in (
                (1, "no_math", "decode_partials_kernel<128, 8, 2, true, false, 1>: the "
                 "static-split partials kernel with the attention math compiled out (page "
                 "walk, LDS copy ring, waits, barriers, slot reads; q setup, table build and "
                 "partial-row stores kept)"),
                (0, "bare_ring", "decode_partials_kernel<128, 8, 2, true, false, 0>: the bare "
                 "copy ring (page walk, copies, waits, barriers, slot reads; no q setup, "
                 "table or stores)")):
            ms_s = time_graph(torch, lambda: diag(mode), args.steps, args.warmup)
            stream_ref[key] = {"us": round(ms_s * 1e3, 2),
                               "layout_GB/s": round(lbytes / (ms_s * 1e-3) / 1e9, 1),
                               "alg_frac": round(alg_bytes(w) / (ms_s * 1e-3) / 1e9 /
                                                 HBM_PEAK_GBS, 4),
                               "what": what}
            log(f"partials diagnostic {key}: {ms_s * 1e3:.1f} us")
        # a plain non-temporal stream over the same cache bytes (both slabs of
        # the cache tensor): the read rate HBM gives without the ring's page
        # walk, dependent start and barriers
        sink = torch.zeros(4, dtype=torch.int32, device=cache.device)
        cbytes = cache.numel() // 16 * 16

        def sread():
            _lib.check(lib.tq_diag_stream_read(cache.data_ptr(), cbytes, sink.data_ptr(),
                                               torch.cuda.current_stream().cuda_stream),
                       "tq_diag_stream_read")
        ms_r = time_graph(torch, sread, args.steps, args.warmup)
        stream_ref["plain_stream"] = {"us": round(ms_r * 1e3, 2), "bytes": cbytes,
                                      "GB/s": round(cbytes / (ms_r * 1e-3) / 1e9, 1),
                                      "what": "stream_read_kernel: non-temporal 16-byte loads "
                                              "over the whole cache tensor, no page table"}
        log(f"plain stream read of {cbytes / 1e6:.1f} MB: {ms_r * 1e3:.1f} us")
    plan = split.cpu().tolist()
    layout_bytes = b * w["seq_len"] * w["hkv"] * 2 * w["ebs"]
    if not (quick or args.no_cpu):
        log("CPU baseline (torch-CPU port) ...")
        cpu = cpu_baseline(torch, w)
        log(f"CPU baseline {cpu['value']} GB/s decode, {cpu['write']['value']} GB/s write on "
            f"{cpu['cores']} threads ({cpu['cpu']})")

    kname = ("decode_partials_kernel<128, 8, 2, true, false>" if args.static else
             "decode_partials_kernel<128, 8, 2, true, true>")
    line = {
        "metric": "decode-attn GB/s & % HBM peak, Qwen3-8B shape B=8 L=32k",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "ms_per_step_eager": round(ms_eager, 5),
        "higher_is_better": True,
        "scaling": "weak",  # one GPU: its work per step is fixed (--gpus > 1 exits)
        "vs_baseline": None,
        "dtype": "u4 codes -> f16 MFMA, f32 accumulate",
        "data": "synthetic (seeded torch RNG, N(0,1) q/K/V, random page permutation)",
        "config": {"workload": "decode attention, configs[2]: Qwen3-8B geometry 32q/8kv/hd128, "
                               "B=8, 32768 cached tokens/seq, 16-token pages, split-KV + LSE merge",
                   "op": op_name, "batch": b, "seq_len": w["seq_len"], "num_qo_heads": hq,
                   "num_kv_heads": w["hkv"], "head_dim": w["hd"], "page_size": 16,
                   "split_rows": plan[b], "unit_tokens": plan[b + 1],
                   "parallelism": "single GPU"},
        "ms_per_step_other_op": round(ms_other, 5),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "layout_GB/s": round(layout_bytes / (ms * 1e-3) / 1e9, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": PROFILED_TRAFFIC.get(("static" if args.static else "balanced",
                                                      S, w["cs"])),
                     "traffic_source": TRAFFIC_SOURCE,
                     "kernel": kname, "kernel_us": round(ms_k * 1e3, 2),
                     "kernel_timing": "HIP events around graph replays of the partials kernel "
                                      "alone, back to back (kernel + graph launch gap)",
                     "combine_us": round(ms_c * 1e3, 2), "alg_bytes": nbytes,
                     # the same kernel time against the bytes of the cache layout
                     # (80-byte entries: pad and second norm copy included), which
                     # whole cache lines make HBM move
                     "layout_bytes": layout_bytes,
                     "layout_frac": round(layout_bytes / (ms_k * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                          4)},
        "cpu_baseline": cpu,
        "configs3_ragged": ragged,
        "e2e": e2e_res,
        "write_kernel": wr,
        "dequant_kernel": dq,
        "algorithm_mse": mse,
        "algorithm_prod": prod,
        "prefill_chunk": pf,
        "prefill_kernel": pk,
        "stream_ref": stream_ref,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
