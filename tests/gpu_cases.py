"""Helpers shared by the GPU decode tests: build a cache on the device with the
write kernel (itself pinned bit-exact against the oracle) and run the decode."""
from __future__ import annotations

import numpy as np
import torch

from turboquant_amd import ops
from turboquant_amd.geometry import choose_splits, hadamard_signs

from turboquant_amd import workloads as W

DEV = torch.device("cuda:0")


def build_cache(case):
    return W.build_cache(case, DEV)


def decode_inputs(case, pd):
    return W.decode_inputs(case, pd, DEV)


def device_case(seed, seq_lens, hq, hkv, hd, k_dist="normal", chunk_tokens=1 << 16):
    return W.device_case(seed, seq_lens, hq, hkv, hd, k_dist, chunk_tokens, DEV)


def run_balanced(case, cache, pd, signs=True, rows=None):
    """The balanced-plan decode; returns (o, qp, scale, split_indptr)."""
    d = decode_inputs(case, pd)
    b, hq, hd = case["q"].shape
    if rows is None:
        rows = ops.balanced_rows(b, hq, case["num_kv_heads"], pd)
    o = torch.empty((b, hq, pd), dtype=torch.float16, device=DEV)
    po = torch.empty((rows, hq, pd), dtype=torch.float32, device=DEV)
    pl = torch.empty((rows, hq), dtype=torch.float32, device=DEV)
    split = torch.full((b + 2,), -7, dtype=torch.int32, device=DEV)
    s = hadamard_signs(pd, DEV) if signs else None
    scale = 1.0 / np.sqrt(hd)
    ops.decode_paged_balanced(d["q"], cache, d["indices"], d["indptr"], d["seq"],
                              case["num_kv_heads"], hd, pd, scale, s, o, po, pl, split)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), d["qp"], scale, split.cpu().numpy()


def run_decode(case, cache, pd, num_splits=None, chunk=None, signs=True, sm_scale=None):
    q = case["q"]
    b, hq, hd = q.shape
    qp = np.zeros((b, hq, pd), np.float16)
    qp[:, :, :hd] = q
    qt = torch.from_numpy(qp).to(DEV)
    bt = torch.from_numpy(case["block_table"]).to(DEV)
    indices = bt.reshape(-1).contiguous()
    indptr = (torch.arange(b + 1, dtype=torch.int32, device=DEV) * bt.shape[1]).contiguous()
    seq = torch.from_numpy(np.asarray(case["seq_lens"], np.int32)).to(DEV)
    max_len = bt.shape[1] * W.BLOCK
    if num_splits is None:
        num_splits, chunk = choose_splits(b, max_len, case["num_kv_heads"], hq, pd)
    elif chunk is None:
        chunk = -(-max_len // num_splits)
    o = torch.empty((b, hq, pd), dtype=torch.float16, device=DEV)
    po = torch.empty((b * num_splits, hq, pd), dtype=torch.float32, device=DEV)
    pl = torch.empty((b * num_splits, hq), dtype=torch.float32, device=DEV)
    s = hadamard_signs(pd, DEV) if signs else None
    scale = sm_scale if sm_scale is not None else 1.0 / np.sqrt(hd)
    ops.decode_paged_splitkv(qt, cache, indices, indptr, seq, case["num_kv_heads"], hd, pd,
                             scale, s, o, po, pl, num_splits, chunk)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), qp, scale


def oracle_decode(case, cache_np, qp, pd, scale, signs=True):
    import oracle
    b = qp.shape[0]
    bt = case["block_table"]
    indptr = np.arange(b + 1, dtype=np.int32) * bt.shape[1]
    s = hadamard_signs(pd).numpy() if signs else None
    return oracle.decode(qp, cache_np, bt.reshape(-1), indptr, case["seq_lens"],
                         case["num_kv_heads"], pd, scale, s)


ATOL, RTOL = 2e-3, 1e-2  # north-star tolerance vs the fp32 dequantize-then-attend result


def assert_close(got, ref, what=""):
    err = np.abs(got - ref)
    lim = ATOL + RTOL * np.abs(ref)
    bad = err > lim
    big = np.abs(ref) > 1e-2
    rel = float((err[big] / np.abs(ref[big])).max()) if big.any() else 0.0
    print(f"  {what}: max abs err {err.max():.3e}, rms {np.sqrt(np.mean(err ** 2)):.3e}, "
          f"max rel err (|ref| > 1e-2) {rel:.3e}, |ref| max {np.abs(ref).max():.3e}", flush=True)
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} outside atol {ATOL} / "
                           f"rtol {RTOL}; max abs err {err.max():.3e}")


def expected_plan(seq_lens, units):
    """The balanced plan's unit size: the smallest multiple of 32 tokens with
    sum_b ceil(L_b / U) <= units."""
    lens = np.maximum(np.asarray(seq_lens, np.int64), 0)
    u = 32
    while int(np.sum(-(-lens // u))) > units:
        u += 32
    return u
