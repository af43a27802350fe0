"""The no-allocation decode entry point (tq_decode_paged_balanced_noalloc),
called through the C ABI: its output equals tq_decode_paged_balanced's (same
kernels; the plan is the same when the scratch holds the rows the workspace
variant uses) on two calls in a row, the second with a smaller batch, and
matches the oracle."""
import ctypes

import numpy as np
import pytest
import torch

from tests import gpu_cases as G
from turboquant_amd import workloads as W
from turboquant_amd import _lib, ops
from turboquant_amd.geometry import hadamard_signs

pytestmark = pytest.mark.gpu


def _noalloc(d, case, cache, pd, o):
    lib = _lib.load()
    b, hq, hd = case["q"].shape
    _, nb, bs, hkv, ebs = cache.shape
    base = cache.data_ptr()
    slab = nb * bs * hkv * ebs
    s = hadamard_signs(pd, G.DEV)
    rc = lib.tq_decode_paged_balanced_noalloc(
        d["q"].data_ptr(), d["q"].stride(0), d["q"].stride(1), base, base + slab,
        d["indices"].data_ptr(), d["indptr"].data_ptr(), d["seq"].data_ptr(), b, hq, hkv, hd,
        pd, bs, ebs, nb, ctypes.c_float(1.0 / np.sqrt(hd)), s.data_ptr(), o.data_ptr(),
        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "tq_decode_paged_balanced_noalloc")


@pytest.mark.parametrize("hq,hkv,hd", [(32, 8, 128), (16, 2, 256)])
def test_noalloc_matches_workspace_entry_twice(hq, hkv, hd):
    cases = [(97, [5000, 17, 0, 3000, 1, 2048, 900, 64]), (98, [700, 33, 1500])]
    for i, (seed, lens) in enumerate(cases):
        print(f"case: noalloc call {i} {hq}/{hkv}/{hd} lens={lens}", flush=True)
        c = W.decode_case(seed, len(lens), lens, hq, hkv, hd)
        cache, pd = G.build_cache(c)
        d = G.decode_inputs(c, pd)
        o = torch.full((len(lens), hq, pd), float("nan"), dtype=torch.float16, device=G.DEV)
        _noalloc(d, c, cache, pd, o)
        torch.cuda.synchronize()
        got = o.float().cpu().numpy()
        want, qp, scale, _ = G.run_balanced(c, cache, pd)
        assert np.array_equal(got, want), f"call {i}: differs from the workspace entry point"
        ref = G.oracle_decode(c, cache.cpu().numpy(), qp, pd, scale)
        G.assert_close(got, ref, f"noalloc call {i}")


def test_noalloc_refuses_batches_beyond_the_scratch():
    """16 MiB of scratch: 1024 sequences x 64 q heads x pd 256 does not fit."""
    lib = _lib.load()
    null = None
    rc = lib.tq_decode_paged_balanced_noalloc(null, 0, 0, null, null, null, null, null, 1024, 64,
                                              8, 256, 256, 16, 144, 10, ctypes.c_float(0.1), null,
                                              null, null)
    assert rc == -22
    assert b"scratch" in lib.tq_last_error()
