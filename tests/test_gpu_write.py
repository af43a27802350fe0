"""GPU parity of the write kernel against the C oracle: bit-exact cache bytes."""
import math

import numpy as np
import pytest
import torch

import oracle
from turboquant_amd import workloads as W
from turboquant_amd import ops
from turboquant_amd.geometry import hadamard_signs

pytestmark = pytest.mark.gpu


def _oracle_cache(shape, k, v, slots, hd, pd, fill=0):
    cache = np.full(shape, fill, np.uint8)
    oracle.write_kv_cache(cache, k, v, hadamard_signs(pd).numpy(), slots, hd, pd)
    return cache


def _gpu_cache(shape, k, v, slots, hd, pd, fill=0, dtype=torch.float16):
    dev = torch.device("cuda:0")
    cache = torch.full(shape, fill, dtype=torch.uint8, device=dev)
    kt = torch.from_numpy(k).to(dev).to(dtype)
    vt = torch.from_numpy(v).to(dev).to(dtype)
    ops.quantize_write_kv_cache(cache, kt, vt, hadamard_signs(pd, dev),
                                torch.from_numpy(slots).to(dev), hd, pd)
    torch.cuda.synchronize()
    return cache.cpu().numpy()


def _diff_report(a, b):
    bad = np.argwhere(a != b)
    return f"{len(bad)} bytes differ, first {bad[:5].tolist()}"


def test_cfg2_write_bit_exact():
    print("case: cfg2 write 8192x8x128 outliers x20, permuted slots", flush=True)
    c = W.cfg2()
    shape, pd = W.cache_bytes(c["num_blocks"], 8, 128)
    ref = _oracle_cache(shape, c["k"], c["v"], c["slots"], 128, pd, fill=0xA5)
    got = _gpu_cache(shape, c["k"], c["v"], c["slots"], 128, pd, fill=0xA5)
    assert np.array_equal(ref, got), _diff_report(ref, got)
    # pad bytes untouched
    assert (got[..., 68:] == 0xA5).all()


@pytest.mark.parametrize("hd", [64, 96, 256])
def test_write_other_head_dims(hd):
    print(f"case: write hd={hd}", flush=True)
    rng = np.random.default_rng(10 + hd)
    n, h, nb = 300, 4, 32
    k, v = W.write_inputs(rng, n, h, hd, k_dist="t3")
    slots = rng.permutation(nb * 16)[:n].astype(np.int32)
    shape, pd = W.cache_bytes(nb, h, hd)
    ref = _oracle_cache(shape, k, v, slots, hd, pd)
    got = _gpu_cache(shape, k, v, slots, hd, pd)
    assert np.array_equal(ref, got), _diff_report(ref, got)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_write_input_dtypes(dtype):
    """fp32 (the reference's own input dtype) and bf16 rows give the oracle's bytes
    for the same fp16-representable values."""
    print(f"case: write dtype={dtype}", flush=True)
    rng = np.random.default_rng(5)
    n, h, hd, nb = 200, 8, 128, 16
    k, v = W.write_inputs(rng, n, h, hd)
    if dtype == torch.bfloat16:  # values exactly representable in both
        k = torch.from_numpy(k).to(torch.bfloat16).to(torch.float16).numpy()
        v = torch.from_numpy(v).to(torch.bfloat16).to(torch.float16).numpy()
    slots = np.arange(n, dtype=np.int32)
    shape, pd = W.cache_bytes(nb, h, hd)
    ref = _oracle_cache(shape, k, v, slots, hd, pd)
    got = _gpu_cache(shape, k, v, slots, hd, pd, dtype=dtype)
    assert np.array_equal(ref, got), _diff_report(ref, got)


def test_write_skips_negative_and_out_of_range_slots():
    print("case: write negative/oob slots", flush=True)
    rng = np.random.default_rng(6)
    n, h, hd, nb = 64, 8, 128, 4
    k, v = W.write_inputs(rng, n, h, hd)
    slots = np.arange(n, dtype=np.int32)
    slots[::3] = -1
    slots[1] = nb * 16 + 5  # beyond the cache
    shape, pd = W.cache_bytes(nb, h, hd)
    ref = _oracle_cache(shape, k, v, slots, hd, pd, fill=0x11)
    got = _gpu_cache(shape, k, v, slots, hd, pd, fill=0x11)
    assert np.array_equal(ref, got), _diff_report(ref, got)
    flat = got[0].reshape(nb * 16, h, -1)
    assert (flat[0] == 0x11).all() and (flat[3] == 0x11).all()


def test_write_strided_rows_and_zero_rows():
    """key/value as strided views of a fused qkv buffer; all-zero rows map to 0x88."""
    print("case: write strided + zero rows", flush=True)
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(7)
    n, h, hd, nb = 48, 8, 128, 4
    qkv = rng.standard_normal((n, (32 + 2 * h) * hd)).astype(np.float16)
    qkv[5] = 0
    k = qkv[:, 32 * hd:(32 + h) * hd].reshape(n, h, hd)
    v = qkv[:, (32 + h) * hd:].reshape(n, h, hd)
    slots = np.arange(n, dtype=np.int32)
    shape, pd = W.cache_bytes(nb, h, hd)
    ref = _oracle_cache(shape, np.ascontiguousarray(k), np.ascontiguousarray(v), slots, hd, pd)
    t = torch.from_numpy(qkv).to(dev)
    kt = t[:, 32 * hd:(32 + h) * hd].view(n, h, hd)
    vt = t[:, (32 + h) * hd:].view(n, h, hd)
    cache = torch.zeros(shape, dtype=torch.uint8, device=dev)
    ops.quantize_write_kv_cache(cache, kt, vt, hadamard_signs(pd, dev),
                                torch.from_numpy(slots).to(dev), hd, pd)
    got = cache.cpu().numpy()
    assert np.array_equal(ref, got), _diff_report(ref, got)
    row5 = got[0].reshape(nb * 16, h, -1)[5]
    assert (row5[:, :64] == 0x88).all() and (row5[:, 64:68] == 0).all()


def test_write_empty_is_noop():
    dev = torch.device("cuda:0")
    cache = torch.zeros((2, 1, 16, 8, 80), dtype=torch.uint8, device=dev)
    e = torch.zeros((0, 8, 128), dtype=torch.float16, device=dev)
    ops.quantize_write_kv_cache(cache, e, e, hadamard_signs(128, dev),
                                torch.zeros(0, dtype=torch.int32, device=dev), 128, 128)
    assert int(cache.sum()) == 0


def test_cfg1_write_matches_golden_fixture():
    """configs[0] written on the GPU hashes to the committed golden cache."""
    import hashlib
    import json
    import os
    print("case: cfg1 write vs tests/golden/cfg1.json", flush=True)
    with open(os.path.join(os.path.dirname(__file__), "golden", "cfg1.json")) as f:
        meta = json.load(f)
    c = W.cfg1()
    shape, pd = W.cache_bytes(c["num_blocks"], 8, 128)
    got = _gpu_cache(shape, c["k"], c["v"], c["slots"], 128, pd)
    assert hashlib.sha256(got.tobytes()).hexdigest() == meta["cache_sha256"]


def test_write_kat_vectors():
    """The golden known-answer rows (normal, tiny, huge, zero, one-hot, outlier
    rows at head sizes 64/96/128/256) written by the GPU equal the fixture."""
    import os
    print("case: write KAT fixture", flush=True)
    kat = np.load(os.path.join(os.path.dirname(__file__), "golden", "write_kat.npz"))
    for hd in (64, 96, 128, 256):
        x, e = kat[f"x{hd}"], kat[f"e{hd}"]
        n = x.shape[0]
        shape, pd = W.cache_bytes(math.ceil(n / 16), 1, hd)
        got = _gpu_cache(shape, x[:, None, :], x[:, None, :], np.arange(n, dtype=np.int32), hd, pd)
        k_entries = got[0].reshape(-1, shape[-1])[:n, :e.shape[1]]
        assert np.array_equal(k_entries, e), f"hd {hd}: {_diff_report(k_entries, e)}"


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_write_nonfinite_and_extreme_rows(hd):
    """Rows holding inf, -inf, NaN, fp16 max and subnormals: the codes match the
    oracle bit for bit (NaN after the rotation -> code 0 everywhere); norms
    match, or are both NaN."""
    print(f"case: write non-finite rows hd={hd}", flush=True)
    rng = np.random.default_rng(40 + hd)
    n, h, nb = 32, 2, 4
    k, v = W.write_inputs(rng, n, h, hd)
    k[0, 0, 3] = np.inf
    k[1, 1, 0] = -np.inf
    k[2, 0, hd - 1] = np.nan
    v[3, 0, :] = np.float16(65504.0)
    v[4, 1, :] = np.float16(-65504.0)
    v[5, 0, :] = np.float16(6e-8)
    v[6, 1, ::2] = np.float16(-6e-8)
    k[7, 0, :] = np.float16(-0.0)
    slots = np.arange(n, dtype=np.int32)
    shape, pd = W.cache_bytes(nb, h, hd)
    ref = _oracle_cache(shape, k, v, slots, hd, pd)
    got = _gpu_cache(shape, k, v, slots, hd, pd)
    qb = pd // 2
    assert np.array_equal(ref[..., :qb], got[..., :qb]), _diff_report(ref[..., :qb], got[..., :qb])
    nr = ref[..., qb:qb + 2 * (pd // 64)].copy().view(np.float16)
    ng = got[..., qb:qb + 2 * (pd // 64)].copy().view(np.float16)
    same = (nr.view(np.uint16) == ng.view(np.uint16)) | (np.isnan(nr) & np.isnan(ng))
    assert same.all()
    assert (got[0].reshape(-1, h, shape[-1])[0, 0, :qb] == 0).all()  # the inf row
