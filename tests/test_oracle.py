"""Pins the C oracle (oracle/tq_oracle.c) with checks that do not restate it.

* codebook / boundaries: the Lloyd-Max optimality conditions of N(0,1),
  solved here from scratch with scipy (turboquant/codebook.py:37-62 holds the
  reference's literals; page_turbo.cuh:18-23 and quantize_write_kernel.cuh:22-28
  their fp32 copies);
* rotation / nibble order / tie rule: a vector built backwards from chosen
  codes (KAT of csrc/tests/test_pack.cpp:47-51, {0x0A, 0x05} -> 0xA5),
  the FWHT against the Sylvester-Hadamard matrix (KAT of
  tests/test_algorithm.py:46-50), boundary values fed to the binary search;
* norm: fp32 -> fp16 conversion against numpy's IEEE round-to-nearest-even;
* write: codes and norms against the independent float64 path of npref.py
  (matrix rotation + searchsorted), mismatches allowed only within a few ulp
  of a boundary (the one place fp32 rounding order may legitimately differ);
* decode: against npref's original-domain fp64 attention, plus closed-form
  cases (one token -> its dequantized V) and page-permutation invariance;
* golden fixtures written by tests/golden/make_golden.py.
"""
import hashlib
import json
import math
import os

import numpy as np
import pytest
from scipy import stats
from scipy.linalg import hadamard

import oracle
from tests import npref
from turboquant_amd import workloads as W

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


def _signs(pd):
    with open(os.path.join(GOLDEN, "signs.json")) as f:
        return np.array(json.load(f)[str(pd)], np.float32)


def _lloyd_max_16():
    """16-level Lloyd-Max quantizer of N(0,1): the fixed point c = E[X | cell(c)]
    with cells split at the midpoints, solved in float64."""
    from scipy import optimize

    def cond_mean(c):
        b = np.concatenate([[-np.inf], (c[:-1] + c[1:]) / 2, [np.inf]])
        lo, hi = b[:-1], b[1:]
        return (stats.norm.pdf(lo) - stats.norm.pdf(hi)) / (stats.norm.cdf(hi) - stats.norm.cdf(lo))

    c = optimize.fsolve(lambda x: cond_mean(x) - x, np.linspace(-2.7, 2.7, 16), xtol=1e-14)
    assert np.max(np.abs(cond_mean(c) - c)) < 1e-12
    return c


def test_codebook_is_lloyd_max_of_standard_normal():
    ref = _lloyd_max_16()
    cb = oracle.codebook().astype(np.float64)
    # The reference's literals (codebook.py:37-55) sit within 3.3e-4 of the
    # true optimum (largest at +-2.069); a transposed, dropped or mis-signed
    # entry would be off by >= 0.1.
    assert np.max(np.abs(cb - ref)) < 5e-4
    assert np.all(np.diff(cb) > 0)
    assert np.array_equal(cb[::-1], -cb)  # odd symmetry used by the GPU dequant
    # the decode constants (page_turbo.cuh:18-23) are the float64 literals of
    # codebook.py:37-55 rounded to 7 decimals, then to fp32
    want = np.array([float(f"{v:.7f}") for v in npref.CENTROIDS_F64]).astype(np.float32)
    assert np.array_equal(oracle.codebook(), want)


def test_boundaries_are_fp32_midpoints():
    c = npref.CENTROIDS_F64
    mids = ((c[:-1] + c[1:]) / 2).astype(np.float32)
    b = oracle.boundaries()
    assert b.dtype == np.float32 and b.shape == (15,)
    assert np.array_equal(b, mids)
    assert b[7] == 0.0
    # each boundary lies between its two centroids of the true optimum too
    ref = _lloyd_max_16()
    assert np.all((b > ref[:-1]) & (b < ref[1:]))


def test_inv_sqrt_pd_bits():
    bits = {pd: int(np.array([oracle.inv_sqrt_pd(pd)], np.float32).view(np.uint32)[0])
            for pd in (64, 128, 256)}
    assert bits == {64: 0x3E000000, 128: 0x3DB504F3, 256: 0x3D800000}
    # 0x3DB504F3 is the correctly rounded 1/sqrt(128)
    assert abs(float(np.float32(oracle.inv_sqrt_pd(128))) - 1 / math.sqrt(128)) < 2.0 ** -28


@pytest.mark.parametrize("n", [4, 64, 128, 256])
def test_fwht_matches_hadamard_matrix(n):
    h = hadamard(n)
    # unit vectors give the matrix columns; [1,0,0,0] -> [1,1,1,1] (x0.5 normalised)
    for j in (0, 1, n - 1):
        e = np.zeros(n, np.float32)
        e[j] = 1
        assert np.array_equal(oracle.fwht_f32(e), h[:, j].astype(np.float32))
    rng = np.random.default_rng(n)
    x = rng.integers(-1000, 1000, n).astype(np.float32)  # exact in fp32
    assert np.array_equal(oracle.fwht_f32(x), (h @ x.astype(np.int64)).astype(np.float32))


def test_bucketize_tie_goes_up():
    pd = 128
    sb = (oracle.boundaries() * oracle.inv_sqrt_pd(pd)).astype(np.float32)
    for j, b in enumerate(sb):
        assert oracle.bucketize(b, sb) == j + 1
        assert oracle.bucketize(np.nextafter(b, np.float32(-np.inf)), sb) == j
    assert oracle.bucketize(0.0, sb) == 8
    assert oracle.bucketize(-0.0, sb) == 8
    assert oracle.bucketize(-1e30, sb) == 0
    assert oracle.bucketize(1e30, sb) == 15


def test_f32_to_f16_is_ieee_rne():
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 5.96e-8, 2.98e-8, 2.99e-8,
                  6.1e-5, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf], np.float32)])
    # exact ties at the fp16 half-ulp
    t = (np.arange(1, 2000, dtype=np.float32) * 2 ** -10 + 2 ** -11 + 1).astype(np.float32)
    x = np.concatenate([x, t, -t])
    got = np.array([oracle.f32_to_f16_bits(v) for v in x], np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_to_f32_roundtrip():
    lib = oracle.lib()
    bits = np.arange(0, 65536, 7, dtype=np.uint32)
    bits = bits[(bits & 0x7C00) != 0x7C00]  # finite values
    got = np.array([lib.tq_oracle_f16_to_f32(int(b)) for b in bits], np.float32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(got, want)


def _vector_from_codes(codes, pd, signs):
    """x with rotated unit vector at the chosen centroids (far from boundaries)."""
    y = npref.CENTROIDS_F64[codes] / np.sqrt(pd)
    y /= np.linalg.norm(y)
    return (npref.rotation_matrix(pd, signs).T @ y), y


def test_kat_nibble_order_and_rotation_direction():
    pd = 128
    s = _signs(pd)
    base = np.array([11, 4, 12, 3, 11, 4, 10, 5] * 16)[:pd]
    codes = base.copy()
    codes[0], codes[1] = 10, 5
    x, y = _vector_from_codes(codes, pd, s)
    scaled = np.sort(npref.CENTROIDS_F64)[codes] / np.sqrt(pd)
    assert np.all(np.abs(y / scaled - 1) < 0.05)  # stays inside each code's cell
    ent = oracle.quantize_vec((x * 3.0).astype(np.float32), pd, s)
    assert ent[0] == 0xA5  # even dim in the high nibble
    assert np.array_equal(npref.unpack_codes(ent[:pd // 2]), codes.astype(np.uint8))
    norm16 = ent[pd // 2:].view(np.float16)
    assert np.all(norm16 == np.float16(3.0))


def test_zero_vector_and_padding():
    for hd, pd in ((64, 64), (96, 128), (128, 128), (256, 256)):
        s = _signs(pd)
        ent = oracle.quantize_vec(np.zeros(hd, np.float32), pd, s)
        assert np.all(ent[:pd // 2] == 0x88) and np.all(ent[pd // 2:] == 0)
    # head_dim 96 is zero-padded to 128 before the rotation
    rng = np.random.default_rng(3)
    x = rng.standard_normal(96).astype(np.float32)
    xp = np.zeros(128, np.float32)
    xp[:96] = x
    s = _signs(128)
    assert np.array_equal(oracle.quantize_vec(x, 128, s), oracle.quantize_vec(xp, 128, s))


@pytest.mark.parametrize("hd", [64, 96, 128, 256])
def test_quantize_matches_independent_float64_path(hd):
    pd = max(64, 1 << (hd - 1).bit_length())
    s = _signs(pd)
    rng = np.random.default_rng(100 + hd)
    x = rng.standard_normal((1500, hd)).astype(np.float16)
    x[:100] *= 30.0
    x[100:120, :4] *= 50.0
    got = np.stack([oracle.quantize_vec(r.astype(np.float32), pd, s) for r in x])
    codes, norms, rot = npref.quantize_rows(x.astype(np.float64), pd, s)
    gc = npref.unpack_codes(got[:, :pd // 2])
    bounds = (npref.CENTROIDS_F64[:-1] + npref.CENTROIDS_F64[1:]) / 2 / np.sqrt(pd)
    dist = np.min(np.abs(rot[..., None] - bounds), axis=-1)
    mism = gc != codes
    # disagreements only where fp32 evaluation order can matter (<= 4 fp32 ulp)
    assert np.all(dist[mism] <= 4 * np.spacing(np.float32(1.0 / np.sqrt(pd))))
    assert mism.sum() <= 3
    n16 = got[:, pd // 2:].copy().view(np.float16)
    assert np.all(n16 == n16[:, :1])
    assert np.array_equal(n16[:, 0], norms.astype(np.float32).astype(np.float16))


def test_write_layout_slots_and_pad_bytes():
    hd, pd, h, nb = 128, 128, 3, 4
    s = _signs(pd)
    rng = np.random.default_rng(11)
    k = rng.standard_normal((10, h, hd)).astype(np.float16)
    v = rng.standard_normal((10, h, hd)).astype(np.float16)
    slots = np.array([5, 63, 0, -1, 17, 64, 30, 31, 2, 40], np.int32)  # -1 and 64 skipped
    cache = np.full((2, nb, 16, h, 80), 0xEE, np.uint8)
    oracle.write_kv_cache(cache, k, v, s, slots, hd, pd)
    written = set()
    for i, sl in enumerate(slots):
        if sl < 0 or sl >= nb * 16:
            continue
        written.add(int(sl))
        for hh in range(h):
            for kv, src in ((0, k), (1, v)):
                e = cache[kv, sl // 16, sl % 16, hh]
                want = oracle.quantize_vec(src[i, hh].astype(np.float32), pd, s)
                assert np.array_equal(e[:68], want)
                assert np.all(e[68:] == 0xEE)  # pad bytes never written
    flat = cache.reshape(2, nb * 16, h, 80)
    for sl in range(nb * 16):
        if sl not in written:
            assert np.all(flat[:, sl] == 0xEE)


def _small_case(seed, seq_lens, hq, hkv, hd):
    c = W.decode_case(seed, len(seq_lens), seq_lens, hq, hkv, hd)
    pd = max(64, 1 << (hd - 1).bit_length())
    shape, _ = W.cache_bytes(c["num_blocks"], hkv, hd)
    cache = np.zeros(shape, np.uint8)
    s = _signs(pd)
    oracle.write_kv_cache(cache, c["k"], c["v"], s, c["slots"], hd, pd)
    bt = c["block_table"]
    ind = bt.reshape(-1)
    ip = (np.arange(len(seq_lens) + 1) * bt.shape[1]).astype(np.int32)
    q = np.zeros((len(seq_lens), hq, pd), np.float16)
    q[:, :, :hd] = c["q"][:, :, :hd]
    return c, cache, ind, ip, q, pd, s


@pytest.mark.parametrize("hd,hq,hkv", [(128, 8, 2), (64, 4, 4), (256, 4, 1), (96, 6, 2)])
def test_decode_matches_original_domain_fp64(hd, hq, hkv):
    c, cache, ind, ip, q, pd, s = _small_case(5 + hd, [37, 1, 130, 0], hq, hkv, hd)
    scale = 1.0 / math.sqrt(hd)
    got = oracle.decode(q, cache, ind, ip, c["seq_lens"], hkv, pd, scale, s)
    ref = npref.decode_original(q, cache, ind, ip, c["seq_lens"], hkv, pd, scale, s,
                                oracle.codebook())
    assert np.max(np.abs(got - ref)) < 2e-6
    assert np.all(got[3] == 0)


def test_decode_single_token_is_its_value():
    c, cache, ind, ip, q, pd, s = _small_case(9, [1, 1], 8, 2, 128)
    got = oracle.decode(q, cache, ind, ip, c["seq_lens"], 2, pd, 0.3, s)
    for b in range(2):
        for h in range(8):
            _, ve = npref.gather_entries(cache, ind, ip, 1, b, h // 4)
            vhat = npref.dequant_original(ve, pd, s, oracle.codebook())[0]
            assert np.max(np.abs(got[b, h] - vhat)) < 1e-6


def test_decode_page_permutation_invariance():
    c, cache, ind, ip, q, pd, s = _small_case(13, [200, 77], 8, 2, 128)
    base = oracle.decode(q, cache, ind, ip, c["seq_lens"], 2, pd, 0.1, s)
    nb = cache.shape[1]
    perm = np.random.default_rng(0).permutation(nb)
    cache2 = np.empty_like(cache)
    cache2[:, perm] = cache  # page p moves to perm[p]
    ind2 = perm[ind].astype(np.int32)
    got = oracle.decode(q, cache2, ind2, ip, c["seq_lens"], 2, pd, 0.1, s)
    assert np.array_equal(got, base)


def test_golden_signs_match_geometry():
    from turboquant_amd.geometry import hadamard_signs
    for pd in (64, 128, 256):
        assert np.array_equal(hadamard_signs(pd).numpy(), _signs(pd))


def test_golden_write_kat():
    kat = np.load(os.path.join(GOLDEN, "write_kat.npz"))
    for hd in (64, 96, 128, 256):
        pd = max(64, 1 << (hd - 1).bit_length())
        s = _signs(pd)
        x, e = kat[f"x{hd}"], kat[f"e{hd}"]
        got = np.stack([oracle.quantize_vec(r.astype(np.float32), pd, s) for r in x])
        assert np.array_equal(got, e)


def test_golden_cfg1():
    with open(os.path.join(GOLDEN, "cfg1.json")) as f:
        meta = json.load(f)
    c = W.cfg1()
    shape, pd = W.cache_bytes(c["num_blocks"], 8, 128)
    cache = np.zeros(shape, np.uint8)
    s = _signs(pd)
    oracle.write_kv_cache(cache, c["k"], c["v"], s, c["slots"], 128, pd)
    assert hashlib.sha256(cache.tobytes()).hexdigest() == meta["cache_sha256"]
    bt = c["block_table"]
    out = oracle.decode(c["q"], cache, bt.reshape(-1), np.array([0, bt.shape[1]], np.int32),
                        c["seq_lens"], 8, pd, meta["sm_scale"], s)
    want = np.load(os.path.join(GOLDEN, "cfg1_decode.npy"))
    assert np.max(np.abs(out - want)) <= 1e-7


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_torch_cpu_port_write_matches_oracle(hd):
    """The torch-CPU port (the bench's CPU baseline) writes the oracle's bytes,
    up to codes within a few ulp of a boundary (its sum of squares is torch's
    reduction, not the reference's lane tree)."""
    import torch

    from oracle import torch_ref
    rng = np.random.default_rng(hd)
    c = W.decode_case(17 + hd, 2, [300, 77], 8, 4, hd)
    shape, pd = W.cache_bytes(c["num_blocks"], 4, hd)
    s = _signs(pd)
    want = np.zeros(shape, np.uint8)
    oracle.write_kv_cache(want, c["k"], c["v"], s, c["slots"], hd, pd)
    got = torch.zeros(shape, dtype=torch.uint8)
    torch_ref.write_kv_cache(got, torch.from_numpy(c["k"]), torch.from_numpy(c["v"]),
                             torch.from_numpy(s), torch.from_numpy(c["slots"]), pd)
    got = got.numpy()
    n = pd // 2
    assert np.array_equal(got[..., n:], want[..., n:])  # norms and pad bytes
    diff = got[..., :n] != want[..., :n]
    assert diff.mean() < 1e-3, diff.mean()
    del rng


@pytest.mark.parametrize("hd,hq,hkv", [(128, 8, 2), (64, 4, 4), (256, 4, 1)])
def test_torch_cpu_port_decode_matches_oracle(hd, hq, hkv):
    import torch

    from oracle import torch_ref
    c, cache, ind, ip, q, pd, s = _small_case(29 + hd, [37, 1, 130, 0], hq, hkv, hd)
    scale = 1.0 / math.sqrt(hd)
    want = oracle.decode(q, cache, ind, ip, c["seq_lens"], hkv, pd, scale, s)
    bt = torch.from_numpy(ind.reshape(len(c["seq_lens"]), -1))
    got = torch_ref.decode(torch.from_numpy(q), torch.from_numpy(cache), bt,
                           torch.from_numpy(c["seq_lens"]), hkv, pd, scale,
                           torch.from_numpy(s)).numpy()
    assert np.max(np.abs(got - want)) < 2e-5
