"""Writes the committed fixtures of tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

* signs.json -- the rotation signs for pd 64/128/256: sign(randn(pd)) from a
  CPU torch.Generator seeded with 42, zeros mapped to +1 (the recipe of
  turboquant/vllm_backend_fused.py:217-224 and hadamard.py:52-60, run with
  torch only; no reference code is imported).
* write_kat.npz -- small write known-answer vectors: 48 fp16 rows per head
  size (64, 96, 128, 256; normal rows, rows scaled by 1e-3 and 1e3, a zero
  row, rows with a single non-zero, rows with outlier channels) and the
  entry bytes the C oracle produces for them.
* cfg1.json + cfg1_decode.npy -- configs[0] (seed 1): sha256 of the whole
  cache the oracle writes, and the oracle's decode output [1, 32, 128] f32.

The generator records what the oracle produced when the oracle was pinned by
the independent checks in tests/test_oracle.py; the fixtures then hold the
oracle (and the GPU path through it) to those bytes in later changes.
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def signs_fixture():
    import torch
    out = {}
    for pd in (64, 128, 256):
        g = torch.Generator(device="cpu")
        g.manual_seed(42)
        s = torch.sign(torch.randn(pd, generator=g))
        s[s == 0] = 1.0
        out[str(pd)] = [int(v) for v in s.tolist()]
    return out


def kat_rows(hd: int, rng) -> np.ndarray:
    rows = [rng.standard_normal(hd) for _ in range(32)]
    rows += [rng.standard_normal(hd) * 1e-3 for _ in range(4)]
    rows += [rng.standard_normal(hd) * 1e3 for _ in range(4)]
    rows.append(np.zeros(hd))
    for j in (0, 1, hd - 1):
        r = np.zeros(hd)
        r[j] = 1.0
        rows.append(r)
    for _ in range(4):
        r = rng.standard_normal(hd)
        r[rng.choice(hd, 3, replace=False)] *= 20.0
        rows.append(r)
    return np.stack(rows).astype(np.float16)


def main():
    import oracle
    from turboquant_amd import workloads as W
    oracle.build()
    signs = signs_fixture()
    with open(os.path.join(HERE, "signs.json"), "w") as f:
        json.dump(signs, f)

    rng = np.random.default_rng(1234)
    kat = {}
    for hd in (64, 96, 128, 256):
        pd = max(64, 1 << (hd - 1).bit_length())
        x = kat_rows(hd, rng)
        s = np.array(signs[str(pd)], np.float32)
        ent = np.stack([oracle.quantize_vec(r.astype(np.float32), pd, s) for r in x])
        kat[f"x{hd}"] = x
        kat[f"e{hd}"] = ent
    np.savez_compressed(os.path.join(HERE, "write_kat.npz"), **kat)

    c = W.cfg1()
    shape, pd = W.cache_bytes(c["num_blocks"], 8, 128)
    cache = np.zeros(shape, np.uint8)
    s = np.array(signs[str(pd)], np.float32)
    oracle.write_kv_cache(cache, c["k"], c["v"], s, c["slots"], 128, pd)
    bt = c["block_table"]
    out = oracle.decode(c["q"], cache, bt.reshape(-1), np.array([0, bt.shape[1]], np.int32),
                        c["seq_lens"], 8, pd, 1.0 / math.sqrt(128), s)
    np.save(os.path.join(HERE, "cfg1_decode.npy"), out.astype(np.float32))
    with open(os.path.join(HERE, "cfg1.json"), "w") as f:
        json.dump({"cache_shape": list(shape),
                   "cache_sha256": hashlib.sha256(cache.tobytes()).hexdigest(),
                   "sm_scale": 1.0 / math.sqrt(128)}, f, indent=1)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
