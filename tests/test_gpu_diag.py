"""The measurement diagnostics of the C ABI (no counterpart in the reference):
tq_diag_decode_stream (the configs[2] partials kernel without its math, or
reduced to its copy ring) and tq_diag_stream_read (a plain streaming read).
They compute no attention; these tests check that they run on valid
inputs, store only what they document and refuse what they do not cover."""
import math

import pytest
import torch

from tests import gpu_cases as G
from turboquant_amd import workloads as W
from turboquant_amd import _lib
from turboquant_amd.geometry import hadamard_signs

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("nbytes", [16, 1 << 20, (1 << 20) + 48, 96 << 20])
def test_stream_read_runs_and_leaves_sink(nbytes):
    print(f"case: diag stream read {nbytes} bytes", flush=True)
    lib = _lib.load()
    g = torch.Generator(device=G.DEV).manual_seed(nbytes)
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=G.DEV, generator=g)
    sink = torch.zeros(4, dtype=torch.int32, device=G.DEV)
    assert lib.tq_diag_stream_read(src.data_ptr(), nbytes, sink.data_ptr(), _stream()) == 0
    torch.cuda.synchronize()
    # the sink is written only by a lane whose xor of the words it read is
    # 0x7e57c0de (for these seeded bytes none is)
    assert sink.abs().sum().item() == 0


def test_decode_stream_modes():
    print("case: diag decode stream modes 0/1, B=2, 32q/8kv/128", flush=True)
    lib = _lib.load()
    lens = [512, 300]
    c = W.decode_case(17, len(lens), lens, 32, 8, 128)
    cache, pd = G.build_cache(c)
    d = G.decode_inputs(c, pd)
    b, hq, hkv, S, cs = len(lens), 32, 8, 2, 256
    ebs = cache.shape[-1]
    signs = hadamard_signs(pd, G.DEV)
    scale = 1.0 / math.sqrt(128)
    po = torch.full((b * S, hq, pd), 7.0, dtype=torch.float32, device=G.DEV)
    pl = torch.full((b * S, hq), 7.0, dtype=torch.float32, device=G.DEV)

    def call(mode, num_splits=S):
        return lib.tq_diag_decode_stream(
            d["q"].data_ptr(), d["q"].stride(0), d["q"].stride(1), cache.data_ptr(),
            cache.data_ptr() + cache[0].numel(), d["indices"].data_ptr(), d["indptr"].data_ptr(),
            d["seq"].data_ptr(), b, hq, hkv, pd, W.BLOCK, ebs, c["num_blocks"], scale,
            signs.data_ptr(), num_splits, cs, po.data_ptr(), pl.data_ptr(), mode, _stream())

    # mode 0 (bare ring) stores nothing
    assert call(0) == 0
    torch.cuda.synchronize()
    assert bool((po == 7.0).all()) and bool((pl == 7.0).all())
    # mode 1 (no math) stores its (zero) partial rows: the first half of each
    # row's bytes, as fp16 rows of pd elements
    assert call(1) == 0
    torch.cuda.synchronize()
    rows16 = po.view(torch.float16).view(-1)[: b * S * hq * pd]
    assert bool((rows16 == 0).all())
    # unknown mode, bad split sizes
    assert call(2) == -22 and b"mode" in lib.tq_last_error()
    assert call(0, num_splits=0) == -22
