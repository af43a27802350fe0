"""configs[4] at its own size: a random-init Qwen3-8B-architecture model
(36 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, vocab 151936, fp16)
served through TurboQuantFusedImpl with 8 prompts of 32768 random tokens,
then a few decode steps over the quantized caches.

* Decode attention of layers 0, 17 and 35 in the first decode step is
  checked against the oracle's dequantize-then-attend over that layer's
  whole cache (max-abs 2e-3 / rel 1e-2), and against attention over the
  fp16 K/V the prefill produced (the quantization error itself: mean
  per-row cosine similarity >= 0.99, the bound the reference's quality
  checks use, reference tests/bench_int4_tc.py:510; every row >= 0.97; one
  4-bit Lloyd-Max vector alone keeps a cosine of about 0.995).
* The graph-captured decode step gives the eager step's tokens.
* Teacher-forced over the captured run's tokens, a decode of the same model
  whose attention reads the quantized cache back as fp16 rows (the
  reference's dequantize-then-attend, triton_decode_ref.py:264-299) picks
  the same top-1 token at >= 90% of the positions and always ranks the
  fused run's token in its top 5: the fused kernel's arithmetic alone
  differs between the two.
"""
import math

import numpy as np
import pytest
import torch

from tests import gpu_cases as G
from turboquant_amd import e2e
from turboquant_amd.geometry import hadamard_signs

pytestmark = pytest.mark.gpu

BATCH, PROMPT, STEPS = 8, 32768, 4
PROBE_LAYERS = (0, 17, 35)


@pytest.fixture(scope="module")
def runner():
    print(f"case: e2e configs[4] full size, B={BATCH} prompt={PROMPT}", flush=True)
    shape = e2e.ModelShape.qwen3_8b()
    r = e2e.Runner(shape, BATCH, PROMPT + STEPS + 2, G.DEV, seed=11, keep_fp16_kv=True)
    g = torch.Generator(device="cpu")
    g.manual_seed(12)
    prompts = torch.randint(0, shape.vocab, (BATCH, PROMPT), generator=g)
    for b in range(BATCH):
        r.prefill(b, prompts[b].to(G.DEV))
        torch.cuda.synchronize()
        print(f"  prefill {b + 1}/{BATCH}", flush=True)
    yield r
    del r
    torch.cuda.empty_cache()


def test_full_size_decode_attention_per_layer(runner):
    import oracle
    r = runner
    pos0, tok0 = r.pos.clone(), r.tok.clone()
    r.probe = []
    r.decode_eager(1)
    torch.cuda.synchronize()
    probe, r.probe = r.probe, None
    assert len(probe) == r.shape.layers
    eager_tok = r.out_buf[0].clone()
    b = r.batch
    bt = r.block_table.cpu().numpy()
    indptr = np.arange(b + 1, dtype=np.int32) * bt.shape[1]
    seq = r.seq_lens.cpu().numpy()
    assert np.all(seq == PROMPT + 1)
    signs = hadamard_signs(128).numpy()
    for li, q, k, v, o in probe:
        if li not in PROBE_LAYERS:
            continue
        print(f"  layer {li}: oracle over {int(seq.sum())} cached tokens", flush=True)
        qp = q.to(torch.float16).cpu().numpy()
        ref = oracle.decode(qp, r.caches[li].cpu().numpy(), bt.reshape(-1), indptr, seq, 8, 128,
                            1.0 / math.sqrt(128), signs)
        got = o.float().cpu().numpy().reshape(b, 32, 128)
        G.assert_close(got, ref, f"configs[4] layer {li}")
        f16 = r.fp16_attention(li, q, k, v).float().reshape(b * 32, 128)
        cos = torch.nn.functional.cosine_similarity(o.float().reshape(b * 32, 128), f16, dim=-1)
        print(f"  layer {li}: cosine vs fp16-KV attention min {cos.min().item():.5f} "
              f"mean {cos.mean().item():.5f}", flush=True)
        assert cos.mean().item() >= 0.99 and cos.min().item() >= 0.97, (li, cos.min().item())
    # the captured step replays the eager step's first token
    r.pos.copy_(pos0)
    r.tok.copy_(tok0)
    r.capture(STEPS)
    toks = r.decode_graph(STEPS).clone()
    torch.cuda.synchronize()
    assert torch.equal(toks[0], eager_tok), (toks[0].tolist(), eager_tok.tolist())
    runner.graph_tokens = toks


def test_full_size_teacher_forced_agreement_with_dequantize_then_attend(runner):
    toks = getattr(runner, "graph_tokens", None)
    if toks is None:
        pytest.skip("needs the decode of test_full_size_decode_attention_per_layer")
    top, rank = runner.decode_fp16_reference(STEPS, forced=toks, kv="dequant")
    torch.cuda.synchronize()
    match = (top == toks).float().mean().item()
    print(f"  teacher-forced top-1 agreement {match:.3f}, max rank {int(rank.max())}", flush=True)
    assert match >= 0.9, match
    assert int(rank.max()) < 5
