"""configs[4] end to end, small: a 2-layer decoder with the Qwen3-8B attention
geometry (32/8/128) run through TurboQuantFusedImpl (write + prefill +
balanced decode).  Every layer's decode attention is checked against the
oracle's dequantize-then-attend (max-abs 2e-3 / rel 1e-2); the graph-captured
decode step must give the eager step's tokens on every replay; e2e.run's
tokens must agree with a dequantize-then-attend decode of the same model."""
import math

import numpy as np
import pytest
import torch

from tests import gpu_cases as G
from turboquant_amd import e2e
from turboquant_amd.geometry import hadamard_signs

pytestmark = pytest.mark.gpu


def _runner(batch=4, prompt=200, new=9, keep16=False, shape=None):
    shape = shape or e2e.ModelShape.tiny(2)
    r = e2e.Runner(shape, batch, prompt + new, G.DEV, seed=5, keep_fp16_kv=keep16)
    g = torch.Generator(device="cpu")
    g.manual_seed(7)
    prompts = torch.randint(0, shape.vocab, (batch, prompt), generator=g)
    for b in range(batch):
        r.prefill(b, prompts[b].to(G.DEV))
    torch.cuda.synchronize()
    return r


@pytest.mark.parametrize("hq,hkv,hd", [(32, 8, 128), (16, 2, 256), (16, 4, 64), (8, 2, 96)])
def test_e2e_decode_attention_matches_oracle_per_layer(hq, hkv, hd):
    """The whole backend flow (write, fresh-prompt prefill, balanced decode)
    at the configs[4] head geometry and at head sizes 256, 64 and 96 (the
    last padded to 128 in the cache and the kernels)."""
    print(f"case: e2e tiny 2 layers B=4 prompt 200 {hq}/{hkv}/{hd}, per-layer oracle", flush=True)
    import oracle
    from turboquant_amd.geometry import padded_dim
    shape = e2e.ModelShape(layers=2, hidden=512, heads=hq, kv_heads=hkv, head_dim=hd,
                           intermediate=1024, vocab=4096)
    r = _runner(shape=shape)
    r.probe = []
    r.decode_eager(1)
    torch.cuda.synchronize()
    probe, r.probe = r.probe, None
    assert len(probe) == r.shape.layers
    b = r.batch
    pd = padded_dim(hd)
    bt = r.block_table.cpu().numpy()
    indptr = np.arange(b + 1, dtype=np.int32) * bt.shape[1]
    seq = r.seq_lens.cpu().numpy()
    assert np.all(seq == 201)
    signs = hadamard_signs(pd).numpy()
    for li, q, _, _, o in probe:
        qp = np.zeros((b, hq, pd), np.float16)
        qp[:, :, :hd] = q.to(torch.float16).cpu().numpy()
        ref = oracle.decode(qp, r.caches[li].cpu().numpy(), bt.reshape(-1), indptr, seq, hkv, pd,
                            1.0 / math.sqrt(hd), signs)[:, :, :hd]
        got = o.float().cpu().numpy().reshape(b, hq, hd)
        G.assert_close(got, ref, f"e2e {hq}/{hkv}/{hd} layer {li}")


def test_e2e_graph_replays_equal_eager_tokens():
    print("case: e2e tiny graph replay vs eager tokens", flush=True)
    r = _runner()
    pos0, tok0 = r.pos.clone(), r.tok.clone()
    eager = r.decode_eager(8).clone()
    torch.cuda.synchronize()
    r.pos.copy_(pos0)
    r.tok.copy_(tok0)
    r.capture(8)
    for rep in range(3):
        r.pos.copy_(pos0)
        r.tok.copy_(tok0)
        torch.cuda.synchronize()
        got = r.decode_graph(8).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay round {rep}: {got.tolist()} vs {eager.tolist()}"
        # eager work between the replay rounds
        _ = (torch.randn(1000, device=G.DEV) * 2).sum().item()


def test_e2e_run_reports_serving_figures():
    print("case: e2e.run tiny, fp16-KV agreement", flush=True)
    res = e2e.run(e2e.ModelShape.tiny(2), batch=2, prompt_len=300, new_tokens=6, seed=3,
                  compare_steps=5)
    a16 = res["attention_vs_fp16"]  # 4-bit Lloyd-Max: a single vector keeps cos ~0.995
    assert a16["cosine_mean"] >= 0.99 and a16["cosine_min"] >= 0.97, a16
    for k in ("output_tok_s", "decode_tok_s", "tpot_ms", "ttft_s"):
        assert res[k] > 0, k
    a = res["agreement"]
    assert a["steps"] == 5
    for k in ("free_run_token_match_rate", "teacher_forced_top1_match_rate",
              "teacher_forced_in_top5_rate"):
        assert 0.0 <= a[k] <= 1.0, k
    print(f"agreement {a}", flush=True)
    # against dequantize-then-attend over the same quantized cache only the
    # fused kernel's arithmetic differs: the tokens must agree
    d = res["agreement_dequant"]
    assert d["steps"] == 5
    print(f"agreement with dequantize-then-attend {d}", flush=True)
    assert d["teacher_forced_top1_match_rate"] >= 0.8, d
    assert d["teacher_forced_in_top5_rate"] == 1.0, d
