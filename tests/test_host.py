"""CPU tests of the host side: geometry, split heuristic, backend class
surface (reference turboquant/vllm_backend_fused.py:32-86), dispatch
(reference tests/test_decoder_dispatch.py), plugin registration, and the
C-ABI library: every symbol include/turboquant_amd.h declares is exported,
argument errors come back as codes + messages without touching a GPU, and a
missing library fails loudly."""
import ctypes
import math
import os
import re

import pytest
import torch

from turboquant_amd import _lib, geometry
from turboquant_amd.geometry import choose_splits, entry_bytes, padded_dim

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "turboquant_amd.h")


def _header_symbols():
    text = open(HEADER).read()
    return set(re.findall(r"^(?:int|int32_t|int64_t|const char\*)\s+(tq_\w+)\(", text, re.M))


def test_geometry_table():
    assert [padded_dim(h) for h in (32, 64, 80, 96, 128, 200, 256)] == [64, 64, 128, 128, 128,
                                                                        256, 256]
    assert entry_bytes(64) == (32, 2, 48)
    assert entry_bytes(96) == (64, 4, 80)
    assert entry_bytes(128) == (64, 4, 80)
    assert entry_bytes(256) == (128, 8, 144)


@pytest.mark.parametrize("batch,max_len,hkv,hq,pd", [
    (8, 32768, 8, 32, 128), (1, 1024, 8, 32, 128), (64, 32768, 8, 32, 128),
    (8, 32768, 2, 16, 256), (8, 4096, 4, 16, 64), (3, 17, 8, 32, 128), (1, 1, 1, 1, 128),
    (2, 100000, 1, 16, 128)])
def test_choose_splits_invariants(batch, max_len, hkv, hq, pd):
    s, c = choose_splits(batch, max_len, hkv, hq, pd)
    assert s >= 1 and c % 16 == 0 and c >= 16
    assert s * c >= max_len and (s - 1) * c < max_len  # no empty trailing split
    if s > 1:
        assert c >= geometry.MIN_CHUNK_TOKENS
    assert choose_splits(batch, max_len, hkv, hq, pd) == (s, c)  # pure


def test_choose_splits_fills_one_round_of_workgroups():
    # B=8, 8 kv heads in one workgroup, 2 workgroups per CU at hd 128
    assert geometry.decode_workgroup_shape(32, 8, 128) == (8, 2)
    assert choose_splits(8, 32768, 8, 32, 128) == (64, 512)


def test_backend_surface():
    from turboquant_amd.vllm_backend_fused import TurboQuantBackend, TurboQuantFusedImpl
    assert TurboQuantBackend.get_name() == "CUSTOM"
    assert TurboQuantBackend.forward_includes_kv_cache_update is False
    assert TurboQuantBackend.get_impl_cls() is TurboQuantFusedImpl
    for dt in ("fp8", "fp8_e4m3"):
        assert TurboQuantBackend.supports_kv_cache_dtype(dt)
        assert TurboQuantBackend.get_kv_cache_shape(100, 16, 8, 128, dt) == (2, 100, 16, 8, 80)
        assert TurboQuantBackend.get_kv_cache_shape(7, 32, 2, 64, dt) == (2, 7, 32, 2, 48)
        assert TurboQuantBackend.get_kv_cache_page_size(16, 8, 128, torch.uint8, dt) == 20480
        assert TurboQuantBackend.get_kv_cache_page_size(16, 2, 256, torch.uint8, dt) == 9216
    assert TurboQuantBackend.get_kv_cache_page_size(16, 8, 128, torch.float16, "auto") is None


def test_impl_constructor_and_signs():
    from turboquant_amd.vllm_backend_fused import TurboQuantFusedImpl
    impl = TurboQuantFusedImpl(32, 128, 1 / math.sqrt(128), 8, None, None, "fp8")
    assert impl.kv_cache_dtype == "fp8" and impl._pd == 128
    assert impl._qbytes == 64 and impl._nbytes == 4
    impl96 = TurboQuantFusedImpl(16, 96, 0.1, 4, None, None, "fp8_e4m3")
    assert impl96._pd == 128 and impl96._qbytes == 64


def test_signs_recipe():
    s = geometry.hadamard_signs(128)
    g = torch.Generator(device="cpu")
    g.manual_seed(42)
    r = torch.sign(torch.randn(128, generator=g))
    r[r == 0] = 1
    assert torch.equal(s, r) and set(s.tolist()) <= {-1.0, 1.0}


def test_dispatch_forced_names(monkeypatch):
    from turboquant_amd import decoder_dispatch as dd
    for name, exc in (("v5", RuntimeError), ("v7", RuntimeError), ("bogus", ValueError)):
        monkeypatch.setenv("TQ_FORCE_KERNEL", name)
        dd.pick_decode_op.cache_clear()
        with pytest.raises(exc, match=name):
            dd.pick_decode_op()
    dd.pick_decode_op.cache_clear()


def test_dispatch_default_registers_reference_op_names(monkeypatch):
    from turboquant_amd import decoder_dispatch as dd
    monkeypatch.delenv("TQ_FORCE_KERNEL", raising=False)
    dd.pick_decode_op.cache_clear()
    op, name = dd.pick_decode_op()
    assert name == dd.KERNEL_NAME
    assert hasattr(torch.ops.turboquant_v5, "decode_v5_from_cache_paged_splitkv_ws")
    assert hasattr(torch.ops.turboquant_write, "quantize_write_kv_cache")
    dd.pick_decode_op.cache_clear()


def test_plugin_register_idempotent():
    from turboquant_amd import vllm_plugin
    vllm_plugin.register()
    vllm_plugin.register()
    assert hasattr(torch.ops.turboquant_write, "quantize_write_kv_cache")


def test_cabi_exports_every_header_symbol():
    syms = _header_symbols()
    assert syms == set(_lib.SIGNATURES), (syms, set(_lib.SIGNATURES))
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for s in syms:
        assert hasattr(lib, s), s
    loaded = _lib.load()
    assert loaded.tq_abi_version() == _lib.ABI_VERSION


def test_cabi_argument_errors_without_gpu():
    lib = _lib.load()
    null = None
    # padded_dim 100 is not a supported head geometry
    rc = lib.tq_decode_paged_splitkv(null, 0, 0, null, null, null, null, null, 1, 32, 8, 100,
                                     100, 16, 80, 10, 0.1, null, 1, 16, null, null, null, null)
    assert rc == -22
    assert b"padded_dim" in lib.tq_last_error()
    # GQA ratio must divide
    rc = lib.tq_decode_paged_splitkv(null, 0, 0, null, null, null, null, null, 1, 30, 8, 128,
                                     128, 16, 80, 10, 0.1, null, 1, 16, null, null, null, null)
    assert rc == -22
    # wrong entry size for the head size
    rc = lib.tq_quantize_write_kv_cache(null, null, null, null, 1, 0, 0, 0, 0, null, null, 4, 8,
                                        128, 128, 16, 96, 10, null)
    assert rc == -22 and lib.tq_last_error()
    rc = lib.tq_combine_splits(null, null, 1, 0, 32, 128, null, null, null)
    assert rc == -22
    # prefill attention: head size 64, 128 or 256 only, GQA ratio must divide, q_len <= kv_len
    rc = lib.tq_prefill_attention(null, 0, 0, null, 0, 0, null, 0, 0, null, 0, 0, 4, 4, 32, 8,
                                  96, 0.1, null)
    assert rc == -22 and b"head_dim" in lib.tq_last_error()
    rc = lib.tq_prefill_attention(null, 0, 0, null, 0, 0, null, 0, 0, null, 0, 0, 4, 4, 30, 8,
                                  128, 0.1, null)
    assert rc == -22 and b"multiple" in lib.tq_last_error()
    rc = lib.tq_prefill_attention(null, 0, 0, null, 0, 0, null, 0, 0, null, 0, 0, 5, 4, 32, 8,
                                  128, 0.1, null)
    assert rc == -22 and b"q_len" in lib.tq_last_error()
    # prefill workspace query: invalid shapes need none
    assert lib.tq_prefill_workspace_bytes(0, 10, 32, 8, 128) == 0
    assert lib.tq_prefill_workspace_bytes(10, 5, 32, 8, 128) == 0
    assert lib.tq_prefill_workspace_bytes(10, 100, 32, 8, 96) == 0
    rc = lib.tq_prefill_attention_ws(null, 0, 0, null, 0, 0, null, 0, 0, null, 0, 0, 4, 4, 32, 8,
                                     96, 0.1, null, 0, null)
    assert rc == -22 and b"head_dim" in lib.tq_last_error()
    # an empty batch is a no-op that succeeds
    assert lib.tq_combine_splits(null, null, 0, 1, 32, 128, null, null, null) == 0
    # the stream-read diagnostic: null source, size not a multiple of 16
    assert lib.tq_diag_stream_read(null, 16, null, null) == -22
    assert lib.tq_diag_stream_read(ctypes.c_void_p(256), 24, ctypes.c_void_p(256), null) == -22
    assert lib.tq_diag_stream_read(ctypes.c_void_p(256), 0, ctypes.c_void_p(256), null) == 0


def test_missing_library_raises(monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", os.path.join(ROOT, "no_such_dir", "libtq_hip.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()


def test_ops_raise_instead_of_falling_back(monkeypatch):
    from turboquant_amd import ops
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", os.path.join(ROOT, "no_such_dir", "libtq_hip.so"))
    cache = torch.zeros((2, 4, 16, 8, 80), dtype=torch.uint8)
    k = torch.zeros((3, 8, 128), dtype=torch.float16)
    with pytest.raises(RuntimeError):
        ops.quantize_write_kv_cache(cache, k, k, geometry.hadamard_signs(128),
                                    torch.zeros(3, dtype=torch.int32), 128, 128)


def test_reference_import_path_is_the_same_modules():
    """The reference's callers import turboquant.vllm_plugin,
    turboquant.vllm_backend_fused and turboquant.decoder_dispatch
    (reference tests/bench_vllm_serve.py:54, tests/test_decoder_dispatch.py:17)."""
    import turboquant
    import turboquant.vllm_plugin
    import turboquant_amd.vllm_plugin
    from turboquant.decoder_dispatch import pick_decode_op
    from turboquant.vllm_backend_fused import TurboQuantBackend, TurboQuantFusedImpl
    from turboquant_amd import decoder_dispatch, vllm_backend_fused
    assert turboquant.vllm_plugin is turboquant_amd.vllm_plugin
    assert pick_decode_op is decoder_dispatch.pick_decode_op
    assert TurboQuantBackend is vllm_backend_fused.TurboQuantBackend
    assert TurboQuantBackend.get_impl_cls() is TurboQuantFusedImpl
    assert turboquant_amd.vllm_plugin.__spec__.name == "turboquant_amd.vllm_plugin"
    from turboquant import QJL, Codebook, TurboQuantMSE, fwht  # noqa: F401
    with pytest.raises(ModuleNotFoundError):
        import turboquant.no_such_module  # noqa: F401


def test_plugin_entry_point_names_the_reference_path():
    text = open(os.path.join(ROOT, "pyproject.toml")).read()
    assert 'turboquant = "turboquant.vllm_plugin:register"' in text
    import importlib
    mod, fn = "turboquant.vllm_plugin:register".split(":")
    assert callable(getattr(importlib.import_module(mod), fn))


def test_plugin_registers_custom_backend_with_vllm_registry(monkeypatch):
    """register() maps CUSTOM to turboquant.vllm_backend_fused.TurboQuantBackend
    through vLLM's registry (reference turboquant/vllm_plugin.py:85-92), checked
    against a stand-in registry module, since vLLM is not installed here."""
    import enum
    import importlib
    import sys
    import types

    calls = []

    class AttentionBackendEnum(enum.Enum):
        FLASH_ATTN = "FLASH_ATTN"
        CUSTOM = "CUSTOM"

    reg = types.ModuleType("vllm.v1.attention.backends.registry")
    reg.AttentionBackendEnum = AttentionBackendEnum
    reg.register_backend = lambda which, path: calls.append((which, path))
    for name in ("vllm", "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backends"):
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    monkeypatch.setitem(sys.modules, "vllm.v1.attention.backends.registry", reg)
    import turboquant.vllm_plugin as plugin
    monkeypatch.setattr(plugin, "_registered", False)
    plugin.register()
    plugin.register()  # idempotent: one registration
    assert calls == [(AttentionBackendEnum.CUSTOM,
                      "turboquant.vllm_backend_fused.TurboQuantBackend")]
    # vLLM resolves the registered path by import + attribute
    mod, cls = calls[0][1].rsplit(".", 1)
    backend = getattr(importlib.import_module(mod), cls)
    assert backend.get_name() == "CUSTOM"
    assert backend.get_kv_cache_shape(10, 16, 8, 128, "fp8") == (2, 10, 16, 8, 80)


def test_fake_impls_trace_without_running():
    """Meta kernels for torch.compile / graph tracing: shapes only, no launch."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from turboquant_amd import ops
    ops.register_ops()
    with FakeTensorMode():
        q = torch.empty(8, 32, 128, dtype=torch.float16)
        cache = torch.empty(2, 10, 16, 8, 80, dtype=torch.uint8)
        i = torch.empty(10, dtype=torch.int32)
        po, pl = torch.empty(8, 32, 128), torch.empty(8, 32)
        o = torch.ops.turboquant_v5.decode_v5_from_cache_paged_splitkv_ws(
            q, cache, i, i, i, i, 8, 16, 128, 128, 0.1, torch.empty(128), 64, 4, q, 100, po,
            pl, i, i, i, i, 1)
        assert o.shape == (8, 32, 128) and o.dtype == torch.float16
        k = torch.empty(3, 8, 128)
        torch.ops.turboquant_write.quantize_write_kv_cache(cache, k, k, torch.empty(128), i,
                                                           128, 128)


def test_write_refuses_rows_narrower_than_head_dim():
    from turboquant_amd import ops
    cache = torch.zeros((2, 4, 16, 8, 80), dtype=torch.uint8)
    k = torch.zeros((3, 8, 96), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="fewer than head_dim"):
        ops.quantize_write_kv_cache(cache, k, k, geometry.hadamard_signs(128),
                                    torch.zeros(3, dtype=torch.int32), 128, 128)


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_impl_hadamard_helpers_match_the_matrix(hd):
    """The impl's torch rotation helpers (the reference keeps them on its impl):
    _fwht is the Sylvester-Hadamard product, _hadamard_forward is
    H (s * q) / sqrt(d), and _hadamard_inverse undoes it."""
    from scipy.linalg import hadamard

    from turboquant_amd.geometry import hadamard_signs
    from turboquant_amd.vllm_backend_fused import TurboQuantFusedImpl
    impl = TurboQuantFusedImpl(8, hd, 1.0 / math.sqrt(hd), 2, None, None, "fp8")
    g = torch.Generator().manual_seed(hd)
    x = torch.randn(3, 5, hd, generator=g, dtype=torch.float64)
    H = torch.from_numpy(hadamard(hd).astype("float64"))
    assert torch.allclose(TurboQuantFusedImpl._fwht(x), x @ H.T, rtol=0, atol=1e-12)
    s = hadamard_signs(hd).double()
    q = torch.randn(4, 8, hd, generator=g).float()
    got = impl._hadamard_forward(q)
    want = ((q.double() * s) @ H.T / math.sqrt(hd)).float()
    assert got.dtype == q.dtype and torch.allclose(got, want, rtol=0, atol=1e-5)
    back = impl._hadamard_inverse(got)
    assert torch.allclose(back, q, rtol=0, atol=1e-5)


def test_balanced_op_schema_declares_its_writes():
    """decode_paged_balanced_ws writes o_ws, the partial rows, the LSEs and
    the row table: its schema marks them (a!)..(d!) and returns nothing, and
    an exported, functionalized graph keeps the call, with the caller's use
    of o_ws reading the op's written value (so neither is dead code)."""
    from turboquant_amd import ops
    ops.register_ops()
    op = torch.ops.turboquant_v5.decode_paged_balanced_ws
    sch = op.default._schema
    written = {a.name for a in sch.arguments if a.alias_info is not None and a.alias_info.is_write}
    assert written == {"o_ws", "partition_o_ws", "partition_lse_ws", "split_indptr"}
    assert len(sch.returns) == 0

    class Step(torch.nn.Module):
        def forward(self, q, cache, i, sl, o, po, pl, si, signs):
            op(q, cache, i, i, sl, 8, 128, 128, 0.1, signs, o, po, pl, si)
            return o * 2

    args = (torch.empty(8, 32, 128, dtype=torch.float16),
            torch.empty(2, 10, 16, 8, 80, dtype=torch.uint8), torch.empty(10, dtype=torch.int32),
            torch.empty(10, dtype=torch.int32), torch.empty(8, 32, 128, dtype=torch.float16),
            torch.empty(16, 32, 128), torch.empty(16, 32), torch.empty(10, dtype=torch.int32),
            torch.empty(128))
    ep = torch.export.export(Step(), args).run_decompositions()
    nodes = list(ep.graph.nodes)
    fn = [n for n in nodes if n.op == "call_function" and "auto_functionalized" in str(n.target)]
    assert len(fn) == 1, ep.graph_module.code
    mul = [n for n in nodes if n.op == "call_function" and "mul" in str(n.target)]
    assert len(mul) == 1
    src = mul[0].args[0]  # getitem of the functionalized op: o_ws as written
    assert src.op == "call_function" and src.args[0] is fn[0], ep.graph_module.code


def test_mse_entry_points_refuse_bad_arguments():
    """tq_mse_quantize / tq_mse_dequantize argument checks (no GPU call)."""
    from turboquant_amd import _lib
    lib = _lib.load()
    null = None
    tab = (ctypes.c_float * 16)()
    # bit width out of range
    assert lib.tq_mse_quantize(null, 4, 128, 128, 5, null, tab, null, null, null) == -22
    assert b"bit_width" in lib.tq_last_error()
    # padded size not the power of two next to dim, or out of 64..1024
    assert lib.tq_mse_quantize(null, 4, 60, 128, 4, null, tab, null, null, null) == -22
    assert lib.tq_mse_quantize(null, 4, 32, 32, 4, null, tab, null, null, null) == -22
    assert lib.tq_mse_dequantize(null, null, 4, 2048, 2048, 4, null, tab, null, null) == -22
    assert b"padded_dim" in lib.tq_last_error()
    # null pointers with work to do
    assert lib.tq_mse_dequantize(null, null, 4, 128, 128, 4, null, tab, null, null) == -22
    # nothing to do: success without touching a pointer
    assert lib.tq_mse_quantize(null, 0, 128, 128, 4, null, tab, null, null, null) == 0


def test_prod_entry_points_refuse_bad_arguments():
    """tq_prod_quantize / tq_prod_dequantize argument checks (no GPU call):
    the residual outputs and the QJL term are required, and the MSE checks
    apply to the MSE stage's bit width."""
    from turboquant_amd import _lib
    lib = _lib.load()
    null = None
    tab = (ctypes.c_float * 16)()
    assert lib.tq_prod_quantize(null, 4, 128, 128, 3, null, tab, tab, null, null, null, null,
                                null) == -22
    assert b"null pointer" in lib.tq_last_error()
    assert lib.tq_prod_dequantize(null, null, null, null, 4, 128, 128, 3, null, tab, null,
                                  null) == -22
    assert b"null pointer" in lib.tq_last_error()
    one = ctypes.c_void_p(16)  # never dereferenced: the checks fail first
    assert lib.tq_prod_quantize(one, 4, 128, 128, 5, one, tab, tab, one, one, one, one,
                                null) == -22
    assert b"bit_width" in lib.tq_last_error()
    assert lib.tq_prod_dequantize(one, one, one, one, 4, 60, 128, 3, one, tab, one,
                                  null) == -22
    assert b"padded_dim" in lib.tq_last_error()
    # the fused QJL kernels: padded sizes 64 and 128 only, all operands required
    assert lib.tq_prod_quantize_qjl(one, 4, 200, 256, 3, one, tab, tab, one, one, one, one, one,
                                    one, null) == -22
    assert b"padded_dim" in lib.tq_last_error()
    assert lib.tq_prod_quantize_qjl(one, 4, 128, 128, 3, one, tab, tab, null, one, one, one, one,
                                    one, null) == -22
    assert b"null pointer" in lib.tq_last_error()
    assert lib.tq_prod_dequantize_qjl(one, one, one, one, 4, 128, 128, 3, one, tab, one, null,
                                      one, null) == -22
    assert b"null pointer" in lib.tq_last_error()
    assert lib.tq_prod_dequantize_qjl(one, one, one, one, 0, 128, 128, 3, one, tab, one, one,
                                      one, null) == 0
    # qjl_signs rows are read and written in 4- and 8-byte pieces: the base
    # must be 8-byte aligned
    odd = ctypes.c_void_p(20)
    assert lib.tq_prod_quantize_qjl(one, 4, 128, 128, 3, one, tab, tab, one, one, one, one, odd,
                                    one, null) == -22
    assert b"8-byte aligned" in lib.tq_last_error()
    assert lib.tq_prod_dequantize_qjl(one, one, odd, one, 4, 128, 128, 3, one, tab, one, one,
                                      one, null) == -22
    assert b"8-byte aligned" in lib.tq_last_error()


def test_ops_refuse_tensors_on_two_devices():
    """The ops check that every tensor is on one GPU before any launch (CPU
    tensors are refused the same way)."""
    from turboquant_amd import ops
    with pytest.raises(RuntimeError, match="GPU only"):
        ops._require_gpu(torch.zeros(1))

    class FakeCuda:
        is_cuda = True

        def __init__(self, i):
            self.device = torch.device("cuda", i)

    ops._require_gpu(FakeCuda(0), FakeCuda(0))
    with pytest.raises(RuntimeError, match="one GPU"):
        ops._require_gpu(FakeCuda(0), FakeCuda(1))


def test_e2e_glue_entry_points_refuse_bad_arguments():
    """tq_e2e_* argument checks (no GPU call)."""
    from turboquant_amd import _lib
    lib = _lib.load()
    one = ctypes.c_void_p(16)
    assert lib.tq_e2e_add_rms_norm(one, one, one, one, 4, 4100, 1e-6, None) == -22
    assert b"hidden" in lib.tq_last_error()
    assert lib.tq_e2e_add_rms_norm(one, one, one, one, 4, 16384, 1e-6, None) == -22
    assert lib.tq_e2e_add_rms_norm(one, None, one, None, 4, 4096, 1e-6, None) == -22
    assert lib.tq_e2e_add_rms_norm(one, one, None, one, 4, 4096, 1e-6, None) == -22
    assert b"null pointer" in lib.tq_last_error()
    assert lib.tq_e2e_add_rms_norm(ctypes.c_void_p(18), one, None, None, 4, 4096, 1e-6,
                                   None) == -22
    assert b"aligned" in lib.tq_last_error()
    assert lib.tq_e2e_add_rms_norm(None, None, None, None, 0, 4096, 1e-6, None) == 0
    assert lib.tq_e2e_qk_norm_rope(one, 6144, one, one, one, one, 100, one, 4, 32, 8, 97, 1e-6,
                                   one, one, None) == -22
    assert b"head_dim" in lib.tq_last_error()
    assert lib.tq_e2e_qk_norm_rope(one, 1000, one, one, one, one, 100, one, 4, 32, 8, 128, 1e-6,
                                   one, one, None) == -22
    assert lib.tq_e2e_qk_norm_rope(one, 6144, one, one, None, one, 100, one, 4, 32, 8, 128, 1e-6,
                                   one, one, None) == -22
    assert lib.tq_e2e_qk_norm_rope(one, 6144, one, one, one, one, -1, one, 4, 32, 8, 128, 1e-6,
                                   one, one, None) == -22
    assert b"geometry" in lib.tq_last_error()
    assert lib.tq_e2e_silu_mul(one, one, 4, 12, None) == -22
    assert lib.tq_e2e_silu_mul(one, None, 4, 16, None) == -22
    assert lib.tq_e2e_silu_mul(None, None, 0, 16, None) == 0


def test_bench_refuses_more_than_one_gpu_and_imports_no_tests():
    """bench.py --gpus N > 1 exits non-zero with a message saying the build
    is one-GPU (no GPU call happens before that check), and the measurement
    harness imports nothing from tests/."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "--gpus 2 is not supported" in (r.stdout + r.stderr)
    src = open(os.path.join(root, "bench.py")).read()
    assert "from tests" not in src and "import tests" not in src


def test_balanced_batch_limit_matches_the_kernel():
    """The backend routes decode batches above BALANCED_MAX_BATCH to the
    static-split op; the constant is the kernel's plan limit."""
    from turboquant_amd.geometry import BALANCED_MAX_BATCH
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = open(os.path.join(root, "turboquant_amd", "csrc", "tq_decode.hip")).read()
    m = re.search(r"constexpr int kPlanMaxBatch = (\d+);", src)
    assert m and int(m.group(1)) == BALANCED_MAX_BATCH
