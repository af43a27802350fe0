"""TurboQuant quantized paged-KV hot path for AMD Instinct MI355X (gfx950).

* ``turboquant_amd.ops`` — quantize-write and split-KV decode over the C ABI
  of libtq_hip.so (include/turboquant_amd.h), registered as the reference's
  torch.library ops.
* ``turboquant_amd.vllm_backend_fused`` — TurboQuantBackend / TurboQuantFusedImpl.
* ``turboquant_amd.vllm_plugin.register`` — vLLM general-plugin entry point.
"""
from .geometry import choose_splits, entry_bytes, hadamard_signs, padded_dim  # noqa: F401

__version__ = "0.1.0"
