"""TurboQuant quantized paged-KV hot path for AMD Instinct MI355X (gfx950).

* ``turboquant_amd.ops`` — quantize-write and split-KV decode over the C ABI
  of libtq_hip.so (include/turboquant_amd.h), registered as the reference's
  torch.library ops.
* ``turboquant_amd.vllm_backend_fused`` — TurboQuantBackend / TurboQuantFusedImpl.
* ``turboquant_amd.vllm_plugin.register`` — vLLM general-plugin entry point.
* ``turboquant_amd.algorithm`` — the TurboQuant quantizers (TurboQuantMSE,
  TurboQuantProd, QJL, Codebook, RandomHadamardRotation, fwht), also importable
  from the package as in the reference (turboquant/__init__.py:9-22).
"""
from .geometry import choose_splits, entry_bytes, hadamard_signs, padded_dim  # noqa: F401

__version__ = "0.1.0"

_ALGORITHM = ("TurboQuantMSE", "TurboQuantProd", "RandomHadamardRotation", "Codebook", "QJL",
              "fwht")


def __getattr__(name):  # the algorithm names load torch only when asked for
    if name in _ALGORITHM:
        from . import algorithm
        return getattr(algorithm, name)
    raise AttributeError(name)
