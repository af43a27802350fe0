"""vLLM plugin entry point (reference turboquant/vllm_plugin.py:85-92).

Declared in pyproject.toml as
``[project.entry-points."vllm.general_plugins"] turboquant = "turboquant.vllm_plugin:register"``
(``turboquant.X`` is this module under the reference's import path).
``register()`` is idempotent and maps the ``CUSTOM`` attention backend to
``turboquant.vllm_backend_fused.TurboQuantBackend`` (the registration the
reference's archived CUSTOM backend needs; its snapshot only patches Triton
kernels).  vLLM is imported inside the function, never at module import.
"""
from __future__ import annotations

BACKEND_PATH = "turboquant.vllm_backend_fused.TurboQuantBackend"

_registered = False
_registration: str | None = None  # how the backend was registered (diagnostics)


def _register_custom_backend() -> str | None:
    try:
        from vllm.v1.attention.backends.registry import (AttentionBackendEnum,
                                                         register_backend)
    except Exception:
        try:
            from vllm.attention.backends.registry import (AttentionBackendEnum,  # type: ignore
                                                          register_backend)
        except Exception:
            return None
    register_backend(AttentionBackendEnum.CUSTOM, BACKEND_PATH)
    return "registry.register_backend(CUSTOM)"


def register() -> None:
    """Called once by vLLM at startup; safe to call again."""
    global _registered, _registration
    if _registered:
        return
    _registered = True
    from . import ops
    try:
        ops.register_ops()
    except Exception as e:  # torch without the library API: ops register on first use
        print(f"[tq-plugin] op registration deferred: {e}", flush=True)
    _registration = _register_custom_backend()
