"""The reference's import path, ``turboquant``, over this build's package.

The reference's callers import ``turboquant.vllm_plugin``,
``turboquant.vllm_backend_fused`` and ``turboquant.decoder_dispatch``
(reference tests/bench_vllm_serve.py:54, tests/profile_decode_step.py:31,
tests/test_decoder_dispatch.py:17), vLLM's plugin loader resolves
``turboquant.vllm_plugin:register`` (reference pyproject.toml:20-21), and users
import the quantizers from the package itself (turboquant/__init__.py:9-22).

Every ``turboquant.<name>`` resolves to the module ``turboquant_amd.<name>``
itself (one module object under two names, so module state such as the
plugin's registration flag is shared).  Submodules load on first import,
never here: importing the plugin must not import vLLM or the backend.
"""
from __future__ import annotations

import importlib
import importlib.abc
import importlib.util
import sys

_REAL = "turboquant_amd"

__version__ = "0.1.0"
__all__ = ["TurboQuantMSE", "TurboQuantProd", "RandomHadamardRotation", "Codebook", "QJL",
           "fwht"]


class _AliasFinder(importlib.abc.MetaPathFinder, importlib.abc.Loader):
    """Finds ``turboquant.X`` as the already-importable ``turboquant_amd.X``."""

    def __init__(self):
        self._specs = {}

    def find_spec(self, fullname, path=None, target=None):
        if not fullname.startswith(__name__ + "."):
            return None
        real = _REAL + fullname[len(__name__):]
        try:
            if importlib.util.find_spec(real) is None:
                return None
        except ModuleNotFoundError:
            return None
        return importlib.util.spec_from_loader(fullname, self, is_package=False)

    def create_module(self, spec):
        module = importlib.import_module(_REAL + spec.name[len(__name__):])
        self._specs[spec.name] = module.__spec__
        return module

    def exec_module(self, module):
        # the import system stamped the alias spec on the shared module: give
        # the module its own spec back
        module.__spec__ = self._specs.pop(module.__spec__.name, module.__spec__)


if not any(isinstance(f, _AliasFinder) for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasFinder())


def __getattr__(name):
    if name in __all__:  # the quantizers load torch only when asked for
        return getattr(importlib.import_module(_REAL + ".algorithm"), name)
    try:
        return importlib.import_module(f"{__name__}.{name}")
    except ModuleNotFoundError:
        raise AttributeError(name) from None
