"""``turboquant.qjl`` of the reference's module layout (turboquant/qjl.py):
the 1-bit quantized Johnson-Lindenstrauss transform, from
``turboquant_amd.algorithm``."""
from .algorithm import QJL

__all__ = ["QJL"]
