"""Decode-op selection (seam of reference turboquant/decoder_dispatch.py:83-139).

This build has one decode kernel, the gfx950 HIP split-KV kernel, behind two
ops: the balanced-split op (default) and the reference's paged split-KV op
(``TQ_FORCE_KERNEL=gfx950_static``); there is no per-architecture fan-out.  The
``TQ_FORCE_KERNEL`` / ``TQ_DEBUG_KERNEL`` environment variables keep their
reference meaning: forcing a name other than the gfx950 kernel raises
ValueError (unknown name) or RuntimeError (known reference name that this
build does not provide), as the reference does for unregistered ops.
"""
from __future__ import annotations

import os
from functools import lru_cache

import torch

KERNEL_NAME = "gfx950_hip_paged_balanced"
STATIC_KERNEL_NAME = "gfx950_hip_paged_splitkv"
_REFERENCE_NAMES = ("v4", "v5", "v6", "v7")


def _has_op(lib: str, name: str) -> bool:
    try:
        return hasattr(getattr(torch.ops, lib), name)
    except (AttributeError, RuntimeError):
        return False


def _op(name: str = KERNEL_NAME):
    from . import ops
    ops.register_ops()
    if name == STATIC_KERNEL_NAME:
        return torch.ops.turboquant_v5.decode_v5_from_cache_paged_splitkv_ws
    return torch.ops.turboquant_v5.decode_paged_balanced_ws


@lru_cache(maxsize=1)
def pick_decode_op():
    """Return (op_callable, kernel_name).  Cached per process; clear with
    ``pick_decode_op.cache_clear()`` after changing the environment.

    The default is the balanced-split op (plan made on the GPU from
    seq_lens); ``TQ_FORCE_KERNEL=gfx950_static`` selects the reference's
    paged split-KV op with host-planned splits, same kernels."""
    forced = os.environ.get("TQ_FORCE_KERNEL", "").strip().lower()
    if forced:
        op, name = _resolve_forced(forced)
    else:
        op, name = _op(), KERNEL_NAME
    if os.environ.get("TQ_DEBUG_KERNEL"):
        print(f"[TQ dispatch] forced={forced!r} -> {name}", flush=True)
    return op, name


def _resolve_forced(name: str):
    if name in ("gfx950", KERNEL_NAME):
        return _op(), KERNEL_NAME
    if name in ("gfx950_static", STATIC_KERNEL_NAME):
        return _op(STATIC_KERNEL_NAME), STATIC_KERNEL_NAME
    if name in _REFERENCE_NAMES:
        raise RuntimeError(
            f"TQ_FORCE_KERNEL={name!r} was requested but the op is not registered in this "
            f"build; the only decode kernel is {KERNEL_NAME!r} (TQ_FORCE_KERNEL=gfx950).")
    raise ValueError(
        f"TQ_FORCE_KERNEL={name!r} not recognised. Choose from "
        f"{sorted(('gfx950', 'gfx950_static') + _REFERENCE_NAMES)}.")
