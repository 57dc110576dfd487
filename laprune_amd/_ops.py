"""Compiled torch binding of the decode path's hot entry points.

``laprune_amd/_lib/liblaprune_torch.so`` (built in-tree by
``laprune_amd.build`` from ``csrc/torch_ops.cpp`` with hipcc against the
installed torch headers) registers torch custom ops in the ``laprune``
namespace, each a direct call into the C ABI of ``liblaprune_hip.so``: sizes
and strides come from the tensors and the stream is the tensors' current
torch stream, so a call costs one dispatcher hop instead of marshalling
every argument through ctypes.  Eager decode (the reference's call pattern,
one call per layer per token) goes through these ops; the rest of the C ABI
stays bound by ctypes (``_native``).  Loading raises when the library is
missing: there is no fallback.
"""
from __future__ import annotations

import threading
from pathlib import Path

import torch

from . import _native as N

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "liblaprune_torch.so"

_lock = threading.Lock()
_ops = None


def ops():
    """``torch.ops.laprune`` after loading the binding (raises if it is not built)."""
    global _ops
    with _lock:
        if _ops is None:
            if not LIB_PATH.exists():
                raise RuntimeError(f"laprune_amd torch binding not built: {LIB_PATH} is missing "
                                   "(run `python -c 'import __graft_entry__ as g; g.build()'`)")
            N.lib()  # the HIP library it links against, loaded once from the same path
            torch.ops.load_library(str(LIB_PATH))
            _ops = torch.ops.laprune
        return _ops
