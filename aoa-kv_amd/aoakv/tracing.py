"""Op-level profiling ranges (roctx).

The reference wraps each step of its attention and of each decoder layer in
nvtx ranges: qkv_proj, RoPE, append_kv, prefill_attn, full_attn, estimate,
topk, approx_attn, o_proj (quest/models/QuestAttention.py:87-176) and
input_norm, LlamaAttention, norm, mlp, embed, layer=<idx>
(quest/models/llama.py:138-164, 394-397, 465-475).  ``aoakv.shim`` opens the
same ranges through this module, so a trace shows the same structure.

Ranges go to roctx: rocprofiler-sdk's library (librocprofiler-sdk-roctx.so,
recorded by ``rocprofv3 --marker-trace``), or where that is absent torch's
``torch.cuda.nvtx`` (roctx in ROCm builds of torch).  They are off unless
enabled (``AOAKV_ROCTX=1`` in the environment, or ``enable()``): each range
is two foreign calls, which at ~20 ranges per layer would add a measurable
share to a decode step.

    from aoakv import tracing
    tracing.enable()
    with tracing.range("estimate"):
        ...
"""
from __future__ import annotations

import contextlib
import ctypes
import os

_ROCTX_LIBS = ("librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so",
               "/opt/rocm/lib/librocprofiler-sdk-roctx.so.1")

_enabled = os.environ.get("AOAKV_ROCTX", "0") not in ("", "0")
_impl = None  # (push(name: str) -> None, pop() -> None), chosen on first use


def _load():
    global _impl
    if _impl is not None:
        return _impl
    for name in _ROCTX_LIBS:
        try:
            lib = ctypes.CDLL(name)
        except OSError:
            continue
        lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
        lib.roctxRangePushA.restype = ctypes.c_int
        lib.roctxRangePop.argtypes = []
        lib.roctxRangePop.restype = ctypes.c_int
        _impl = (lambda s, f=lib.roctxRangePushA: f(s.encode()), lib.roctxRangePop, name)
        return _impl
    import torch
    _impl = (torch.cuda.nvtx.range_push, torch.cuda.nvtx.range_pop, "torch.cuda.nvtx")
    return _impl


def enable(on: bool = True) -> None:
    """Turns the ranges on (or off) for the rest of the process."""
    global _enabled
    _enabled = bool(on)


def enabled() -> bool:
    return _enabled


def backend() -> str:
    """The library the ranges go to (loads it)."""
    return _load()[2]


def push(name: str) -> None:
    if _enabled:
        _load()[0](name)


def pop() -> None:
    if _enabled:
        _load()[1]()


@contextlib.contextmanager
def range(name: str):  # noqa: A001  (the reference's word for it)
    """A named range around the body (nothing when disabled)."""
    if not _enabled:
        yield
        return
    push(name)
    try:
        yield
    finally:
        pop()
