"""aoakv -- MI355X (gfx950) implementation of AOA-KV's decode hot path.

Kernels live in libaoakv.so (hand-written HIP, C ABI in include/aoakv.h);
this package binds them with ctypes and mirrors the reference's
``quest.utils`` interface in ``aoakv.utils``.  Importing the package loads
the library and fails if it is missing: there is no fallback.
"""
# torch first: libaoakv.so then binds to the HIP runtime torch already
# loaded, so the process holds one runtime, not torch's and /opt/rocm's.
import torch  # noqa: F401

from . import _lib
from ._lib import AoakvError, version

_lib.load()

from . import ops  # noqa: E402
from . import utils  # noqa: E402

__all__ = ["ops", "utils", "AoakvError", "version"]
