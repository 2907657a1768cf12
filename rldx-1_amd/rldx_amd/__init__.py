"""rldx_amd: MI355X (gfx950) kernels for RLDX-1's real-time inference hot path.

Compute runs only through librldx_amd.so (hand-written HIP, C ABI in
include/rldx_amd.h).  `import rldx_amd.ops` registers the reference's
`torch.library` operators (ds::, ss::, rldx_backbone::) on top of it.
"""

from . import functional, workloads  # noqa: F401
from ._lib import lib_path, load  # noqa: F401

__all__ = ["functional", "workloads", "load", "lib_path"]
