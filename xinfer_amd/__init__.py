"""xinfer_amd -- MI355X (gfx950) INT4-G128-SYM projection path of XInfer.

The product is ``lib/libxinfer_hip.so`` (hand-written HIP kernels behind the
C-ABI in ``include/xinfer_hip/xinfer_ops.h``).  This package adds:

* ``xinfer_amd.ops``   -- Python mirror of the reference's ``xinfer::ops``
  entry points (src/ops/linear.h, src/ops/sampling.h) over torch tensors;
* ``xinfer_amd.synth`` -- seeded synthetic inputs (SplitMix64, Box-Muller);
* ``xinfer_amd.build`` -- the in-tree hipcc build.
"""
from ._lib import XinferError, load_library  # noqa: F401

__version__ = "0.1.0"
