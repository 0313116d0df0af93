"""MI355X (gfx950) SSM scan kernels behind the dbydd/metal-kernelops API.

The import names match the reference's (``src/metal_kernelops/__init__.py:23-43``):
``from metal_kernelops import selective_scan`` for the Mamba-1 scan, and
``from metal_kernelops.cv import mamba2_chunk_scan, mamba2_state_update`` for Mamba-2.
Hand-written HIP kernels (``libmko.so``, C ABI in ``include/mko.h``) do the work on a
ROCm GPU; importing the package neither loads the library nor launches anything.

The Mamba-1 scan carries, per channel d and state n, the state
``h[t] = exp(delta[t] A[d, n]) h[t-1] + delta[t] u[t] B[n, t]`` from ``h[-1] = 0`` and
reads out ``y[t] = sum_n C[n, t] h[t]``.  ``u``, ``delta`` and ``z`` are laid out
(batch, dim, length); ``A`` is (dim, dstate) with negative entries; ``B`` and ``C``
are (batch, groups, dstate, length), one row per group of dim / groups channels;
``D`` is (dim,).
"""

from . import reference
from .scan import (
    BLOCK,
    CHUNK,
    scan_mps,
    scan_reference,
    selective_scan,
    selective_scan_fn,
)

__all__ = [
    "BLOCK",
    "CHUNK",
    "reference",
    "scan_mps",
    "scan_reference",
    "selective_scan",
    "selective_scan_fn",
]

__version__ = "0.3.0+mi355x"
