"""MI355X (gfx950) SSM scan kernels behind the dbydd/metal-kernelops API.

Same import names as the reference (``src/metal_kernelops/__init__.py:23-43``):
``from metal_kernelops import selective_scan`` and ``from metal_kernelops.cv
import mamba2_chunk_scan, mamba2_state_update``.  The compute runs in hand-written
HIP kernels (``libmko.so``, C ABI in ``include/mko.h``) on a ROCm GPU; importing
the package loads nothing and launches nothing.

The recurrence is the one from mamba_ssm's ``selective_scan_fn``:

    x_t = exp(dt_t * A) * x_{t-1} + dt_t * B_t * u_t
    y_t = <x_t, C_t>

Layouts:
    u, dt:  (batch, dim, length)
    A:      (dim, dstate)          negative reals
    B, C:   (batch, groups, dstate, length)
    D:      (dim,)
    z:      (batch, dim, length)
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
