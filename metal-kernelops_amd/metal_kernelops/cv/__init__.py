"""Mamba-2 operators of ``metal_kernelops.cv`` on MI355X (HIP kernels).

Same names as the reference's ``cv/__init__.py:15-40`` for the SSM scan path:
the chunked SSD scan and the single-token decode update, each with its pure-torch
reference twin.  The reference's other ``cv`` operators (causal conv, gated
RMSNorm, path scan, NSA selection, RoIAlign) are not part of this package.
Importing it registers the ``mko::`` custom ops and launches nothing.
"""

from .mamba2_chunk import last_path, mamba2_chunk_scan, mamba2_chunk_scan_reference
from .mamba2_state import CHECKED_TORCH, mamba2_state_update, mamba2_state_update_reference

__all__ = [
    "CHECKED_TORCH",
    "last_path",
    "mamba2_chunk_scan",
    "mamba2_chunk_scan_reference",
    "mamba2_state_update",
    "mamba2_state_update_reference",
]
