"""Mamba-2 operators of ``metal_kernelops.cv`` on MI355X (HIP kernels).

The names follow the reference's ``cv/__init__.py:15-40`` for the SSM scan path and
its neighbours in a Mamba block: the chunked SSD scan and the single-token decode
update (each with its pure-torch twin), the four-path 2D scan (VMamba's ss2d) built
on the Mamba-1 scan kernels, the causal depthwise conv1d ahead of the scan and the
gated RMSNorm after it.  The reference's other ``cv`` operators (NSA selection,
RoIAlign and the rest) are not part of this package.  Importing it registers the
``mko::`` custom ops and launches nothing.
"""

from .causal_conv1d import causal_conv1d_fn, causal_conv1d_ref, causal_conv1d_update
from .gated_norm import rmsnorm_gated, rmsnorm_gated_reference
from .mamba2_chunk import last_path, mamba2_chunk_scan, mamba2_chunk_scan_reference
from .mamba2_state import CHECKED_TORCH, mamba2_state_update, mamba2_state_update_reference
from .path_scan import MAX_STATES, MERGE_MODES, path_orders, ss2d_scan, ss2d_scan_reference

__all__ = [
    "CHECKED_TORCH",
    "MAX_STATES",
    "MERGE_MODES",
    "causal_conv1d_fn",
    "causal_conv1d_ref",
    "causal_conv1d_update",
    "last_path",
    "mamba2_chunk_scan",
    "mamba2_chunk_scan_reference",
    "mamba2_state_update",
    "mamba2_state_update_reference",
    "path_orders",
    "rmsnorm_gated",
    "rmsnorm_gated_reference",
    "ss2d_scan",
    "ss2d_scan_reference",
]
