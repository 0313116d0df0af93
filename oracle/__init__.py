"""CPU oracle for the SSM scan hot path -- test infrastructure, never product code.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or as the timed CPU
baseline.  The HIP product path in ``metal-kernelops_amd/`` never imports it.

Everything here is plain PyTorch on the CPU, evaluated in float64 unless a caller
asks otherwise, and restates the reference's algorithms from the mathematics.
Each function cites the reference ``file:line`` it follows.  How each function is
pinned (closed forms, independent formulations, finite differences) is listed in
``tests/test_oracle.py``; no function here is left "parity unpinned".
"""

from .ssm import (  # noqa: F401
    mamba2_chunk_scan_composition,
    mamba2_chunk_scan_recurrence,
    mamba2_state_update,
    normalize_initial_states,
    selective_scan,
    selective_scan_loop,
    softplus,
    ss2d_path_orders,
    ss2d_scan,
    ssd_minimal_discrete,
)
from .conv1d import causal_conv1d, causal_conv1d_update  # noqa: F401,E402
from .norm import rmsnorm_gated, rmsnorm_gated_bwd  # noqa: F401,E402
