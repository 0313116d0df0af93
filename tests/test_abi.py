"""The C ABI library loads on the CPU host and exports what include/mko.h declares.

No kernel is launched here: only host-side entry points (version, sizes, argument
validation) are called.
"""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mko.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mko_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def native():
    from metal_kernelops import _native
    return _native


def test_library_exports_every_declared_symbol(native):
    lib = native.lib()
    declared = _declared()
    assert len(declared) >= 10
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) <= set(native.exported_symbols()) | {"mko_last_error"}


def test_abi_version_and_struct_layouts(native):
    lib = native.lib()
    assert lib.mko_abi_version() == native.ABI_VERSION
    assert ctypes.sizeof(native.SelscanParams) == lib.mko_sizeof_selscan_params()
    assert ctypes.sizeof(native.StateUpdateParams) == lib.mko_sizeof_state_update_params()
    assert ctypes.sizeof(native.SsdParams) == lib.mko_sizeof_ssd_params()
    assert ctypes.sizeof(native.PathParams) == lib.mko_sizeof_path_params()


def test_path_layout_validation_without_gpu(native):
    lib = native.lib()
    p = native.PathParams()
    p.batch, p.rows, p.height, p.width, p.dtype, p.scale = 1, 4, -3, 5, 0, 1.0
    assert lib.mko_path_stack(ctypes.byref(p), None) == 1
    assert b"negative" in lib.mko_last_error()
    p.height, p.dtype = 3, 7
    assert lib.mko_path_merge(ctypes.byref(p), None) == 1
    assert b"dtype" in lib.mko_last_error()
    p.dtype = 0
    assert lib.mko_path_stack(ctypes.byref(p), None) == 1  # null src/dst with elements
    p.height = 0  # an empty map launches nothing and needs no pointers
    assert lib.mko_path_stack(ctypes.byref(p), None) == 0
    assert lib.mko_path_merge(ctypes.byref(p), None) == 0


def test_host_side_validation_without_gpu(native):
    lib = native.lib()
    p = native.SelscanParams()
    p.batch, p.dim, p.length, p.dstate, p.ngroups = 2, 8, 64, 16, 3  # 8 % 3 != 0
    assert lib.mko_selscan_fwd(ctypes.byref(p), None) == 1
    assert b"divisible" in lib.mko_last_error()
    p.ngroups, p.dstate = 2, 40
    assert lib.mko_selscan_fwd(ctypes.byref(p), None) == 3
    p.dstate = 16
    assert lib.mko_selscan_fwd_workspace_size(ctypes.byref(p)) > 0
    assert lib.mko_selscan_num_checkpoints(130) == 9  # ceil(130 / MKO_SS_CHECKPOINT), 16-step saves
    p.workspace, p.workspace_bytes = None, 0
    for name in ("u", "delta", "A", "B", "C", "out", "states"):
        setattr(p, name, 16)  # never dereferenced: the workspace check fails first
    assert lib.mko_selscan_fwd(ctypes.byref(p), None) == 4
    q = native.StateUpdateParams()
    q.batch, q.nheads, q.headdim, q.dstate, q.ngroups = 1, 4, 8, 16, 3
    assert lib.mko_state_update_fwd(ctypes.byref(q), None) == 1


def test_gated_norm_validation_without_gpu(native):
    lib = native.lib()
    assert ctypes.sizeof(native.GatedNormParams) == lib.mko_sizeof_gated_norm_params()
    p = native.GatedNormParams()
    p.rows, p.features, p.group, p.eps, p.dtype, p.gate = 4, 300, 7, 1e-5, 0, 0  # 300 % 7 != 0
    assert lib.mko_gated_norm_fwd(ctypes.byref(p), None) == 1
    assert b"divide" in lib.mko_last_error()
    p.group, p.gate = 100, 5
    assert lib.mko_gated_norm_fwd(ctypes.byref(p), None) == 1
    assert b"gate" in lib.mko_last_error()
    p.gate, p.dtype = 2, 9
    assert lib.mko_gated_norm_bwd(ctypes.byref(p), None) == 1
    assert b"dtype" in lib.mko_last_error()
    p.dtype, p.eps = 2, -1.0
    assert lib.mko_gated_norm_fwd(ctypes.byref(p), None) == 1
    p.eps = 1e-5
    assert lib.mko_gated_norm_fwd(ctypes.byref(p), None) == 1  # x, weight, out, z missing
    assert b"required" in lib.mko_last_error()
    p.rows = 0  # no rows: nothing to launch, no pointers needed
    assert lib.mko_gated_norm_fwd(ctypes.byref(p), None) == 0
    assert lib.mko_gated_norm_bwd(ctypes.byref(p), None) == 0
    assert lib.mko_gated_norm_bwd_workspace_size(ctypes.byref(p)) == 0
    # dweight wanted: a partial row per row block; a group past the register set adds c1
    p.rows, p.features, p.group, p.gate = 256, 2560, 2560, 2
    for name in ("x", "z", "weight", "dout", "dx", "dz", "rstd"):
        setattr(p, name, 256)  # 16-byte aligned, never dereferenced
    p.dweight = 256
    dense = lib.mko_gated_norm_bwd_workspace_size(ctypes.byref(p))
    assert dense > 0 and dense % (2 * 2560 * 4) == 0
    p.features = p.group = 32768
    wide = lib.mko_gated_norm_bwd_workspace_size(ctypes.byref(p))
    assert wide > 0 and (wide - 256 * 4) % (2 * 32768 * 4) == 0
    p.workspace, p.workspace_bytes = None, 0
    assert lib.mko_gated_norm_bwd(ctypes.byref(p), None) == 4


def test_static_decode_backward_refuses_an_oversized_problem_on_the_host(native):
    # Host-side validation only: the size check comes before any pointer is read or any
    # HIP call is made.
    lib = native.lib()
    p = native.StateUpdateParams()
    p.batch, p.nheads, p.headdim, p.dstate, p.ngroups = 1 << 16, 8, 16, 32, 2
    p.state_dtype = p.x_dtype = p.dt_dtype = p.bc_dtype = 0
    for name in ("state", "x", "dt", "A", "B", "C", "grad_state", "dx", "ddt", "dA", "dB", "dC"):
        setattr(p, name, 256)
    assert lib.mko_state_update_bwd_workspace_size(ctypes.byref(p)) > native.STATIC_SCRATCH_BYTES
    assert lib.mko_state_update_bwd_static(ctypes.byref(p), None) == 4  # MKO_EWORKSPACE
    assert b"static scratch" in lib.mko_last_error()
    p.dA = None
    assert lib.mko_state_update_bwd_static(ctypes.byref(p), None) == 1  # a missing output first


def test_lane_backward_refused_past_its_32_bit_offsets(native):
    """The lane-per-state backward addresses B/C with 32-bit lane offsets.  With groups of
    4 channels B/C hold four times as many elements as u, so a geometry whose rows x length
    still fits 2^31 while batch x groups x 16 x length does not must plan the
    lane-per-channel backward; the forward (64-bit offsets) keeps its lane mapping."""
    lib = native.lib()

    def plan(batch, dim, length, groups):
        p = native.SelscanParams()
        p.batch, p.dim, p.length, p.dstate, p.ngroups = batch, dim, length, 16, groups
        fwd, bwd = ctypes.c_int(-1), ctypes.c_int(-1)
        assert lib.mko_selscan_plan(ctypes.byref(p), ctypes.byref(fwd), ctypes.byref(bwd)) == 0
        return fwd.value, bwd.value

    # c3's geometry takes the lane kernels both ways
    assert plan(4, 5120, 4096, 1) == (1, 1)
    # 4-channel groups: B/C = 4 * rows * length elements; rows * length = 2^29
    assert plan(1, 8192, 65536, 2048) == (1, 0)
    # one step shorter per 16: B/C just under 2^31 elements, the lane backward again
    assert plan(1, 8192, 65536 - 16, 2048) == (1, 1)
    # 16-channel groups at the same sizes: B/C = rows * length, inside the bound
    assert plan(1, 8192, 65536, 512) == (1, 1)
    # rows * length itself at 2^31
    assert plan(1, 8192, 262144, 1) == (1, 0)
