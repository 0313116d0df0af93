"""ctypes binding of libmko.so, the C ABI declared in ``include/mko.h``.

The library is loaded on first use from ``_lib/libmko.so`` next to this file (or
from ``$MKO_LIBRARY``).  There is no fallback: if the library is missing or was
built against another ABI version, every GPU entry point raises ``RuntimeError``.
Tensors cross the boundary as raw device pointers; the current torch HIP stream
is passed as the launch stream.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

ABI_VERSION = 1

F32, F16, BF16, F64 = 0, 1, 2, 3  # MKO_F64: the SSD entry points only
_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float64: F64}

_LIB_PATH = os.environ.get(
    "MKO_LIBRARY", os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libmko.so"))

_lock = threading.Lock()
_lib = None

_vp = ctypes.c_void_p


class SelscanParams(ctypes.Structure):
    """Mirror of ``mko_selscan_params``."""

    _fields_ = [
        ("u", _vp), ("delta", _vp), ("A", _vp), ("B", _vp), ("C", _vp), ("D", _vp), ("z", _vp),
        ("delta_bias", _vp), ("out", _vp), ("states", _vp), ("dout", _vp), ("du", _vp),
        ("ddelta", _vp), ("dA", _vp), ("dB", _vp), ("dC", _vp), ("dD", _vp), ("dz", _vp),
        ("ddelta_bias", _vp), ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("batch", ctypes.c_int64), ("dim", ctypes.c_int64), ("length", ctypes.c_int64),
        ("dstate", ctypes.c_int64), ("ngroups", ctypes.c_int64),
        ("u_dtype", ctypes.c_int32), ("delta_dtype", ctypes.c_int32), ("bc_dtype", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]


class StateUpdateParams(ctypes.Structure):
    """Mirror of ``mko_state_update_params``."""

    _fields_ = [
        ("state", _vp), ("x", _vp), ("dt", _vp), ("A", _vp), ("B", _vp), ("C", _vp), ("D", _vp),
        ("z", _vp), ("dt_bias", _vp), ("new_state", _vp), ("y", _vp), ("dy", _vp),
        ("dnew_state", _vp), ("grad_state", _vp), ("dx", _vp), ("ddt", _vp), ("dA", _vp),
        ("dB", _vp), ("dC", _vp), ("dD", _vp), ("dz", _vp), ("ddt_bias", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("batch", ctypes.c_int64), ("nheads", ctypes.c_int64), ("headdim", ctypes.c_int64),
        ("dstate", ctypes.c_int64), ("ngroups", ctypes.c_int64),
        ("state_dtype", ctypes.c_int32), ("x_dtype", ctypes.c_int32), ("dt_dtype", ctypes.c_int32),
        ("bc_dtype", ctypes.c_int32), ("flags", ctypes.c_uint32),
    ]


class SsdParams(ctypes.Structure):
    """Mirror of ``mko_ssd_params``."""

    _fields_ = [
        ("x", _vp), ("dt", _vp), ("A", _vp), ("B", _vp), ("C", _vp), ("D", _vp), ("z", _vp),
        ("dt_bias", _vp), ("initial_states", _vp), ("y", _vp), ("final_state", _vp), ("saved", _vp),
        ("dy", _vp), ("dfinal", _vp), ("dx", _vp), ("ddt", _vp), ("dA", _vp), ("dB", _vp),
        ("dC", _vp), ("dD", _vp), ("dz", _vp), ("ddt_bias", _vp), ("dinitial", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("batch", ctypes.c_int64), ("length", ctypes.c_int64), ("nheads", ctypes.c_int64),
        ("headdim", ctypes.c_int64), ("ngroups", ctypes.c_int64), ("dstate", ctypes.c_int64),
        ("x_dtype", ctypes.c_int32), ("dt_dtype", ctypes.c_int32), ("bc_dtype", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]


class PathParams(ctypes.Structure):
    """Mirror of ``mko_path_params``."""

    _fields_ = [
        ("src", _vp), ("dst", _vp),
        ("batch", ctypes.c_int64), ("rows", ctypes.c_int64), ("height", ctypes.c_int64),
        ("width", ctypes.c_int64), ("dtype", ctypes.c_int32), ("scale", ctypes.c_float),
    ]


class Conv1dParams(ctypes.Structure):
    """Mirror of ``mko_conv1d_params``."""

    _fields_ = [
        ("x", _vp), ("weight", _vp), ("bias", _vp), ("initial_state", _vp), ("out", _vp),
        ("final_state", _vp), ("dout", _vp), ("dx", _vp), ("dweight", _vp), ("dbias", _vp),
        ("dinitial", _vp), ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("batch", ctypes.c_int64), ("channels", ctypes.c_int64), ("length", ctypes.c_int64),
        ("width", ctypes.c_int64), ("dtype", ctypes.c_int32), ("flags", ctypes.c_uint32),
    ]


class Conv1dUpdateParams(ctypes.Structure):
    """Mirror of ``mko_conv1d_update_params``."""

    _fields_ = [
        ("x", _vp), ("state", _vp), ("weight", _vp), ("bias", _vp), ("out", _vp),
        ("batch", ctypes.c_int64), ("channels", ctypes.c_int64), ("q", ctypes.c_int64),
        ("span", ctypes.c_int64), ("width", ctypes.c_int64), ("state_stride_b", ctypes.c_int64),
        ("state_stride_c", ctypes.c_int64), ("dtype", ctypes.c_int32), ("flags", ctypes.c_uint32),
    ]


class GatedNormParams(ctypes.Structure):
    """Mirror of ``mko_gated_norm_params``."""

    _fields_ = [
        ("x", _vp), ("z", _vp), ("weight", _vp), ("bias", _vp), ("out", _vp), ("rstd", _vp),
        ("dout", _vp), ("dx", _vp), ("dz", _vp), ("dweight", _vp), ("dbias", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("rows", ctypes.c_int64), ("features", ctypes.c_int64), ("group", ctypes.c_int64),
        ("eps", ctypes.c_float), ("dtype", ctypes.c_int32), ("gate", ctypes.c_int32),
        ("wdtype", ctypes.c_int32),
    ]


_SIGNATURES = {
    "mko_abi_version": ([], ctypes.c_int),
    "mko_last_error": ([], ctypes.c_char_p),
    "mko_sizeof_selscan_params": ([], ctypes.c_size_t),
    "mko_sizeof_state_update_params": ([], ctypes.c_size_t),
    "mko_sizeof_ssd_params": ([], ctypes.c_size_t),
    "mko_sizeof_path_params": ([], ctypes.c_size_t),
    "mko_path_stack": ([ctypes.POINTER(PathParams), _vp], ctypes.c_int),
    "mko_path_merge": ([ctypes.POINTER(PathParams), _vp], ctypes.c_int),
    "mko_sizeof_conv1d_params": ([], ctypes.c_size_t),
    "mko_sizeof_conv1d_update_params": ([], ctypes.c_size_t),
    "mko_conv1d_fwd": ([ctypes.POINTER(Conv1dParams), _vp], ctypes.c_int),
    "mko_conv1d_bwd_workspace_size": ([ctypes.POINTER(Conv1dParams)], ctypes.c_size_t),
    "mko_conv1d_bwd": ([ctypes.POINTER(Conv1dParams), _vp], ctypes.c_int),
    "mko_conv1d_update": ([ctypes.POINTER(Conv1dUpdateParams), _vp], ctypes.c_int),
    "mko_sizeof_gated_norm_params": ([], ctypes.c_size_t),
    "mko_gated_norm_fwd": ([ctypes.POINTER(GatedNormParams), _vp], ctypes.c_int),
    "mko_gated_norm_bwd_workspace_size": ([ctypes.POINTER(GatedNormParams)], ctypes.c_size_t),
    "mko_gated_norm_bwd": ([ctypes.POINTER(GatedNormParams), _vp], ctypes.c_int),
    "mko_ssd_saved_bytes": ([ctypes.POINTER(SsdParams)], ctypes.c_size_t),
    "mko_ssd_fwd_workspace_size": ([ctypes.POINTER(SsdParams)], ctypes.c_size_t),
    "mko_ssd_fwd": ([ctypes.POINTER(SsdParams), _vp], ctypes.c_int),
    "mko_ssd_bwd_workspace_size": ([ctypes.POINTER(SsdParams)], ctypes.c_size_t),
    "mko_ssd_bwd": ([ctypes.POINTER(SsdParams), _vp], ctypes.c_int),
    "mko_selscan_num_checkpoints": ([ctypes.c_int64], ctypes.c_int64),
    "mko_selscan_fwd_workspace_size": ([ctypes.POINTER(SelscanParams)], ctypes.c_size_t),
    "mko_selscan_fwd": ([ctypes.POINTER(SelscanParams), _vp], ctypes.c_int),
    "mko_selscan_bwd_workspace_size": ([ctypes.POINTER(SelscanParams)], ctypes.c_size_t),
    "mko_selscan_bwd": ([ctypes.POINTER(SelscanParams), _vp], ctypes.c_int),
    "mko_stream_copy": ([_vp, _vp, ctypes.c_size_t, ctypes.c_uint32, _vp], ctypes.c_int),
    "mko_selscan_plan": ([ctypes.POINTER(SelscanParams), ctypes.POINTER(ctypes.c_int),
                          ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "mko_state_update_fwd": ([ctypes.POINTER(StateUpdateParams), _vp], ctypes.c_int),
    "mko_profile_enable": ([ctypes.c_int], ctypes.c_int),
    "mko_profile_reset": ([], None),
    "mko_profile_count": ([], ctypes.c_int),
    "mko_profile_entry": ([ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t,
                           ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)], ctypes.c_int),
    "mko_state_update_bwd_workspace_size": ([ctypes.POINTER(StateUpdateParams)], ctypes.c_size_t),
    "mko_state_update_bwd": ([ctypes.POINTER(StateUpdateParams), _vp], ctypes.c_int),
    "mko_state_update_bwd_static": ([ctypes.POINTER(StateUpdateParams), _vp], ctypes.c_int),
}

STATIC_SCRATCH_BYTES = 32 << 20
"""MKO_SU_STATIC_SCRATCH_BYTES: the static partials array of mko_state_update_bwd_static."""


def library_path():
    return _LIB_PATH


def lib():
    """The loaded library; raises ``RuntimeError`` when it is missing or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"libmko.so not found at {_LIB_PATH}: build it with "
                "`python metal-kernelops_amd/build.py` (hipcc, gfx950)")
        handle = ctypes.CDLL(_LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        version = handle.mko_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libmko.so ABI version {version}, this binding expects {ABI_VERSION}")
        for struct, fn in ((SelscanParams, handle.mko_sizeof_selscan_params),
                           (StateUpdateParams, handle.mko_sizeof_state_update_params),
                           (SsdParams, handle.mko_sizeof_ssd_params),
                           (PathParams, handle.mko_sizeof_path_params),
                           (Conv1dParams, handle.mko_sizeof_conv1d_params),
                           (Conv1dUpdateParams, handle.mko_sizeof_conv1d_update_params),
                           (GatedNormParams, handle.mko_sizeof_gated_norm_params)):
            if ctypes.sizeof(struct) != fn():
                raise RuntimeError(f"{struct.__name__} layout does not match libmko.so")
        _lib = handle
        return _lib


def kernel_timing(enable):
    """Turn the library's per-kernel HIP-event timing on or off; returns the old setting."""
    return bool(lib().mko_profile_enable(1 if enable else 0))


def kernel_timing_reset():
    lib().mko_profile_reset()


def kernel_times():
    """``{kernel: (total_ms, launches)}`` since the last reset (synchronises on the events)."""
    out = {}
    handle = lib()
    name = ctypes.create_string_buffer(128)
    total = ctypes.c_double()
    count = ctypes.c_int64()
    for i in range(handle.mko_profile_count()):
        if handle.mko_profile_entry(i, name, 128, ctypes.byref(total), ctypes.byref(count)) == 0:
            out[name.value.decode()] = (total.value, count.value)
    return out


STREAM_NONTEMPORAL = 1
"""MKO_STREAM_NONTEMPORAL."""


def stream_copy(src, dst, nontemporal=True):
    """Copies ``src`` into ``dst`` (same byte count, 16-byte aligned) with the library's
    streaming copy kernel on the current stream."""
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("stream_copy: src and dst differ in size")
    check(lib().mko_stream_copy(src.data_ptr(), dst.data_ptr(), nbytes, STREAM_NONTEMPORAL if nontemporal else 0,
                                stream_of(src.device)), "mko_stream_copy")


def exported_symbols():
    return list(_SIGNATURES)


def check(status, what):
    if status != 0:
        msg = lib().mko_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def ptr(t):
    return None if t is None else t.data_ptr()


def code(dtype):
    return _DTYPE_CODE[dtype]


def stream_of(device):
    return torch.cuda.current_stream(device).cuda_stream


def workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
