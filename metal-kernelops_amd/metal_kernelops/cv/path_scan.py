"""Four-path 2D selective scan (VMamba's ``ss2d``) on MI355X.

Public surface, as in dbydd/metal-kernelops ``cv/path_scan.py:94-639``:
``ss2d_scan(u, dt, A, B, C, merge="sum")``, ``ss2d_scan_reference``,
``path_orders``, ``MERGE_MODES``, ``MAX_STATES``.

A ``(batch, channels, height, width)`` map is traversed along four paths (row-major,
column-major, and their reverses; ``path_orders``), each path is the Mamba-1 scan
``x_t = exp(dt_t A) x_{t-1} + dt_t B_t u_t``, ``y_t = <C_t, x_t>`` with zero initial
state and no skip, gate or bias, and the four results are added at every pixel
(``merge="mean"`` divides by four).

How it runs: the four paths of every channel are one Mamba-1 problem with four times
the channels and groups.  ``mko::path_stack`` (a HIP gather) writes u, dt, B and C in
path-step order, ``mko::selscan_fwd`` scans the stacked rows with the same kernels as
``selective_scan``, and ``mko::path_merge`` (a HIP gather) adds the four step-ordered
slices back per pixel in the reference's ``(0 + 2) + (1 + 3)`` order.  The backward
re-stacks the inputs and the output gradient, runs ``mko::selscan_bwd`` on the stacked
problem, and folds du, ddt, dB and dC back with ``path_merge``; dA sums the four
paths.  The reference stacks for its backward in the same way (``:477-543``) and
walks the paths with a cursor in its forward; here both directions share the 1-D
scan's kernels and their deterministic dB/dC reductions.

Differences from the reference, all widenings: tensors live on the ROCm GPU (the
reference runs on MPS only); u, B and C may also be float16 or bfloat16 (computed in
float32, dt taken as float32), and gradients come back in each input's dtype.
``states`` is limited to 32 as in the reference (``:97``), here by the scan kernels'
register budget.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from .. import _native as nat
from .._contract import Rules
from ..scan import _require_gpu, selscan_bwd_impl, selscan_fwd_impl

__all__ = ["MAX_STATES", "MERGE_MODES", "path_orders", "ss2d_scan", "ss2d_scan_reference"]

MERGE_MODES = ("sum", "mean")
"""How the four path outputs combine: elementwise sum, or their mean."""

MAX_STATES = 32
"""Largest state axis the scan kernels carry (``dstate <= 32``)."""

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def _check_merge(merge):
    if merge not in MERGE_MODES:
        Rules("ss2d_scan").fail(f"merge={merge!r} is not one of {MERGE_MODES}")


def _shape_contract(u, dt, A, B, C, where):
    """The shape rules every 2D-scan entry shares (``cv/path_scan.py:116-150``, same
    order); returns (batch, channels, groups, states, height, width)."""
    rules = Rules(where)
    rules.dims("u", u, 4, "(batch, channels, height, width)")
    batch, channels, height, width = u.shape
    rules.shape("dt", dt, tuple(u.shape))
    rules.dims("A", A, 2, "(channels, states)")
    rules.require(A.shape[0] == channels, f"A has {A.shape[0]} rows; u has {channels} channels")
    rules.dims("B", B, 5, "(batch, groups, states, height, width)")
    rules.shape("C", C, tuple(B.shape))
    groups, states = B.shape[1], A.shape[1]
    rules.require(B.shape[0] == batch, f"B holds {B.shape[0]} images; u holds {batch}")
    rules.require(B.shape[2] == states, f"B carries {B.shape[2]} states per group; A carries {states}")
    rules.require(tuple(B.shape[3:]) == (height, width),
                  f"B covers a {tuple(B.shape[3:])} map; u covers {(height, width)}")
    rules.require(not channels or groups >= 1, f"{channels} channels but no group to read B and C from")
    rules.require(not groups or channels % groups == 0,
                  f"{channels} channels do not divide evenly into {groups} groups")
    return batch, channels, groups, states, height, width


def path_orders(height, width, device=None):
    """For each of the four paths, the pixel (flat index ``h * width + w``) it visits at
    every step: row-major, down each column, and those two reversed."""
    step = torch.arange(height * width, device=device)
    down_columns = (step % height) * width + step // height
    return [step, down_columns, step.flip(0), down_columns.flip(0)]


def _zero_result(shape, tensors):
    """Zeros of ``shape`` that depend on every tensor in ``tensors`` (each times zero), so
    a backward through an empty problem still reaches them (``cv/path_scan.py:191-197``)."""
    tie = sum(t.sum() for t in tensors) * 0
    return tensors[0].new_zeros(shape) + tie


# --------------------------------------------------------------------------- layout ops


def _path_call(fn, x, out, height, width, scale):
    p = nat.PathParams()
    p.src, p.dst = x.data_ptr(), out.data_ptr()
    p.batch, p.height, p.width = x.shape[0], height, width
    p.rows = out.shape[1] if fn == "mko_path_merge" else x.shape[1]
    p.dtype, p.scale = nat.code(x.dtype), float(scale)
    lib = nat.lib()
    nat.check(getattr(lib, fn)(ctypes.byref(p), nat.stream_of(x.device)), fn)


def _stack_impl(x: Tensor, height: int, width: int, scale: float) -> Tensor:
    """(batch, rows, H*W) -> (batch, 4 rows, H*W): the four paths in step order."""
    out = x.new_empty(x.shape[0], 4 * x.shape[1], x.shape[2])
    if out.numel():
        _path_call("mko_path_stack", x, out, height, width, scale)
    return out


def _merge_impl(x: Tensor, height: int, width: int, scale: float) -> Tensor:
    """(batch, 4 rows, H*W) in step order -> (batch, rows, H*W) per pixel."""
    out = x.new_empty(x.shape[0], x.shape[1] // 4, x.shape[2])
    if out.numel():
        _path_call("mko_path_merge", x, out, height, width, scale)
    return out


# The layout launches as torch ops; the 2D scan's own autograd function calls the
# implementations directly (a dispatcher round trip per launch costs more host time than
# the launch itself on these small maps).
_path_stack = torch.library.custom_op("mko::path_stack", _stack_impl, mutates_args=(), device_types="cuda")
_path_merge = torch.library.custom_op("mko::path_merge", _merge_impl, mutates_args=(), device_types="cuda")


@_path_stack.register_fake
def _(x, height, width, scale):
    return x.new_empty(x.shape[0], 4 * x.shape[1], x.shape[2])


@_path_merge.register_fake
def _(x, height, width, scale):
    return x.new_empty(x.shape[0], x.shape[1] // 4, x.shape[2])


def _stacked(u, dt, A, B, C):
    """The four-path problem as one Mamba-1 problem: (b, 4C, L), (4C, N), (b, 4G, N, L)."""
    batch, channels, height, width = u.shape
    groups, states = B.shape[1], A.shape[1]
    length = height * width
    stack = _stack_impl
    su = stack(u.reshape(batch, channels, length), height, width, 1.0)
    sdt = stack(dt.reshape(batch, channels, length), height, width, 1.0)
    sb = stack(B.reshape(batch, groups * states, length), height, width, 1.0)
    sc = stack(C.reshape(batch, groups * states, length), height, width, 1.0)
    shape = (batch, 4 * groups, states, length)
    return su, sdt, A.repeat(4, 1).contiguous(), sb.view(shape), sc.view(shape)


class _PathScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u, dt, A, B, C, scale):
        batch, channels, height, width = u.shape
        su, sdt, sa, sb, sc = _stacked(u, dt, A, B, C)
        ys, ck = selscan_fwd_impl(su, sdt, sa, sb, sc, None, None, None, False)
        out = _merge_impl(ys, height, width, scale)
        ctx.scale = scale
        ctx.dims = (batch, channels, height, width, B.shape[1], A.shape[1])
        ctx.u_dtype = u.dtype
        # the stacked inputs (four times the inputs' size) are kept for the backward
        # rather than stacked again: four launches fewer per step
        ctx.save_for_backward(su, sdt, sa, sb, sc, ck)
        return out.view(batch, channels, height, width)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dy):
        su, sdt, sa, sb, sc, ck = ctx.saved_tensors
        batch, channels, height, width, groups, states = ctx.dims
        length = height * width
        sdy = _stack_impl(dy.to(ctx.u_dtype).contiguous().reshape(batch, channels, length), height, width, ctx.scale)
        dus, ddts, das, dbs, dcs, _, _, _ = selscan_bwd_impl(sdy, su, sdt, sa, sb, sc, None, None, None, False, ck)
        merge = _merge_impl
        du = merge(dus, height, width, 1.0).view(batch, channels, height, width)
        ddt = merge(ddts, height, width, 1.0).view(batch, channels, height, width)
        rows = (batch, 4 * groups * states, length)
        dB = merge(dbs.reshape(rows), height, width, 1.0).view(batch, groups, states, height, width)
        dC = merge(dcs.reshape(rows), height, width, 1.0).view(batch, groups, states, height, width)
        dA = das.view(4, channels, states).sum(0)
        return du, ddt, dA, dB, dC, None


def ss2d_scan(u, dt, A, B, C, merge="sum"):
    """Four-path 2D selective scan on the ROCm GPU.

    Args:
        u, dt: (batch, channels, height, width)
        A: (channels, states), negative; states <= 32
        B, C: (batch, groups, states, height, width), groups dividing channels
        merge: ``"sum"`` adds the four path outputs, ``"mean"`` divides by four.

    Returns:
        (batch, channels, height, width), contiguous, in u's dtype.  Strided inputs are
        accepted (copied to their dense layout first), as in ``cv/path_scan.py:546-576``.
    """
    _check_merge(merge)
    batch, channels, groups, states, height, width = _shape_contract(u, dt, A, B, C, "ss2d_scan")
    for name, tensor in (("u", u), ("dt", dt), ("A", A), ("B", B), ("C", C)):
        _require_gpu(tensor)
        if tensor.dtype not in _FLOATS:
            raise ValueError(f"ss2d_scan takes float32, float16 or bfloat16, {name} is {tensor.dtype}")
        if tensor.device != u.device:
            raise ValueError(f"ss2d_scan: {name} is on {tensor.device}, u is on {u.device}")
    if states > MAX_STATES:
        raise ValueError(f"ss2d_scan carries at most {MAX_STATES} states, got {states}")
    if u.numel() == 0 or B.numel() == 0:
        return _zero_result((batch, channels, height, width), (u, dt, A, B, C))
    # the scan kernels take float32 step sizes and decays, and B and C of one dtype;
    # autograd casts each gradient back to its input's dtype
    dt = dt.float() if dt.dtype != torch.float32 else dt
    A = A.float() if A.dtype != torch.float32 else A
    if B.dtype != C.dtype:
        B, C = B.float(), C.float()
    u, dt, A, B, C = (t.contiguous() for t in (u, dt, A, B, C))
    return _PathScan.apply(u, dt, A, B, C, 0.25 if merge == "mean" else 1.0)


def ss2d_scan_reference(u, dt, A, B, C, merge="sum"):
    """Pure-torch twin of :func:`ss2d_scan` on any device and dtype (``:608-639``).

    Built from index lists rather than views: the four paths are gathered with
    ``path_orders`` into one stacked problem of four times the channels and groups,
    scanned step by step with :func:`metal_kernelops.reference.selective_scan`, and
    each path is scattered back with its inverse order, so it also checks the GPU
    path's permutations.
    """
    from ..reference import selective_scan as reference_scan

    _check_merge(merge)
    batch, channels, groups, states, height, width = _shape_contract(u, dt, A, B, C, "ss2d_scan_reference")
    if u.numel() == 0 or B.numel() == 0:
        return _zero_result((batch, channels, height, width), (u, dt, A, B, C))
    length = height * width
    orders = path_orders(height, width, u.device)

    def stacked(x, rows):
        flat = x.reshape(batch, rows, length)
        return torch.cat([flat.index_select(-1, order) for order in orders], dim=1)

    bc_shape = (batch, 4 * groups, states, length)
    steps = reference_scan(stacked(u, channels), stacked(dt, channels), A.repeat(4, 1),
                           stacked(B, groups * states).view(bc_shape),
                           stacked(C, groups * states).view(bc_shape))
    paths = steps.view(batch, 4, channels, length)
    # path k stands on pixel orders[k][i] at step i; argsort inverts that map
    back = [paths[:, k].index_select(-1, torch.argsort(order)) for k, order in enumerate(orders)]
    total = (back[0] + back[2]) + (back[1] + back[3])
    if merge == "mean":
        total = total * 0.25
    return total.reshape(batch, channels, height, width)
