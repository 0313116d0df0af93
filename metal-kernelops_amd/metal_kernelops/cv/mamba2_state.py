"""Mamba-2 selective state update (one decode step) on MI355X, HIP kernels.

The operator is ``selective_state_update`` of state-spaces/mamba as the reference
defines it (``cv/mamba2_state.py:1-79``)::

    delta = softplus(dt + dt_bias)            (dt_softplus=True)
    a     = exp(A_h * delta)
    s'    = a * s + delta * x * B[g]          (g = h // (nheads / ngroups))
    y     = sum_n s' * C[g] + D * x
    y     = y * silu(z)                       (z given)

Layouts: ``state (batch, nheads, dim, dstate)``, ``x/z (batch, nheads, dim)``,
``dt (batch, nheads)`` or ``(batch, nheads, dim)``, ``A/dt_bias (nheads,)``,
``B/C (batch, ngroups, dstate)``, ``D (nheads,)`` or ``(nheads, dim)``.

Kernels (``libmko.so``): the forward is one fused read-modify-write of the state
per step; with no input requiring grad the entry point launches it directly, the
path a decode loop takes.  The backward is two launches with one writer per
gradient element, so repeated runs are bit-identical.  Inputs are read in the
dtype the reference would hand its kernel: x/dt/B/C/z are rounded to
``state.dtype`` first when that narrows them (a widening cast is exact and is
folded into the kernel's loads); A, D and dt_bias are read as float32.  The
backward computes in float32 and casts each gradient to its input's dtype.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch
from torch import Tensor

from .. import _native as nat
from .._contract import Rules

CHECKED_TORCH = "2.10.0"
"""Torch release this module was written and measured against (ROCm build)."""

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)
_SOFTPLUS, _DT_PER_ROW, _D_PER_ROW = 1, 2, 4


def _check(state, x, dt, A, B, C, D, z, dt_bias, out_state):
    """The reference's argument rules (``cv/mamba2_state.py:565-598``) in its order, plus
    this build's limits (3-D B/C, dstate <= 1024, one device, floating inputs) at the
    points where they first apply."""
    rules = Rules("mamba2_state_update")
    rules.dims("state", state, 4, "(batch, nheads, headdim, dstate)")
    batch, nheads, dim, dstate = state.shape
    rules.require(dstate >= 1, "state has an empty dstate axis")
    rows = (batch, nheads, dim)
    rules.shape("x", x, rows)
    rules.shape("z", z, rows)
    rules.shape("dt", dt, (batch, nheads), rows)
    rules.shape("A", A, (nheads,))
    rules.dims("B", B, 3, "(batch, ngroups, dstate)")
    groups = B.shape[1]
    rules.require(tuple(B.shape) == (batch, groups, dstate) and tuple(C.shape) == tuple(B.shape),
                  f"B and C should both be (batch, ngroups, dstate) = {(batch, groups, dstate)}; "
                  f"they are {tuple(B.shape)} and {tuple(C.shape)}")
    rules.require(groups >= 1 and nheads % groups == 0,
                  f"{nheads} heads do not split evenly into {groups} groups")
    rules.shape("D", D, (nheads,), (nheads, dim))
    rules.shape("dt_bias", dt_bias, (nheads,))
    rules.require(dstate <= 1024, f"dstate is at most 1024 here (got {dstate})")
    for name, tensor in (("x", x), ("dt", dt), ("A", A), ("B", B), ("C", C), ("D", D), ("z", z),
                         ("dt_bias", dt_bias)):
        if tensor is None:
            continue
        rules.same_device(state.device, **{name: tensor})
        rules.require(tensor.is_floating_point(), f"{name} should be a floating tensor; it is {tensor.dtype}")
    if out_state is not None:
        rules.require(out_state.device == state.device,
                      f"out_state lives on {out_state.device}, state on {state.device}")
        rules.require(tuple(out_state.shape) == tuple(state.shape) and out_state.dtype == state.dtype,
                      "out_state should have the shape and dtype of state")
        rules.require(out_state.is_contiguous(), "out_state should be contiguous")
        rules.require(not out_state.requires_grad,
                      "out_state is overwritten in place, so it may not require grad")


def _as_kernel_dtype(t, state_dtype):
    """The tensor the kernel reads for an activation input (see the module notes)."""
    if t is None:
        return None
    if t.dtype not in _FLOATS:
        t = t.to(state_dtype)
    elif t.dtype != state_dtype and not (state_dtype == torch.float32):
        t = t.to(state_dtype)
    return t.contiguous()


def _f32(t):
    return None if t is None else (t if t.dtype == torch.float32 else t.float()).contiguous()


def _params(state, x, dt, A, B, C, D, z, dt_bias, softplus):
    batch, nheads, dim, dstate = state.shape
    p = nat.StateUpdateParams()
    p.state, p.x, p.dt, p.A, p.B, p.C = (nat.ptr(t) for t in (state, x, dt, A, B, C))
    p.D, p.z, p.dt_bias = nat.ptr(D), nat.ptr(z), nat.ptr(dt_bias)
    p.batch, p.nheads, p.headdim, p.dstate, p.ngroups = batch, nheads, dim, dstate, B.shape[1]
    p.state_dtype, p.x_dtype = nat.code(state.dtype), nat.code(x.dtype)
    p.dt_dtype, p.bc_dtype = nat.code(dt.dtype), nat.code(B.dtype)
    p.flags = ((_SOFTPLUS if softplus else 0) | (_DT_PER_ROW if dt.dim() == 3 else 0)
               | (_D_PER_ROW if D is not None and D.dim() == 2 else 0))
    return p


def _launch(state, x, dt, A, B, C, D, z, dt_bias, softplus, new_state, y):
    if y.numel() == 0:
        return
    p = _params(state, x, dt, A, B, C, D, z, dt_bias, softplus)
    p.new_state, p.y = new_state.data_ptr(), y.data_ptr()
    lib = nat.lib()
    nat.check(lib.mko_state_update_fwd(ctypes.byref(p), nat.stream_of(state.device)),
              "mko_state_update_fwd")


@torch.library.custom_op("mko::state_update_fwd", mutates_args=(), device_types="cuda")
def _su_fwd(state: Tensor, x: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor,
            D: Optional[Tensor], z: Optional[Tensor], dt_bias: Optional[Tensor], softplus: bool
            ) -> Tuple[Tensor, Tensor]:
    new_state = torch.empty_like(state)
    y = torch.empty(state.shape[:3], dtype=state.dtype, device=state.device)
    _launch(state, x, dt, A, B, C, D, z, dt_bias, softplus, new_state, y)
    return y, new_state


@_su_fwd.register_fake
def _(state, x, dt, A, B, C, D, z, dt_bias, softplus):
    return state.new_empty(state.shape[:3]), torch.empty_like(state)


@torch.library.custom_op("mko::state_update_bwd", mutates_args=(), device_types="cuda")
def _su_bwd(state: Tensor, x: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor,
            D: Optional[Tensor], z: Optional[Tensor], dt_bias: Optional[Tensor], softplus: bool,
            dy: Optional[Tensor], dnew: Optional[Tensor]
            ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    f32 = dict(dtype=torch.float32, device=state.device)
    gstate = torch.empty(state.shape, **f32)
    dx = torch.empty(x.shape, **f32)
    ddt = torch.zeros(dt.shape, **f32)
    dA = torch.zeros(A.shape, **f32)
    dB = torch.zeros(B.shape, **f32)
    dC = torch.zeros(C.shape, **f32)
    dD = torch.zeros(D.shape if D is not None else (0,), **f32)
    dz = torch.zeros(z.shape if z is not None else (0,), **f32)
    dbias = torch.zeros(dt_bias.shape if dt_bias is not None else (0,), **f32)
    if dx.numel() == 0:
        gstate.zero_()
        return gstate, dx, ddt, dA, dB, dC, dD, dz, dbias
    lib = nat.lib()
    p = _params(state, x, dt, A, B, C, D, z, dt_bias, softplus)
    p.dy, p.dnew_state = nat.ptr(dy), nat.ptr(dnew)
    p.grad_state, p.dx, p.ddt, p.dA, p.dB, p.dC = (t.data_ptr() for t in (gstate, dx, ddt, dA, dB, dC))
    p.dD = dD.data_ptr() if D is not None else None
    p.dz = dz.data_ptr() if z is not None else None
    p.ddt_bias = dbias.data_ptr() if dt_bias is not None else None
    ws = nat.workspace(lib.mko_state_update_bwd_workspace_size(ctypes.byref(p)), state.device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    nat.check(lib.mko_state_update_bwd(ctypes.byref(p), nat.stream_of(state.device)),
              "mko_state_update_bwd")
    return gstate, dx, ddt, dA, dB, dC, dD, dz, dbias


@_su_bwd.register_fake
def _(state, x, dt, A, B, C, D, z, dt_bias, softplus, dy, dnew):
    def f(shape):
        return state.new_empty(shape, dtype=torch.float32)
    return (f(state.shape), f(x.shape), f(dt.shape), f(A.shape), f(B.shape), f(C.shape),
            f(D.shape if D is not None else (0,)), f(z.shape if z is not None else (0,)),
            f(dt_bias.shape if dt_bias is not None else (0,)))


def _narrow(t, like):
    return None if like is None else (t if t.dtype == like.dtype else t.to(like.dtype))


class _StateUpdate(torch.autograd.Function):
    """Autograd wiring of the two custom ops (once-differentiable, as the reference)."""

    @staticmethod
    def forward(ctx, state, x, dt, A, B, C, D, z, dt_bias, softplus):
        y, new_state = torch.ops.mko.state_update_fwd(state, x, dt, A, B, C, D, z, dt_bias, softplus)
        ctx.softplus = softplus
        # An unused output reaches backward as None, not as a zero tensor the size
        # of the state.
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(state, x, dt, A, B, C, D, z, dt_bias)
        return y, new_state

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dy, dnew):
        state, x, dt, A, B, C, D, z, dt_bias = ctx.saved_tensors
        dy = None if dy is None else dy.float().contiguous()
        dnew = None if dnew is None else dnew.float().contiguous()
        g = torch.ops.mko.state_update_bwd(state, x, dt, A, B, C, D, z, dt_bias, ctx.softplus, dy, dnew)
        gstate, dx, ddt, dA, dB, dC, dD, dz, dbias = g
        return (_narrow(gstate, state), _narrow(dx, x), _narrow(ddt, dt), _narrow(dA, A),
                _narrow(dB, B), _narrow(dC, C), _narrow(dD, D), _narrow(dz, z),
                _narrow(dbias, dt_bias), None)


def mamba2_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                        dt_softplus=False, out_state=None):
    """Advance a Mamba-2 decode state by one token on the ROCm GPU; returns ``(y, new_state)``.

    Per head ``h`` (group ``g = h // (nheads // ngroups)``) and row ``p``:
    ``delta = softplus(dt + dt_bias)`` (the bias and softplus optional),
    ``new_state = exp(A[h] * delta) * state + delta * x * B[g]`` and
    ``y = <new_state, C[g]> + D * x``, times ``silu(z)`` when ``z`` is given.

    Shapes (b = batch, H = nheads, P = headdim, N = dstate, G = ngroups):
    ``state`` (b, H, P, N) in float32, float16 or bfloat16, which fixes the compute and
    output dtype; ``x`` and ``z`` (b, H, P); ``dt`` (b, H), shared by a head's rows, or
    (b, H, P); ``A`` and ``dt_bias`` (H,); ``B`` and ``C`` (b, G, N); ``D`` (H,) or (H, P).

    ``state`` is read, never written, unless it is passed again as ``out_state``.  With
    ``out_state`` (contiguous, the state's shape and dtype, not requiring grad) the new
    state is written there and returned as that tensor, outside the autograd graph; the
    state may be its own destination, the in-place form a decode loop uses.  Without it,
    ``new_state`` is a fresh tensor.  ``y`` is (b, H, P) in the state's dtype.
    """
    if state.device.type != "cuda" or torch.version.hip is None:
        raise ValueError("mamba2_state_update runs on a ROCm GPU (torch device 'cuda')")
    if state.dtype not in _FLOATS:
        raise ValueError(f"state must be float32, float16 or bfloat16, got {state.dtype}")
    _check(state, x, dt, A, B, C, D, z, dt_bias, out_state)

    dtype = state.dtype
    kx, kdt, kB, kC, kz = (_as_kernel_dtype(t, dtype) for t in (x, dt, B, C, z))
    if kB.dtype != kC.dtype:
        kB, kC = kB.to(dtype).contiguous(), kC.to(dtype).contiguous()
    if kz is not None and kz.dtype != kx.dtype:
        # the kernel reads z in x's element type: meet in the state dtype, which with a
        # float32 state widens both exactly (what the reference's cast to state.dtype does)
        kx, kz = kx.to(dtype).contiguous(), kz.to(dtype).contiguous()
    kA, kD, kbias = _f32(A), _f32(D), _f32(dt_bias)

    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (state, x, dt, A, B, C, D, z, dt_bias))
    if not needs_grad:
        kstate = state if state.is_contiguous() else state.contiguous()
        new_state = out_state if out_state is not None else torch.empty_like(kstate)
        y = torch.empty(state.shape[:3], dtype=dtype, device=state.device)
        _launch(kstate, kx, kdt, kA, kB, kC, kD, kz, kbias, bool(dt_softplus), new_state, y)
        return y, new_state

    if (out_state is not None and state.requires_grad
            and out_state.untyped_storage().data_ptr() == state.untyped_storage().data_ptr()):
        # The backward needs the entering state, which an aliasing destination overwrites.
        state = state.clone()
    y, new_state = _StateUpdate.apply(state.contiguous(), kx, kdt, kA, kB, kC, kD, kz, kbias,
                                      bool(dt_softplus))
    if out_state is None:
        return y, new_state
    # The in-place destination is not part of the graph (the reference returns
    # new_state.detach() in this case).
    with torch.no_grad():
        out_state.copy_(new_state)
    return y, out_state


def mamba2_state_update_reference(state, x, dt, A, B, C, D=None, z=None,
                                  dt_bias=None, dt_softplus=False):
    """Step the recurrence in torch ops on any device and dtype; ``state`` untouched.

    The public pure-torch twin of the kernel (``cv/mamba2_state.py:822-849``).
    Returns ``(y, new_state)``.
    """
    if dt.dim() == 2:
        dt = dt.unsqueeze(-1)
    if D is not None and D.dim() == 1:
        D = D.unsqueeze(-1)
    if dt_bias is not None:
        dt = dt + dt_bias[None, :, None]
    if dt_softplus:
        dt = torch.nn.functional.softplus(dt)
    rep = state.shape[1] // B.shape[1]
    Bh = B.repeat_interleave(rep, dim=1)
    Ch = C.repeat_interleave(rep, dim=1)
    new_state = torch.exp(A[None, :, None, None] * dt[..., None]) * state \
        + (dt * x)[..., None] * Bh[:, :, None, :]
    y = (new_state * Ch[:, :, None, :]).sum(-1)
    if D is not None:
        y = y + x * D
    if z is not None:
        y = y * torch.nn.functional.silu(z)
    return y, new_state
