"""Mamba-2 chunked SSD scan on MI355X: HIP kernels on the CDNA4 matrix cores.

The function is ``mamba_chunk_scan_combined`` as the reference defines it
(``cv/mamba2_chunk.py:1-68``)::

    dt_t  = softplus(dt_t + dt_bias)                      (dt_softplus)
    a_t   = exp(dt_t * A)                                 A negative, per head
    s_t   = a_t * s_{t-1} + dt_t * x_t (x) B_t            s (batch, head, d_head, d_state)
    y_t   = <C_t, s_t> + D * x_t                          D (heads,) or (heads, d_head)
    y_t   = y_t * silu(z_t)                               z gate
    final = s_{L-1}

Layouts: ``x/z (batch, length, nheads, d_head)``, ``dt (batch, length, nheads)``,
``A/dt_bias (nheads,)``, ``B/C (batch, length, ngroups, d_state)``, ``D (nheads,)``
or ``(nheads, d_head)``, ``initial_states (batch, nheads, d_head, d_state)`` (the
transposed and 5-D spellings of the reference are accepted).  Returns ``(y,
final_state)`` in ``x.dtype``.

Kernels (``libmko.so``): the block factorisation of the SSD paper with the
intra-chunk product, the chunk states and the state-to-output product on the
matrix cores (bf16/f16 operands for bf16/f16 inputs, fp32 operands for fp32
inputs; fp32 accumulation, decays and states), and an O(nchunks) sequential
state pass instead of the reference's O(nchunks^2) transfer matrix.  float64
inputs, which the reference's composition also takes, run the per-token
recurrence in float64 on the vector units (d_state <= 256).  The chunk
length is the kernels' own choice: ``chunk_size`` is accepted for signature
parity and, as in the reference, does not change the result.  The backward is a
hand-written set of kernels (the reference differentiates its torch
composition); it is once-differentiable.  Tensors must live on a ROCm GPU.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch
from torch import Tensor

from .. import _native as nat
from .._contract import Rules

__all__ = ["mamba2_chunk_scan", "mamba2_chunk_scan_reference", "last_path"]

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)
_X_FLOATS = _FLOATS + (torch.float64,)
_SOFTPLUS, _D_PER_ROW, _SAVE_Y = 1, 2, 4

_path = "none"
"""Which path the last :func:`mamba2_chunk_scan` call took."""


def last_path():
    """``"hip"`` once a scan has run (``"none"`` before): the path the last scan took."""
    return _path


def _initial_layout(rules, states, batch, nheads, headdim, dstate):
    """``initial_states`` in the (batch, nheads, headdim, dstate) layout the kernels read.

    Besides that layout the reference accepts a 5-D tensor with a unit second axis and,
    when headdim and dstate differ, the (batch, nheads, dstate, headdim) transpose."""
    want = (batch, nheads, headdim, dstate)
    if states.dim() == 5 and states.shape[1] == 1:
        states = states.squeeze(1)
    if tuple(states.shape) == want:
        return states
    if headdim != dstate and tuple(states.shape) == (batch, nheads, dstate, headdim):
        return states.transpose(-1, -2)
    rules.fail(f"initial_states should be (batch, nheads, headdim, dstate) = {want}; "
               f"its shape is {tuple(states.shape)}")


def _check(x, dt, A, B, C, D, z, dt_bias, initial_states, chunk_size):
    """The reference's argument rules (``cv/mamba2_chunk.py:398-444``), in its order.

    Returns the sizes and ``initial_states`` in the kernels' layout.  ``x`` may be float32,
    float16, bfloat16 or float64, as in the reference."""
    rules = Rules("mamba2_chunk_scan")
    rules.require(chunk_size >= 1, f"chunk_size must be at least 1 (got {chunk_size})")
    rules.dims("x", x, 4, "(batch, length, nheads, headdim)")
    batch, length, nheads, headdim = x.shape
    rules.shape("dt", dt, (batch, length, nheads))
    rules.shape("A", A, (nheads,))
    rules.require(B.dim() == 4 and tuple(C.shape) == tuple(B.shape),
                  f"B and C should share one (batch, length, ngroups, dstate) shape; "
                  f"they are {tuple(B.shape)} and {tuple(C.shape)}")
    rules.require(tuple(B.shape[:2]) == (batch, length),
                  f"B and C should lead with (batch, length) = {(batch, length)}; they are {tuple(B.shape)}")
    ngroups, dstate = B.shape[2], B.shape[3]
    rules.require(ngroups >= 1 and nheads % ngroups == 0,
                  f"{nheads} heads do not split evenly into {ngroups} groups")
    rules.shape("z", z, tuple(x.shape))
    rules.shape("D", D, (nheads,), (nheads, headdim))
    rules.shape("dt_bias", dt_bias, (nheads,))
    if initial_states is not None:
        initial_states = _initial_layout(rules, initial_states, batch, nheads, headdim, dstate)
    rules.dtype_in(_X_FLOATS, x=x)
    rules.same_device(x.device, dt=dt, A=A, B=B, C=C)
    rules.dtype_in(_X_FLOATS, dt=dt, B=B, C=C, z=z, D=D, dt_bias=dt_bias, initial_states=initial_states, A=A)
    return batch, length, nheads, headdim, ngroups, dstate, initial_states


def _params(x, dt, A, B, C, D, z, dt_bias, init, softplus, save_y=False):
    batch, length, nheads, headdim = x.shape
    p = nat.SsdParams()
    p.x, p.dt, p.A, p.B, p.C = (nat.ptr(t) for t in (x, dt, A, B, C))
    p.D, p.z, p.dt_bias, p.initial_states = nat.ptr(D), nat.ptr(z), nat.ptr(dt_bias), nat.ptr(init)
    p.batch, p.length, p.nheads, p.headdim = batch, length, nheads, headdim
    p.ngroups, p.dstate = B.shape[2], B.shape[3]
    p.x_dtype, p.dt_dtype, p.bc_dtype = nat.code(x.dtype), nat.code(dt.dtype), nat.code(B.dtype)
    p.flags = ((_SOFTPLUS if softplus else 0) | (_D_PER_ROW if D is not None and D.dim() == 2 else 0)
               | (_SAVE_Y if save_y else 0))
    return p


@torch.library.custom_op("mko::ssd_fwd", mutates_args=(), device_types="cuda")
def _ssd_fwd(x: Tensor, dt: Tensor, A: Tensor, B: Tensor, C: Tensor, D: Optional[Tensor],
             z: Optional[Tensor], dt_bias: Optional[Tensor], initial_states: Optional[Tensor],
             softplus: bool, save_y: bool) -> Tuple[Tensor, Tensor, Tensor]:
    batch, length, nheads, headdim = x.shape
    y = torch.empty_like(x)
    final = torch.empty(batch, nheads, headdim, B.shape[3], dtype=x.dtype, device=x.device)
    lib = nat.lib()
    p = _params(x, dt, A, B, C, D, z, dt_bias, initial_states, softplus, save_y)
    saved = nat.workspace(lib.mko_ssd_saved_bytes(ctypes.byref(p)), x.device)
    p.y, p.final_state, p.saved = y.data_ptr(), final.data_ptr(), saved.data_ptr()
    nat.check(lib.mko_ssd_fwd(ctypes.byref(p), nat.stream_of(x.device)), "mko_ssd_fwd")
    return y, final, saved


@_ssd_fwd.register_fake
def _(x, dt, A, B, C, D, z, dt_bias, initial_states, softplus, save_y):
    batch, length, nheads, headdim = x.shape
    return (torch.empty_like(x), x.new_empty(batch, nheads, headdim, B.shape[3]),
            x.new_empty(0, dtype=torch.uint8))


@torch.library.custom_op("mko::ssd_bwd", mutates_args=(), device_types="cuda")
def _ssd_bwd(dy: Tensor, dfinal: Optional[Tensor], x: Tensor, dt: Tensor, A: Tensor, B: Tensor,
             C: Tensor, D: Optional[Tensor], z: Optional[Tensor], dt_bias: Optional[Tensor],
             initial_states: Optional[Tensor], softplus: bool, save_y: bool, saved: Tensor
             ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    # the parameters' gradients in the arithmetic's precision: float64 for float64 inputs
    f32 = dict(dtype=torch.float64 if x.dtype == torch.float64 else torch.float32, device=x.device)
    dx, ddt = torch.empty_like(x), torch.empty_like(dt)
    dA = torch.empty(A.shape, **f32)
    dB, dC = torch.empty_like(B), torch.empty_like(C)
    dD = torch.empty(D.shape if D is not None else (0,), **f32)
    dz = torch.empty_like(z) if z is not None else x.new_empty(0)
    dbias = torch.empty(dt_bias.shape if dt_bias is not None else (0,), **f32)
    dinit = torch.empty_like(initial_states) if initial_states is not None else x.new_empty(0)
    lib = nat.lib()
    p = _params(x, dt, A, B, C, D, z, dt_bias, initial_states, softplus, save_y)
    p.saved, p.dy, p.dfinal = saved.data_ptr(), dy.data_ptr(), nat.ptr(dfinal)
    p.dx, p.ddt, p.dA, p.dB, p.dC = (t.data_ptr() for t in (dx, ddt, dA, dB, dC))
    p.dD = dD.data_ptr() if D is not None else None
    p.dz = dz.data_ptr() if z is not None else None
    p.ddt_bias = dbias.data_ptr() if dt_bias is not None else None
    p.dinitial = dinit.data_ptr() if initial_states is not None else None
    ws = nat.workspace(lib.mko_ssd_bwd_workspace_size(ctypes.byref(p)), x.device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    nat.check(lib.mko_ssd_bwd(ctypes.byref(p), nat.stream_of(x.device)), "mko_ssd_bwd")
    return dx, ddt, dA, dB, dC, dD, dz, dbias, dinit


@_ssd_bwd.register_fake
def _(dy, dfinal, x, dt, A, B, C, D, z, dt_bias, initial_states, softplus, save_y, saved):
    def f(shape):
        return x.new_empty(shape, dtype=torch.float64 if x.dtype == torch.float64 else torch.float32)
    return (torch.empty_like(x), torch.empty_like(dt), f(A.shape), torch.empty_like(B),
            torch.empty_like(C), f(D.shape if D is not None else (0,)),
            torch.empty_like(z) if z is not None else x.new_empty(0),
            f(dt_bias.shape if dt_bias is not None else (0,)),
            torch.empty_like(initial_states) if initial_states is not None else x.new_empty(0))


def _setup(ctx, inputs, output):
    x, dt, A, B, C, D, z, dt_bias, init, softplus, save_y = inputs
    ctx.save_for_backward(x, dt, A, B, C, D, z, dt_bias, init, output[2])
    ctx.softplus = softplus
    ctx.save_y = save_y
    ctx.set_materialize_grads(False)  # no zero-filled gradient for the save area


def _backward(ctx, dy, dfinal, _dsaved):
    x, dt, A, B, C, D, z, bias, init, saved = ctx.saved_tensors
    if dy is None:
        dy = torch.zeros_like(x)
    dx, ddt, dA, dB, dC, dD, dz, dbias, dinit = torch.ops.mko.ssd_bwd(
        dy.contiguous(), None if dfinal is None else dfinal.contiguous(), x, dt, A, B, C, D, z, bias,
        init, ctx.softplus, ctx.save_y, saved)
    return (dx, ddt, dA, dB, dC, dD if D is not None else None, dz if z is not None else None,
            dbias if bias is not None else None, dinit if init is not None else None, None, None)


torch.library.register_autograd("mko::ssd_fwd", _backward, setup_context=_setup)


def _as(t, dtype):
    return None if t is None else (t if t.dtype == dtype else t.to(dtype)).contiguous()


def mamba2_chunk_scan(x, dt, A, B, C, chunk_size=64, D=None, z=None, dt_bias=None,
                      dt_softplus=False, initial_states=None):
    """Mamba-2 SSD over a whole sequence on the ROCm GPU; returns ``(y, final_state)``.

    The recurrence runs per head over ``length`` tokens; the heads of one group read
    the same ``B`` and ``C``.  Shapes (b = batch, L = length, H = nheads, P = headdim,
    G = ngroups dividing H, N = dstate):

    ========================  ==============================  ==============================
    argument                  shape                           meaning
    ========================  ==============================  ==============================
    ``x``                     (b, L, H, P)                    input; its dtype (float32,
                                                              float16, bfloat16, float64) is
                                                              the operand and output dtype
    ``dt``                    (b, L, H)                       step sizes before the optional
                                                              bias and softplus
    ``A``                     (H,)                            per-head log decay (negative)
    ``B``, ``C``              (b, L, G, N)                    input and output projections
    ``chunk_size``            int >= 1                        kept for the reference's
                                                              signature; the kernels pick
                                                              their own chunk, and the result
                                                              does not depend on it
    ``D``                     (H,) or (H, P), optional        skip weight on ``x``
    ``z``                     (b, L, H, P), optional          gate: ``y * silu(z)``
    ``dt_bias``               (H,), optional                  added to ``dt``
    ``dt_softplus``           bool                            softplus on ``dt + dt_bias``
    ``initial_states``        (b, H, P, N), optional          state before the first token
    ========================  ==============================  ==============================

    ``y`` is (b, L, H, P) and ``final_state`` (b, H, P, N), both in ``x.dtype``.
    """
    global _path
    if x.device.type != "cuda" or torch.version.hip is None:
        raise ValueError("mamba2_chunk_scan runs on a ROCm GPU (torch device 'cuda'), "
                         f"got {x.device}")
    batch, length, nheads, headdim, ngroups, dstate, initial_states = _check(
        x, dt, A, B, C, D, z, dt_bias, initial_states, chunk_size)
    x = x.contiguous()
    # B and C take x's dtype: every contraction runs with x.dtype operands (as the
    # reference's composition does); autograd casts their gradients back.  The step sizes
    # and the per-head parameters are float32, or float64 for float64 x (the reference
    # computes in float64 then, cv/mamba2_chunk.py:447-462).
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    dt = dt.contiguous() if acc == torch.float32 else _as(dt, acc)
    B, C = B.to(x.dtype).contiguous(), C.to(x.dtype).contiguous()
    if z is not None:
        z = (z if z.dtype == x.dtype else z.to(x.dtype)).contiguous()
    if initial_states is not None:
        initial_states = initial_states.to(x.dtype).contiguous()
    A, D, dt_bias = _as(A, acc), _as(D, acc), _as(dt_bias, acc)
    _path = "hip"
    # The forward keeps its chunk output for the backward only when a gradient will be taken.
    save_y = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (x, dt, A, B, C, D, z, dt_bias, initial_states))
    y, final, _ = torch.ops.mko.ssd_fwd(x, dt, A, B, C, D, z, dt_bias, initial_states,
                                        bool(dt_softplus), bool(save_y))
    return y, final


def mamba2_chunk_scan_reference(x, dt, A, B, C, chunk_size=64, D=None, z=None,
                                dt_bias=None, dt_softplus=False, initial_states=None,
                                dtype=torch.float64):
    """Step-by-step recurrence: the definition the chunked scan must reproduce.

    The public twin of ``cv/mamba2_chunk.py:681-723``: it walks ``length`` one
    token at a time in ``dtype`` (float64 by default) on the tensors' own device,
    ``chunk_size`` is ignored, and the results are cast back to ``x.dtype``.
    """
    out_dtype = x.dtype
    x, dt, A, B, C = (t.to(dtype) for t in (x, dt, A, B, C))
    batch, length, nheads, headdim = x.shape
    ngroups, dstate = B.shape[2], B.shape[3]
    rep = nheads // ngroups
    Bh = B.repeat_interleave(rep, dim=2)
    Ch = C.repeat_interleave(rep, dim=2)
    if dt_bias is not None:
        dt = dt + dt_bias.to(dtype).view(1, 1, nheads)
    if dt_softplus:
        dt = torch.nn.functional.softplus(dt)
    state = torch.zeros(batch, nheads, headdim, dstate, dtype=dtype, device=x.device)
    if initial_states is not None:
        init = initial_states.to(dtype)
        if init.dim() == 5:
            init = init[:, 0]
        if init.shape != state.shape and init.shape == state.transpose(-1, -2).shape:
            init = init.transpose(-1, -2)
        state = init.clone()
    steps = []
    for t in range(length):
        delta = dt[:, t]
        state = state * torch.exp(delta * A)[..., None, None] \
            + (delta[..., None] * x[:, t])[..., :, None] * Bh[:, t][:, :, None, :]
        steps.append((state * Ch[:, t][:, :, None, :]).sum(-1))
    y = torch.stack(steps, dim=1) if steps else x.new_zeros(x.shape)
    if D is not None:
        skip = D.to(dtype)
        y = y + x * (skip.view(1, 1, nheads, 1) if skip.dim() == 1 else skip.view(1, 1, nheads, headdim))
    if z is not None:
        y = y * torch.nn.functional.silu(z.to(dtype))
    return y.to(out_dtype), state.to(out_dtype)
