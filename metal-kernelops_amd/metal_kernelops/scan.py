"""Mamba-1 selective scan on MI355X: fused forward, analytic backward, HIP kernels.

Public surface, as in dbydd/metal-kernelops ``scan.py:283-329``:

* ``selective_scan(u, dt, A, B, C, D=None, z=None, delta_bias=None,
  delta_softplus=False)`` and its alias ``selective_scan_fn``;
* ``scan_mps(u, dt, A, B, C)``: the bare scan, kept under the reference's name so
  callers switch without edits (it runs on the ROCm GPU, not on MPS);
* ``scan_reference(u, dt, A, B, C)``: the pure-torch recurrence;
* ``CHUNK``, ``BLOCK``.

Differences from the reference, all widenings: the discretisation, the ``D`` skip
and the ``silu(z)`` gate run inside the kernel instead of as separate torch ops
(``scan.py:311-319``); u/z/B/C may be float16 or bfloat16 (computed in float32,
rounded once on the store); dB/dC are summed over channels in a fixed order (the
reference adds them with float atomics, ``scan.py:226-227``), so the backward is
bit-deterministic.  The backward is once-differentiable, as in the reference
(``scan.py:258``).  Tensors must live on a ROCm GPU; there is no CPU path.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _native as nat

CHUNK = 16
"""Steps between the scan states the forward saves for the backward, which recomputes each
16-step block from its saved state (the reference's CHUNK, 64, is its replay chunk and
per-thread history length)."""

BLOCK = 16
"""Channels whose dB/dC terms the backward adds inside one workgroup before it writes a
partial sum (the lane-per-state backward; groups whose width is not a multiple of 16 use
4-channel partials).  The reference's BLOCK, 8, plays the same role for its threadgroups.
Informational: the kernels choose their own reduction widths from the shapes."""

_SOFTPLUS = 1
_FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def _params(u, delta, A, B, C, D, z, bias, softplus):
    batch, dim, length = u.shape
    p = nat.SelscanParams()
    p.u, p.delta, p.A, p.B, p.C = (nat.ptr(t) for t in (u, delta, A, B, C))
    p.D, p.z, p.delta_bias = nat.ptr(D), nat.ptr(z), nat.ptr(bias)
    p.batch, p.dim, p.length = batch, dim, length
    p.dstate, p.ngroups = A.shape[1], B.shape[1]
    p.u_dtype, p.delta_dtype, p.bc_dtype = nat.code(u.dtype), nat.code(delta.dtype), nat.code(B.dtype)
    p.flags = _SOFTPLUS if softplus else 0
    return p


_CHECKPOINT = 16  # MKO_SS_CHECKPOINT: steps between the scan states the forward saves


def _num_checkpoints(length):
    return (length + _CHECKPOINT - 1) // _CHECKPOINT


def selscan_fwd_impl(u: Tensor, delta: Tensor, A: Tensor, B: Tensor, C: Tensor, D: Optional[Tensor],
                     z: Optional[Tensor], delta_bias: Optional[Tensor], softplus: bool
                     ) -> Tuple[Tensor, Tensor]:
    """The forward launch behind ``mko::selscan_fwd``; callers that compose several launches
    in their own autograd function (the 2D scan) call it without the dispatcher."""
    batch, dim, length = u.shape
    out = torch.empty_like(u)
    states = torch.empty(batch, _num_checkpoints(length), dim, A.shape[1], dtype=torch.float32,
                         device=u.device)
    if out.numel() == 0:
        return out, states
    lib = nat.lib()
    p = _params(u, delta, A, B, C, D, z, delta_bias, softplus)
    p.out, p.states = out.data_ptr(), states.data_ptr()
    ws = nat.workspace(lib.mko_selscan_fwd_workspace_size(ctypes.byref(p)), u.device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    nat.check(lib.mko_selscan_fwd(ctypes.byref(p), nat.stream_of(u.device)), "mko_selscan_fwd")
    return out, states


_selscan_fwd = torch.library.custom_op("mko::selscan_fwd", selscan_fwd_impl, mutates_args=(), device_types="cuda")


@_selscan_fwd.register_fake
def _(u, delta, A, B, C, D, z, delta_bias, softplus):
    batch, dim, length = u.shape
    return torch.empty_like(u), u.new_empty(batch, _num_checkpoints(length), dim, A.shape[1],
                                            dtype=torch.float32)


def selscan_bwd_impl(dout: Tensor, u: Tensor, delta: Tensor, A: Tensor, B: Tensor, C: Tensor,
                     D: Optional[Tensor], z: Optional[Tensor], delta_bias: Optional[Tensor],
                     softplus: bool, states: Tensor, out: Optional[Tensor] = None
                     ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The backward launch behind ``mko::selscan_bwd`` (see ``selscan_fwd_impl``).  ``out``, the
    forward's output, lets the kernels recover the pre-gate output for dz as out / silu(z)
    instead of summing it over the states again; it is optional."""
    dim = u.shape[1]
    f32 = dict(dtype=torch.float32, device=u.device)
    du, ddelta = torch.empty_like(u), torch.empty_like(delta)
    if u.numel() == 0:
        return (du, ddelta, torch.zeros(A.shape, **f32), torch.zeros_like(B), torch.zeros_like(C),
                torch.zeros(dim if D is not None else 0, **f32),
                torch.zeros_like(z) if z is not None else u.new_empty(0),
                torch.zeros(dim if delta_bias is not None else 0, **f32))
    # every element of these is written by the kernels
    dA = torch.empty(A.shape, **f32)
    dB, dC = torch.empty_like(B), torch.empty_like(C)
    dD = torch.empty(dim if D is not None else 0, **f32)
    dz = torch.empty_like(z) if z is not None else u.new_empty(0)
    dbias = torch.empty(dim if delta_bias is not None else 0, **f32)
    lib = nat.lib()
    p = _params(u, delta, A, B, C, D, z, delta_bias, softplus)
    p.states, p.dout = states.data_ptr(), dout.data_ptr()
    p.out = nat.ptr(out)
    p.du, p.ddelta, p.dA, p.dB, p.dC = (t.data_ptr() for t in (du, ddelta, dA, dB, dC))
    p.dD = dD.data_ptr() if D is not None else None
    p.dz = dz.data_ptr() if z is not None else None
    p.ddelta_bias = dbias.data_ptr() if delta_bias is not None else None
    ws = nat.workspace(lib.mko_selscan_bwd_workspace_size(ctypes.byref(p)), u.device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    nat.check(lib.mko_selscan_bwd(ctypes.byref(p), nat.stream_of(u.device)), "mko_selscan_bwd")
    return du, ddelta, dA, dB, dC, dD, dz, dbias


_selscan_bwd = torch.library.custom_op("mko::selscan_bwd", selscan_bwd_impl, mutates_args=(), device_types="cuda")


@_selscan_bwd.register_fake
def _(dout, u, delta, A, B, C, D, z, delta_bias, softplus, states, out=None):
    dim = u.shape[1]
    return (torch.empty_like(u), torch.empty_like(delta), A.new_empty(A.shape, dtype=torch.float32),
            torch.empty_like(B), torch.empty_like(C), u.new_empty(dim if D is not None else 0,
                                                                  dtype=torch.float32),
            torch.empty_like(z) if z is not None else u.new_empty(0),
            u.new_empty(dim if delta_bias is not None else 0, dtype=torch.float32))


def _setup(ctx, inputs, output):
    u, delta, A, B, C, D, z, delta_bias, softplus = inputs
    # the output too: with a gate, the backward reads the pre-gate output back from it
    ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, output[1], output[0] if z is not None else None)
    ctx.softplus = softplus
    # the saved states (the op's second output) never receive a gradient: without this,
    # autograd would fill a zero tensor of their size (335 MB at 4 x 5120 x 4096) per backward
    ctx.set_materialize_grads(False)


def _backward(ctx, dout, _dstates):
    if dout is None:
        return (None,) * 9
    u, delta, A, B, C, D, z, bias, states, out = ctx.saved_tensors
    du, ddelta, dA, dB, dC, dD, dz, dbias = torch.ops.mko.selscan_bwd(
        dout.contiguous(), u, delta, A, B, C, D, z, bias, ctx.softplus, states, out)
    return (du, ddelta, dA, dB, dC, dD if D is not None else None, dz if z is not None else None,
            dbias if bias is not None else None, None)


torch.library.register_autograd("mko::selscan_fwd", _backward, setup_context=_setup)


def _require_gpu(t):
    if t.device.type != "cuda" or torch.version.hip is None:
        raise ValueError("HIP kernels need tensors on a ROCm GPU (torch device 'cuda'), "
                         f"got {t.device}")


def _check_shapes(u, dt, A, B, C, D, z, delta_bias):
    if u.dim() != 3:
        raise ValueError(f"u must be (batch, dim, length), got {tuple(u.shape)}")
    batch, dim, length = u.shape
    if tuple(dt.shape) != (batch, dim, length):
        raise ValueError(f"dt must be {(batch, dim, length)}, got {tuple(dt.shape)}")
    if A.dim() != 2 or A.shape[0] != dim:
        raise ValueError(f"A must be ({dim}, dstate), got {tuple(A.shape)}")
    dstate = A.shape[1]
    if B.dim() != 4 or tuple(C.shape) != tuple(B.shape):
        raise ValueError(f"B and C must both be (batch, groups, dstate, length), got "
                         f"{tuple(B.shape)} and {tuple(C.shape)}")
    if B.shape[0] != batch or B.shape[2] != dstate or B.shape[3] != length:
        raise ValueError(f"B/C must be ({batch}, groups, {dstate}, {length}), got {tuple(B.shape)}")
    groups = B.shape[1]
    if groups < 1 or dim % groups:
        raise ValueError(f"dim={dim} must be divisible by groups={groups}")
    if dstate < 1 or dstate > 32:
        raise ValueError(f"dstate must be in [1, 32], got {dstate}")
    if D is not None and tuple(D.shape) != (dim,):
        raise ValueError(f"D must be ({dim},), got {tuple(D.shape)}")
    if z is not None and tuple(z.shape) != (batch, dim, length):
        raise ValueError(f"z must be {(batch, dim, length)}, got {tuple(z.shape)}")
    if delta_bias is not None and tuple(delta_bias.shape) != (dim,):
        raise ValueError(f"delta_bias must be ({dim},), got {tuple(delta_bias.shape)}")
    for name, t in (("u", u), ("dt", dt), ("A", A), ("B", B), ("C", C), ("D", D), ("z", z),
                    ("delta_bias", delta_bias)):
        if t is None:
            continue
        if t.dtype not in _FLOATS:
            raise ValueError(f"{name} must be float32, float16 or bfloat16, got {t.dtype}")
        if t.device != u.device:
            raise ValueError(f"{name} is on {t.device}, u is on {u.device}")


def _run(u, dt, A, B, C, D, z, delta_bias, softplus):
    _require_gpu(u)
    _check_shapes(u, dt, A, B, C, D, z, delta_bias)
    if dt.dtype != torch.float32:
        dt = dt.float()  # the kernels take float32 step sizes (autograd casts ddelta back)
    if B.dtype != C.dtype:
        B, C = B.float(), C.float()
    if z is not None and z.dtype != u.dtype:
        z = z.to(u.dtype)
    f32 = [None if t is None else (t if t.dtype == torch.float32 else t.float()) for t in (A, D, delta_bias)]
    A, D, delta_bias = (None if t is None else t.contiguous() for t in f32)
    u, dt, B, C = (t.contiguous() for t in (u, dt, B, C))
    z = None if z is None else z.contiguous()
    out, _ = torch.ops.mko.selscan_fwd(u, dt, A, B, C, D, z, delta_bias, bool(softplus))
    return out


def scan_mps(u, dt, A, B, C):
    """Bare selective scan on the ROCm GPU (name kept from the reference's Metal entry).

    Follows ``scan.py:283-292``: a ``ValueError`` for tensors off the GPU or not
    contiguous.  float16/bfloat16 are accepted in addition to float32.
    """
    _require_gpu(u)
    for name, tensor in (("u", u), ("dt", dt), ("A", A), ("B", B), ("C", C)):
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    return _run(u, dt, A, B, C, None, None, None, False)


def selective_scan(u, dt, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False):
    """The Mamba-1 selective scan with mamba_ssm's ``selective_scan_fn`` call signature.

    ``u`` and the step sizes ``dt`` are ``(batch, dim, length)``.  ``A`` is the
    ``(dim, dstate)`` state matrix (negative entries; at most 32 states).  ``B`` and ``C``
    are ``(batch, groups, dstate, length)``, each group shared by ``dim / groups``
    consecutive channels.  Optional: ``D``, a ``(dim,)`` skip weight on ``u``; ``z``, a
    ``(batch, dim, length)`` gate that multiplies the result by ``silu(z)``;
    ``delta_bias``, ``(dim,)``, added to ``dt``; ``delta_softplus``, which passes
    ``dt + delta_bias`` through softplus (threshold 20) before the scan.

    Returns the ``(batch, dim, length)`` output in ``u``'s dtype, differentiable in
    every tensor argument.
    """
    return _run(u, dt, A, B, C, D, z, delta_bias, delta_softplus)


selective_scan_fn = selective_scan


def scan_reference(u, dt, A, B, C):
    """Pure torch selective scan, evaluated step by step."""
    from .reference import selective_scan as reference_scan
    return reference_scan(u, dt, A, B, C)
