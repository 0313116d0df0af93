"""Gated RMSNorm on MI355X: the normalisation after the SSM scan in a Mamba-2 block.

Public surface, as in dbydd/metal-kernelops ``cv/gated_norm.py:647-721``:
``rmsnorm_gated`` (fused HIP forward, analytic backward) and
``rmsnorm_gated_reference`` (the float64 torch definition it is checked against).

Per ``(row, group)`` of ``group_size`` consecutive features (the whole feature axis
when ``group_size`` is None)::

    gate = silu(z)                         when z is given
    x'   = x * gate                        if norm_before_gate is False
    r    = rsqrt(mean(x'^2 over the group) + eps)     (biased mean)
    out  = (x' * r * weight + bias) * gate  if norm_before_gate is True

Every intermediate is float32 and the result comes back in ``x.dtype``, as in the
reference (``:537-561``).

How it runs: ``mko_gated_norm_fwd`` gives each ``(row, group)`` to a team of
wavefronts that holds the group in registers from the load to the store (x and z
read once, out written once) and saves ``r`` per group; ``mko_gated_norm_bwd``
walks blocks of rows per group, writes dx and dz in the same pass and sums
``dweight``/``dbias`` in a fixed order.  Both are called through the C ABI from a
plain autograd Function (first-order, as in the reference).  Groups wider than the register set
(32768 elements forward, 8192 backward, fewer for unaligned groups) stream.

Differences from the reference: tensors live on the ROCm GPU; float32, float16 and
bfloat16 run the kernels and float64 raises ``ValueError`` (the reference's composed
float64/CPU path, ``:471-480, 537-561``, is :func:`rmsnorm_gated_reference` here).  A
``z`` of another dtype than ``x`` makes both float32 for the kernel, which is the
reference's composed arithmetic for that case.
"""

from __future__ import annotations

import ctypes

import torch
from torch.autograd.function import once_differentiable

from .. import _native as nat
from .._contract import Rules
from ..scan import _require_gpu

__all__ = ["rmsnorm_gated", "rmsnorm_gated_reference"]

GATE_NONE = 0
"""No z."""
GATE_BEFORE = 1
"""``norm_before_gate=False``: silu(z) multiplies x before the mean square."""
GATE_AFTER = 2
"""``norm_before_gate=True``: silu(z) multiplies the normalised, scaled output."""

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def _params(x, weight, bias, z, eps, group, gate):
    p = nat.GatedNormParams()
    p.x, p.z, p.weight, p.bias = x.data_ptr(), nat.ptr(z), weight.data_ptr(), nat.ptr(bias)
    p.rows, p.features = x.shape
    p.group, p.eps = group, eps
    p.dtype, p.gate, p.wdtype = nat.code(x.dtype), gate, nat.code(weight.dtype)
    return p


def _forward(x, weight, bias, z, eps, group, gate):
    """``(out, rstd)`` for contiguous ``(rows, features)`` x (and z) on the GPU."""
    rows, features = x.shape
    out = torch.empty_like(x)
    rstd = torch.empty(rows * (features // group), dtype=torch.float32, device=x.device)
    if x.numel():
        p = _params(x, weight, bias, z, eps, group, gate)
        p.out, p.rstd = out.data_ptr(), rstd.data_ptr()
        nat.check(nat.lib().mko_gated_norm_fwd(ctypes.byref(p), nat.stream_of(x.device)), "mko_gated_norm_fwd")
    return out, rstd


def _backward(dout, x, weight, bias, z, rstd, group, gate, need_weight, need_bias):
    """``(dx, dz, dweight, dbias)``; dz is None without z, dweight/dbias float32 or None."""
    features = x.shape[1]
    dx = torch.empty_like(x)
    dz = torch.empty_like(z) if z is not None else None
    dweight = torch.zeros(features, dtype=torch.float32, device=x.device) if need_weight else None
    dbias = torch.zeros(features, dtype=torch.float32, device=x.device) if need_bias else None
    if x.numel():
        p = _params(x, weight, bias, z, 0.0, group, gate)
        p.rstd, p.dout, p.dx = rstd.data_ptr(), dout.data_ptr(), dx.data_ptr()
        p.dz, p.dweight, p.dbias = nat.ptr(dz), nat.ptr(dweight), nat.ptr(dbias)
        size = nat.lib().mko_gated_norm_bwd_workspace_size(ctypes.byref(p))
        ws = nat.workspace(size, x.device) if size else None
        p.workspace, p.workspace_bytes = nat.ptr(ws), size
        nat.check(nat.lib().mko_gated_norm_bwd(ctypes.byref(p), nat.stream_of(x.device)), "mko_gated_norm_bwd")
    return dx, dz, dweight, dbias


class _GatedRMSNorm(torch.autograd.Function):
    """Fused forward, analytic first-order backward (as the reference's ``_GatedRMSNorm``,
    ``cv/gated_norm.py:563-645``).  A plain autograd Function calling the C ABI: the
    host cost per call is a few microseconds, which is what a layer this short needs."""

    @staticmethod
    def forward(ctx, x, weight, bias, z, eps, group, gate):
        out, rstd = _forward(x, weight, bias, z, eps, group, gate)
        ctx.save_for_backward(x, weight, bias, z, rstd)
        ctx.group, ctx.gate = group, gate
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        x, weight, bias, z, rstd = ctx.saved_tensors
        need = ctx.needs_input_grad
        need_bias = bool(need[2] and bias is not None)
        dx, dz, dweight, dbias = _backward(dout.contiguous(), x, weight, bias, z, rstd, ctx.group, ctx.gate,
                                           bool(need[1]), need_bias)
        return (dx, dweight.to(weight.dtype) if need[1] else None, dbias.to(bias.dtype) if need_bias else None,
                dz if z is not None and need[3] else None, None, None, None)


def _checked_group(x, weight, bias, z, group_size):
    """Width of the normalisation groups after the reference's argument rules
    (``cv/gated_norm.py:674-684``, same order), for a non-empty feature axis."""
    rules = Rules("rmsnorm_gated")
    features = x.shape[-1]
    group = int(group_size) if group_size is not None else features
    rules.require(group > 0 and features % group == 0,
                  f"{features} features do not split into whole groups of {group}")
    rules.shape("weight", weight, (features,))
    rules.shape("bias", bias, (features,))
    rules.shape("z", z, tuple(x.shape))
    return group


def rmsnorm_gated(x, weight, bias=None, z=None, eps=1e-5, group_size=None, norm_before_gate=True):
    """Gated RMSNorm over the last axis, as in ``mamba_ssm``'s ``RMSNorm``.

    Args:
        x: ``(..., features)``, float32, float16 or bfloat16 on the ROCm GPU.
        weight: ``(features,)`` scale, any float dtype (read as float32; its gradient
            comes back in its own dtype).
        bias: ``(features,)`` shift, added before the gate, or None.
        z: the gate, shaped like ``x``, or None.
        eps: added to the mean square before the reciprocal square root.
        group_size: elements per normalisation group; None means the whole feature
            axis.  Must divide ``features``.
        norm_before_gate: True applies silu(z) after the normalisation, False to the
            input before it.

    Returns:
        ``(..., features)`` in ``x.dtype``.
    """
    if x.dim() < 1:
        raise ValueError("rmsnorm_gated needs a feature axis")
    features = x.shape[-1]
    if features == 0:
        return x.clone()  # nothing to average over, as in the reference
    group = _checked_group(x, weight, bias, z, group_size)
    for t in (x, weight, bias, z):
        if t is not None:
            _require_gpu(t)
    if x.dtype not in _FLOATS:
        raise ValueError(f"rmsnorm_gated runs float32, float16 or bfloat16 on the GPU, got {x.dtype}; "
                         "rmsnorm_gated_reference evaluates other dtypes")
    if z is not None and z.dtype not in _FLOATS:
        raise ValueError(f"z must be float32, float16 or bfloat16, got {z.dtype}")
    work = x.dtype if z is None or z.dtype == x.dtype else torch.float32
    shape = x.shape
    rows_x = x.reshape(-1, features).to(work).contiguous()
    rows_z = z.reshape(-1, features).to(work).contiguous() if z is not None else None
    gate = GATE_NONE if z is None else (GATE_AFTER if norm_before_gate else GATE_BEFORE)
    # weight and bias are read in their own dtype when it is one the kernels take
    pdtype = weight.dtype if weight.dtype in _FLOATS else torch.float32
    w = weight.to(pdtype).contiguous()
    b = bias.to(pdtype).contiguous() if bias is not None else None
    out = _GatedRMSNorm.apply(rows_x, w, b, rows_z, float(eps), group, gate)
    return out.reshape(shape).to(x.dtype)


def rmsnorm_gated_reference(x, weight, bias=None, z=None, eps=1e-5, group_size=None, norm_before_gate=True):
    """``rms_norm_ref`` of mamba's ``layernorm_gated.py``, evaluated in float64 with torch.

    The specification the kernels are checked against (``cv/gated_norm.py:689-721``):
    gate before the mean, scale, shift, gate after, biased mean.  Like the
    reference it runs on the CPU and returns a CPU tensor of ``x.dtype``;
    differentiable.
    """
    out_dtype = x.dtype
    xf = x.to("cpu").double()
    weightf = weight.to("cpu").double()
    biasf = bias.to("cpu").double() if bias is not None else None
    zf = z.to("cpu").double() if z is not None else None
    features = xf.shape[-1]
    if features == 0:
        return torch.empty(x.shape, dtype=out_dtype)
    group = features if group_size is None else group_size
    if zf is not None and not norm_before_gate:
        xf = xf * torch.nn.functional.silu(zf)
    grouped = xf.reshape(xf.shape[:-1] + (features // group, group))
    rstd = torch.rsqrt(grouped.square().mean(-1, keepdim=True) + eps)
    out = (grouped * rstd).reshape(xf.shape) * weightf
    if biasf is not None:
        out = out + biasf
    if zf is not None and norm_before_gate:
        out = out * torch.nn.functional.silu(zf)
    return out.to(out_dtype)
