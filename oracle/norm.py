"""Float64 CPU restatement of the reference's gated RMSNorm (test oracle).

Reference paths are relative to dbydd/metal-kernelops ``src/metal_kernelops/``.
Nothing here is imported by the product.
"""

from __future__ import annotations

import torch

F64 = torch.float64


def _grouped(t, group):
    return t.reshape(t.shape[:-1] + (t.shape[-1] // group, group))


def rmsnorm_gated(x, weight, bias=None, z=None, eps=1e-5, group_size=None, norm_before_gate=True, dtype=F64):
    """Gated RMSNorm forward in ``dtype``, differentiable.

    Restates ``rms_norm_ref`` as the reference states it (``cv/gated_norm.py:1-20`` and
    ``:689-721``): silu(z) multiplies x before the mean square when
    ``norm_before_gate`` is False and the output after the shift when it is True; the
    mean is biased, over ``group_size`` consecutive features.  Returns
    ``(out, rstd)`` with ``rstd`` shaped ``x.shape[:-1] + (features // group,)``.
    """
    features = x.shape[-1]
    group = features if group_size is None else group_size
    xf = x.to(dtype)
    gate = torch.nn.functional.silu(z.to(dtype)) if z is not None else None
    if gate is not None and not norm_before_gate:
        xf = xf * gate
    g = _grouped(xf, group)
    rstd = torch.rsqrt(g.square().mean(-1) + eps)
    out = (g * rstd.unsqueeze(-1)).reshape(xf.shape) * weight.to(dtype)
    if bias is not None:
        out = out + bias.to(dtype)
    if gate is not None and norm_before_gate:
        out = out * gate
    return out, rstd


def rmsnorm_gated_bwd(dout, x, weight, bias=None, z=None, eps=1e-5, group_size=None, norm_before_gate=True,
                      dtype=F64):
    """The analytic gradients ``(dx, dweight, dbias, dz)`` in ``dtype`` (dz None without z).

    Restates the backward of ``cv/gated_norm.py:185-250`` (and its wide-group split,
    ``:283-340``): with ``xh = x' r`` and ``g = dout * silu(z)`` (gate after) or ``dout``,
    ``c1 = sum(xh g w) / group`` per group, ``dx' = r (g w - xh c1)``; the gate before
    gives ``dx = dx' silu(z)`` and ``dz = dx' x silu'(z)``, the gate after
    ``dz = dout (xh w + b) silu'(z)``; ``dweight = sum over rows of g xh`` and
    ``dbias = sum over rows of g``.  ``silu'(z) = s (1 + z (1 - s))``, ``s = sigmoid(z)``.
    """
    features = x.shape[-1]
    group = features if group_size is None else group_size
    xf, dy, w = x.to(dtype), dout.to(dtype), weight.to(dtype)
    b = bias.to(dtype) if bias is not None else torch.zeros_like(w)
    if z is not None:
        zf = z.to(dtype)
        s = torch.sigmoid(zf)
        silu = zf * s
        slope = s * (1 + zf * (1 - s))
    xp = xf * silu if z is not None and not norm_before_gate else xf
    rstd = torch.rsqrt(_grouped(xp, group).square().mean(-1) + eps)
    r = rstd.repeat_interleave(group, dim=-1)
    xh = xp * r
    g = dy * silu if z is not None and norm_before_gate else dy
    c1 = _grouped(xh * g * w, group).sum(-1) / group
    dxp = (g * w - xh * c1.repeat_interleave(group, dim=-1)) * r
    dz = None
    if z is not None and not norm_before_gate:
        dz = dxp * xf * slope
        dx = dxp * silu
    else:
        dx = dxp
        if z is not None:
            dz = dy * (xh * w + b) * slope
    lead = tuple(range(x.dim() - 1))
    dweight = (g * xh).sum(lead) if lead else g * xh
    dbias = g.sum(lead) if lead else g
    return dx, dweight, dbias, dz
