"""Float64 CPU restatement of the reference's causal depthwise conv1d (test oracle).

Reference paths are relative to dbydd/metal-kernelops ``src/metal_kernelops/``.
Nothing here is imported by the product.
"""

from __future__ import annotations

import torch

F64 = torch.float64


def causal_conv1d(x, weight, bias=None, activation=None, initial_state=None, dtype=F64):
    """Causal depthwise conv1d as an explicit window product, differentiable.

    Restates the definition of ``cv/causal_conv1d.py:1-19`` and ``:495-530``: with
    ``z = cat(initial_state or zeros(K-1), x)``, each output is the K-window of z ending at
    its own step, dotted with the channel's taps, plus the bias, then SiLU if asked.
    The windows come from ``unfold``.  Returns ``(out, final_state)`` in ``dtype``.
    """
    w = weight.reshape(weight.shape[0], -1).to(dtype)
    channels, width = w.shape
    taps = width - 1
    z = x.to(dtype)
    lead = initial_state.to(dtype) if initial_state is not None else z.new_zeros(z.shape[:-1] + (taps,))
    z = torch.cat([lead, z], dim=-1)
    windows = z.unfold(-1, width, 1)                      # (b, c, L, K)
    out = (windows * w[None, :, None, :]).sum(-1)
    if bias is not None:
        out = out + bias.to(dtype)[None, :, None]
    if activation is not None:
        out = out * torch.sigmoid(out)
    return out, z[..., x.shape[-1]:]


def causal_conv1d_update(state, x, weight, bias=None, activation=None, dtype=F64):
    """One decode call: ``x`` (b, c, q) against a rolling ``state`` (b, c, s), s >= K-1.

    Restates ``cv/causal_conv1d.py:676-756``: the outputs are the convolution of
    ``cat(state, x)`` at the q new tokens and the new state is ``cat(state, x)[..., -s:]``.
    Returns ``(out, new_state)``.
    """
    w = weight.reshape(weight.shape[0], -1).to(dtype)
    width = w.shape[1]
    q, span = x.shape[-1], state.shape[-1]
    joined = torch.cat([state.to(dtype), x.to(dtype)], dim=-1)
    windows = joined[..., span + q - (q + width - 1):].unfold(-1, width, 1)   # the q windows ending at new tokens
    out = (windows * w[None, :, None, :]).sum(-1)
    if bias is not None:
        out = out + bias.to(dtype)[None, :, None]
    if activation is not None:
        out = out * torch.sigmoid(out)
    return out, joined[..., -span:]
