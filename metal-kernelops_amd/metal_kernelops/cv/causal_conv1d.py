"""Causal depthwise conv1d on MI355X: the convolution ahead of every Mamba block.

Public surface, as in dbydd/metal-kernelops ``cv/causal_conv1d.py:495-756``:
``causal_conv1d_fn`` (prefill over a sequence, with an analytic backward),
``causal_conv1d_update`` (decode: q tokens against a rolling state, in place) and
``causal_conv1d_ref`` (the pure-torch definition).

With ``z = cat(initial_state or zeros(K-1), x)`` along time::

    out[b, c, t] = act(bias[c] + sum_{j < K} weight[c, j] * z[b, c, t + j])
    final_state  = z[..., L : L + K - 1]

``act`` is ``None`` or SiLU (``"silu"`` / ``"swish"``).  Arithmetic follows
``weight.dtype`` (x, bias and the state are cast to it) and the result comes back
in ``x.dtype``, as in the reference; the HIP kernels compute in float32 and round
once on the store.

How it runs: ``mko::conv1d_fwd`` fuses the taps, the bias, the SiLU and (without
autograd) the final state in one pass; ``mko::conv1d_bwd`` recomputes the
pre-activation over each lane's window and writes dx, the initial-state gradient and
deterministic per-segment tap/bias partials that a second kernel sums in a fixed
order.  With a gradient in play the final state is a slice of ``cat(initial_state,
x)`` taken in torch, so its gradient flows to both, as in the reference
(``:483-492, 642-673``).  ``mko::conv1d_update`` advances the state through its
strides in place.

Differences from the reference: tensors live on the ROCm GPU (the reference's other
devices and dtypes run an ATen composition, ``:471-480, 676-687``); float32, float16
and bfloat16 run the kernels and other dtypes raise ``ValueError``; ``K <= 32``.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor

from .. import _native as nat
from .._contract import Rules
from ..scan import _require_gpu

__all__ = ["causal_conv1d_fn", "causal_conv1d_ref", "causal_conv1d_update"]

_ACTIVATIONS = (None, "silu", "swish")
_FLOATS = (torch.float32, torch.float16, torch.bfloat16)
_SILU = 1
_MAX_WIDTH = 32


def _as_depthwise(weight, op="causal_conv1d"):
    """The taps as a (channels, K) matrix.

    Accepts the (channels, K) matrix itself or the (channels, 1, K) weight of an
    ``nn.Conv1d`` with ``groups == channels``; K must be at least 1."""
    rules = Rules(op)
    if weight.dim() == 3:
        rules.require(weight.shape[1] == 1, "a 3-d weight must be the depthwise (channels, 1, K) layout; "
                                            f"its shape is {tuple(weight.shape)}")
        weight = weight.squeeze(1)
    rules.require(weight.dim() == 2, "weight should be (channels, K) or (channels, 1, K); "
                                     f"its shape is {tuple(weight.shape)}")
    rules.require(weight.shape[1] >= 1, "weight has no taps (K = 0)")
    return weight


def _check_activation(activation, op="causal_conv1d"):
    """Only no activation, "silu" or its alias "swish" are implemented."""
    if activation not in _ACTIVATIONS:
        Rules(op).fail(f"activation {activation!r} is not implemented; use one of {_ACTIVATIONS}",
                       NotImplementedError)


def _final_state(z_input, initial_state, taps):
    """The state leaving the sequence: the last ``taps`` columns of the concatenation
    ``[initial_state or zeros, z_input]`` along time, kept in the autograd graph."""
    length = z_input.shape[-1]
    short = taps - length  # columns that must come from before the sequence
    if short <= 0:
        return z_input[..., -taps:].contiguous() if taps else z_input[..., length:].contiguous()
    if initial_state is None:
        before = z_input.new_zeros(*z_input.shape[:-1], short)
    else:
        before = initial_state[..., initial_state.shape[-1] - short:]
    return torch.cat([before, z_input], dim=-1)


# --------------------------------------------------------------------------- kernels


def _params(x, weight, bias, init, silu):
    p = nat.Conv1dParams()
    p.x, p.weight, p.bias, p.initial_state = nat.ptr(x), nat.ptr(weight), nat.ptr(bias), nat.ptr(init)
    p.batch, p.channels, p.length = x.shape
    p.width = weight.shape[1]
    p.dtype = nat.code(x.dtype)
    p.flags = _SILU if silu else 0
    return p


@torch.library.custom_op("mko::conv1d_fwd", mutates_args=(), device_types="cuda")
def _conv1d_fwd(x: Tensor, weight: Tensor, bias: Optional[Tensor], init: Optional[Tensor], silu: bool,
                write_final: bool) -> Tuple[Tensor, Tensor]:
    out = torch.empty_like(x)
    final = x.new_empty(x.shape[0], x.shape[1], weight.shape[1] - 1 if write_final else 0)
    if x.numel() == 0:
        return out, final
    p = _params(x, weight, bias, init, silu)
    p.out = out.data_ptr()
    p.final_state = final.data_ptr() if write_final and final.numel() else None
    nat.check(nat.lib().mko_conv1d_fwd(ctypes.byref(p), nat.stream_of(x.device)), "mko_conv1d_fwd")
    return out, final


@_conv1d_fwd.register_fake
def _(x, weight, bias, init, silu, write_final):
    return torch.empty_like(x), x.new_empty(x.shape[0], x.shape[1], weight.shape[1] - 1 if write_final else 0)


@torch.library.custom_op("mko::conv1d_bwd", mutates_args=(), device_types="cuda")
def _conv1d_bwd(dout: Tensor, x: Tensor, weight: Tensor, bias: Optional[Tensor], init: Optional[Tensor],
                silu: bool, need_weight: bool, need_bias: bool, need_init: bool
                ) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    channels, width = weight.shape
    dx = torch.empty_like(x)
    # the kernels write every element of these; an empty input launches nothing and
    # leaves zeros
    empty = x.numel() == 0
    wnew = weight.new_zeros if empty else weight.new_empty
    dweight = wnew(weight.shape) if need_weight else weight.new_empty(0)
    dbias = wnew(channels) if need_bias else weight.new_empty(0)
    dinit = (x.new_zeros if empty else x.new_empty)(x.shape[0], channels, width - 1) if need_init else x.new_empty(0)
    if empty:
        return dx, dweight, dbias, dinit
    p = _params(x, weight, bias, init, silu)
    p.dout, p.dx = dout.data_ptr(), dx.data_ptr()
    p.dweight = dweight.data_ptr() if need_weight else None
    p.dbias = dbias.data_ptr() if need_bias else None
    p.dinitial = dinit.data_ptr() if need_init and dinit.numel() else None
    ws = nat.workspace(nat.lib().mko_conv1d_bwd_workspace_size(ctypes.byref(p)), x.device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    nat.check(nat.lib().mko_conv1d_bwd(ctypes.byref(p), nat.stream_of(x.device)), "mko_conv1d_bwd")
    return dx, dweight, dbias, dinit


@_conv1d_bwd.register_fake
def _(dout, x, weight, bias, init, silu, need_weight, need_bias, need_init):
    channels, width = weight.shape
    return (torch.empty_like(x), weight.new_empty(weight.shape if need_weight else (0,)),
            weight.new_empty(channels if need_bias else 0),
            x.new_empty((x.shape[0], channels, width - 1) if need_init else (0,)))


def _setup(ctx, inputs, output):
    x, weight, bias, init, silu, _ = inputs
    ctx.save_for_backward(x, weight, bias, init)
    ctx.silu = silu


def _backward(ctx, dout, _dfinal):
    x, weight, bias, init = ctx.saved_tensors
    need = ctx.needs_input_grad
    dx, dweight, dbias, dinit = torch.ops.mko.conv1d_bwd(
        dout.contiguous(), x, weight, bias, init, ctx.silu, bool(need[1]), bool(need[2] and bias is not None),
        bool(need[3] and init is not None))
    return (dx, dweight if need[1] else None, dbias if need[2] and bias is not None else None,
            dinit if need[3] and init is not None else None, None, None)


torch.library.register_autograd("mko::conv1d_fwd", _backward, setup_context=_setup)


@torch.library.custom_op("mko::conv1d_update", mutates_args=("state",), device_types="cuda")
def _conv1d_update(x: Tensor, state: Tensor, weight: Tensor, bias: Optional[Tensor], silu: bool) -> Tensor:
    out = torch.empty_like(x)
    if x.numel() == 0:
        return out
    p = nat.Conv1dUpdateParams()
    p.x, p.state, p.weight, p.bias, p.out = x.data_ptr(), state.data_ptr(), weight.data_ptr(), nat.ptr(bias), \
        out.data_ptr()
    p.batch, p.channels, p.q = x.shape
    p.span, p.width = state.shape[-1], weight.shape[1]
    p.state_stride_b, p.state_stride_c = state.stride(0), state.stride(1)
    p.dtype, p.flags = nat.code(x.dtype), _SILU if silu else 0
    nat.check(nat.lib().mko_conv1d_update(ctypes.byref(p), nat.stream_of(x.device)), "mko_conv1d_update")
    return out


@_conv1d_update.register_fake
def _(x, state, weight, bias, silu):
    return torch.empty_like(x)


# --------------------------------------------------------------------------- public API


def causal_conv1d_ref(x, weight, bias=None, activation=None, initial_state=None, return_final_state=False):
    """Reference definition, explicit taps on any device and dtype, differentiable.

    Same contract as :func:`causal_conv1d_fn` (``cv/causal_conv1d.py:495-530``):
    computed in ``weight.dtype``, rounded to ``x.dtype``, then the SiLU.
    """
    weight = _as_depthwise(weight)
    _check_activation(activation)
    channels, width = weight.shape
    if x.dim() != 3 or x.shape[1] != channels:
        raise ValueError(f"x must be (batch, {channels}, length), got {tuple(x.shape)}")
    taps, length = width - 1, x.shape[-1]
    z = x.to(weight.dtype)
    lead = initial_state.to(weight.dtype) if initial_state is not None else z.new_zeros(z.shape[:-1] + (taps,))
    z = torch.cat([lead, z], dim=-1)
    out = sum(z[..., j:j + length] * weight[:, j].view(1, channels, 1) for j in range(width))
    if bias is not None:
        out = out + bias.to(weight.dtype).view(1, channels, 1)
    out = out.to(x.dtype)
    if activation is not None:
        out = F.silu(out)
    if return_final_state:
        return out, z[..., length:].to(x.dtype)
    return out


def _check_prefill(x, weight, bias, initial_state):
    """The prefill contract, rule by rule: x is 3-d with weight's channel count, bias is
    one value per channel, the initial state spans K-1 steps of every (batch, channel)."""
    rules = Rules("causal_conv1d_fn")
    rules.dims("x", x, 3, "(batch, channels, length)")
    channels, width = weight.shape
    rules.require(x.shape[1] == channels, f"x carries {x.shape[1]} channels against {channels} in weight")
    rules.require(bias is None or (bias.dim() == 1 and bias.shape[0] == channels),
                  f"bias should hold one value per channel, ({channels},); its shape is "
                  f"{None if bias is None else tuple(bias.shape)}")
    rules.shape("initial_state", initial_state, (x.shape[0], channels, width - 1))
    return rules


def causal_conv1d_fn(x, weight, bias=None, activation=None, initial_state=None, return_final_state=False):
    """Prefill: the causal depthwise convolution of a whole sequence, on the ROCm GPU.

    ``x`` is ``(batch, channels, length)``; ``weight`` holds K taps per channel, either as
    the ``(channels, 1, K)`` weight of a depthwise ``nn.Conv1d`` or as a ``(channels, K)``
    matrix, with K at most 32.  ``bias`` adds one value per channel.  ``activation`` is
    ``None`` (identity) or SiLU, spelled ``"silu"`` or ``"swish"``.  ``initial_state``,
    ``(batch, channels, K-1)``, stands for the K-1 steps before the sequence (zeros when
    absent).

    The result has ``x``'s shape and dtype.  With ``return_final_state`` the call returns
    ``(out, final_state)``, the last K-1 steps of ``cat(initial_state, x)``, shaped like
    ``initial_state``.
    """
    weight = _as_depthwise(weight)
    _check_activation(activation)
    rules = _check_prefill(x, weight, bias, initial_state)
    width = weight.shape[1]
    for t in (x, weight, bias, initial_state):
        if t is not None:
            _require_gpu(t)
    rules.dtype_in(_FLOATS, weight=weight)
    rules.require(width <= _MAX_WIDTH, f"at most {_MAX_WIDTH} taps run on the kernels; weight has {width}")

    compute = weight.dtype
    work = x.to(compute).contiguous()
    init = initial_state.to(compute).contiguous() if initial_state is not None else None
    shift = bias.to(compute).contiguous() if bias is not None else None
    grads = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (work, weight, init, shift))
    # without autograd the kernel writes the final state; with it, the final state is a
    # slice of cat(initial_state, x) so that its gradient reaches both
    fused_final = return_final_state and not grads
    out, final = torch.ops.mko.conv1d_fwd(work, weight.contiguous(), shift, init, activation is not None,
                                          bool(fused_final and work.numel()))
    out = out.to(x.dtype)
    if not return_final_state:
        return out
    if not (fused_final and work.numel()):
        final = _final_state(work, init, width - 1)
    return out, final.to(x.dtype)


def _check_update(x, state, weight, bias):
    """The decode contract: x is (batch, channels, q) with weight's channels; the state
    covers the same (batch, channel) pairs with at least K-1 unit-stride columns."""
    rules = Rules("causal_conv1d_update")
    rules.dims("x", x, 3, "(batch, channels) or (batch, channels, q)")
    channels, width = weight.shape
    taps = width - 1
    batch = x.shape[0]
    rules.require(x.shape[1] == channels, f"x carries {x.shape[1]} channels against {channels} in weight")
    rules.require(state.dim() == 3 and tuple(state.shape[:2]) == (batch, channels),
                  f"state should be ({batch}, {channels}, s) with s >= {taps}; its shape is {tuple(state.shape)}")
    rules.require(state.shape[-1] >= taps,
                  f"state should keep at least K-1 = {taps} columns; it keeps {state.shape[-1]}")
    rules.require(state.stride(-1) == 1,
                  f"state should have stride 1 in its last dimension (a cache slice may be strided elsewhere); "
                  f"its strides are {state.stride()}")
    rules.require(bias is None or (bias.dim() == 1 and bias.shape[0] == channels),
                  f"bias should hold one value per channel, ({channels},); its shape is "
                  f"{None if bias is None else tuple(bias.shape)}")
    return rules


def causal_conv1d_update(x, state, weight, bias=None, activation=None):
    """Decode: convolve q new tokens against a rolling state, which advances in place.

    ``x`` is ``(batch, channels)`` for one token or ``(batch, channels, q)``.  ``state``
    is ``(batch, channels, s)`` with ``s >= K-1`` and unit stride along its last axis (it
    may be a slice of a larger cache); afterwards it holds the last ``s`` columns of
    ``cat(state, x)``.  ``weight``, ``bias`` and ``activation`` are as in
    :func:`causal_conv1d_fn`.

    Returns the outputs of the q new tokens, with ``x``'s rank.  This path is for
    inference: inputs that require grad raise ``RuntimeError``
    (``cv/causal_conv1d.py:690-756``).
    """
    weight = _as_depthwise(weight)
    _check_activation(activation)
    squeezed = x.dim() == 2
    if squeezed:
        x = x.unsqueeze(-1)
    rules = _check_update(x, state, weight, bias)
    if x.requires_grad or weight.requires_grad or state.requires_grad:
        raise RuntimeError("causal_conv1d_update: the decode update carries no autograd; call it under "
                           "torch.no_grad() or on detached tensors")
    for t in (x, state, weight, bias):
        if t is not None:
            _require_gpu(t)
    rules.dtype_in(_FLOATS, state=state)
    width = weight.shape[1]
    rules.require(width <= _MAX_WIDTH, f"at most {_MAX_WIDTH} taps run on the kernels; weight has {width}")
    # the kernel reads and writes every tensor in the state's dtype, computing in float32
    dtype = state.dtype
    work = x.to(dtype).contiguous()
    out = torch.ops.mko.conv1d_update(work, state, weight.to(dtype).contiguous(),
                                      bias.to(dtype).contiguous() if bias is not None else None,
                                      activation is not None)
    out = out.to(x.dtype)
    return out.squeeze(-1) if squeezed else out
