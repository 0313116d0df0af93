"""Pure PyTorch selective scan: the explicit recurrence, on any device.

Public twin of the reference's ``reference.py``: ``x_t = exp(dt_t A) x_{t-1} +
dt_t B_t u_t`` and ``y_t = <x_t, C_t>``, zero initial state, no ``D``/``z``.  It
is written functionally (the state is rebuilt every step, vectorised over batch,
channels and states), so autograd can differentiate it; it walks the sequence one
step at a time and is meant for small inputs.
"""

import torch


def selective_scan(u, dt, A, B, C):
    """Reference selective scan.

    Args:
        u, dt: (batch, dim, length)
        A: (dim, dstate)
        B, C: (batch, groups, dstate, length), groups dividing dim

    Returns:
        (batch, dim, length) in u's dtype.
    """
    batch, dim, length = u.shape
    groups = B.shape[1]
    if dim % groups != 0:
        raise ValueError("dim must be divisible by groups")
    per_group = dim // groups
    Bc = B.repeat_interleave(per_group, dim=1)
    Cc = C.repeat_interleave(per_group, dim=1)
    x = u.new_zeros(batch, dim, A.shape[1])
    outs = []
    for t in range(length):
        step = dt[:, :, t]
        x = torch.exp(step.unsqueeze(-1) * A) * x + (step * u[:, :, t]).unsqueeze(-1) * Bc[..., t]
        outs.append((x * Cc[..., t]).sum(-1))
    if not outs:
        return u.new_zeros(batch, dim, 0)
    return torch.stack(outs, dim=-1).to(u.dtype)
