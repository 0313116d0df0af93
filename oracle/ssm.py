"""Float64 CPU restatements of the reference's three SSM operators (test oracle).

Reference paths are relative to dbydd/metal-kernelops ``src/metal_kernelops/``
unless they start with ``benchmarks/``.  Nothing here is imported by the product.

Notation: ``b`` batch, ``D`` channels (Mamba-1) or ``H`` heads / ``P`` head dim
(Mamba-2), ``L`` length, ``N`` state size, ``G`` groups, ``Q`` chunk size.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

F64 = torch.float64


def softplus(v: torch.Tensor) -> torch.Tensor:
    """torch's softplus with beta 1 and threshold 20: ``v`` above 20, else log1p(exp(v)).

    Follows the rule the reference relies on at ``scan.py:314``,
    ``cv/mamba2_chunk.py:457`` and ``cv/mamba2_state.py:837`` (``F.softplus``
    defaults), written out so the threshold is explicit.
    """
    return torch.where(v > 20.0, v, torch.log1p(torch.exp(torch.clamp(v, max=20.0))))


def silu(v: torch.Tensor) -> torch.Tensor:
    return v * torch.sigmoid(v)


# --------------------------------------------------------------------------- Mamba-1


def selective_scan_loop(u, dt, A, B, C, dtype=F64):
    """Literal per-(t, b, g, d) loop of the Mamba-1 recurrence, zero initial state.

    Restates ``reference.py:5-49``: ``x_t = exp(dt_t A) x_{t-1} + dt_t B_t u_t`` and
    ``y_t = <x_t, C_t>`` with channel ``g * (D / G) + d`` reading group ``g``.
    Python loops over every index, so only tiny shapes are practical.  Returns
    ``(b, D, L)`` in ``dtype``.
    """
    u, dt, A, B, C = (t.detach().to(dtype) for t in (u, dt, A, B, C))
    batch, dim, length = u.shape
    groups, states = B.shape[1], A.shape[1]
    if dim % groups:
        raise ValueError("dim must be divisible by groups")
    per_group = dim // groups
    y = torch.zeros(batch, dim, length, dtype=dtype)
    x = torch.zeros(batch, dim, states, dtype=dtype)
    for t in range(length):
        for b in range(batch):
            for g in range(groups):
                for d in range(per_group):
                    ch = g * per_group + d
                    step = float(dt[b, ch, t])
                    decay = torch.exp(A[ch] * step)
                    x[b, ch] = decay * x[b, ch] + step * float(u[b, ch, t]) * B[b, g, :, t]
                    y[b, ch, t] = torch.dot(x[b, ch], C[b, g, :, t])
    return y


def selective_scan(u, dt, A, B, C, D=None, z=None, delta_bias=None,
                   delta_softplus=False, dtype=F64):
    """Differentiable Mamba-1 selective scan with the reference's pre/post ops.

    Order follows ``scan.py:311-319``: ``dt += delta_bias``; ``dt = softplus(dt)``;
    the scan; ``+ u * D``; ``* silu(z)``.  The scan itself is the functional
    per-timestep recurrence of ``cv/path_scan.py:579-605`` (state rebuilt each step
    so autograd can differentiate it), vectorised over ``(b, D, N)``.

    Shapes: ``u, dt, z`` (b, D, L); ``A`` (D, N); ``B, C`` (b, G, N, L);
    ``D, delta_bias`` (D,).  Returns ``(b, D, L)`` in ``dtype``.
    """
    def cast(t):
        return None if t is None else t.to(dtype)

    u, dt, A, B, C, D, z, delta_bias = map(cast, (u, dt, A, B, C, D, z, delta_bias))
    if delta_bias is not None:
        dt = dt + delta_bias[..., None]
    if delta_softplus:
        dt = softplus(dt)
    batch, dim, length = u.shape
    groups = B.shape[1]
    per_group = dim // groups
    Bc = B.repeat_interleave(per_group, dim=1)  # (b, D, N, L)
    Cc = C.repeat_interleave(per_group, dim=1)
    x = u.new_zeros(batch, dim, A.shape[1])
    outs = []
    for t in range(length):
        step = dt[:, :, t]
        x = torch.exp(step[..., None] * A) * x + (step * u[:, :, t])[..., None] * Bc[..., t]
        outs.append((x * Cc[..., t]).sum(-1))
    y = torch.stack(outs, dim=-1) if outs else u.new_zeros(batch, dim, 0)
    if D is not None:
        y = y + u * D[..., None]
    if z is not None:
        y = y * silu(z)
    return y


def ss2d_path_orders(height, width):
    """The four traversal orders of an ``height x width`` map as Python lists.

    Entry ``i`` of path ``k`` is the flat ``h * width + w`` pixel visited at step ``i``:
    row-major, column-major (down each column, columns left to right), and the two
    reversed (``cv/path_scan.py:9-22, 153-162``).
    """
    row = [h * width + w for h in range(height) for w in range(width)]
    col = [h * width + w for w in range(width) for h in range(height)]
    return [row, col, row[::-1], col[::-1]]


def ss2d_scan(u, dt, A, B, C, merge="sum", dtype=F64):
    """Four-path 2D selective scan (VMamba's ss2d), differentiable.

    Restates ``cv/path_scan.py:579-639``: each path of :func:`ss2d_path_orders` is the
    Mamba-1 recurrence (:func:`selective_scan`, zero state, no skip/gate/bias) over the
    pixels in that order; the path outputs are written back at the pixels they were
    computed for and added as ``(p0 + p2) + (p1 + p3)``, times 1/4 for ``"mean"``.

    Shapes: ``u, dt`` (b, C, H, W); ``A`` (C, N); ``B, C`` (b, G, N, H, W).
    """
    batch, channels, height, width = u.shape
    groups, states = B.shape[1], B.shape[2]
    length = height * width
    uf = u.to(dtype).reshape(batch, channels, length)
    df = dt.to(dtype).reshape(batch, channels, length)
    bf = B.to(dtype).reshape(batch, groups, states, length)
    cf = C.to(dtype).reshape(batch, groups, states, length)
    paths = []
    for order in ss2d_path_orders(height, width):
        idx = torch.tensor(order, dtype=torch.long)
        yk = selective_scan(uf[..., idx], df[..., idx], A, bf[..., idx], cf[..., idx], dtype=dtype)
        back = uf.new_zeros(batch, channels, length)
        back[..., idx] = yk
        paths.append(back)
    total = (paths[0] + paths[2]) + (paths[1] + paths[3])
    if merge == "mean":
        total = total * 0.25
    return total.reshape(batch, channels, height, width)


# --------------------------------------------------------------------------- Mamba-2


def normalize_initial_states(initial_states, batch, nheads, headdim, dstate):
    """The ``initial_states`` spellings accepted by ``cv/mamba2_chunk.py:426-438``.

    A leading singleton chunk axis (5-D, the ``ssd_minimal`` form) is dropped; the
    transposed ``(b, H, N, P)`` spelling is accepted when ``N != P``; anything else
    that is not ``(b, H, P, N)`` raises ``ValueError``.
    """
    if initial_states is None:
        return None
    if initial_states.dim() == 5 and initial_states.shape[1] == 1:
        initial_states = initial_states[:, 0]
    canonical = (batch, nheads, headdim, dstate)
    if tuple(initial_states.shape) != canonical:
        if tuple(initial_states.shape) == (batch, nheads, dstate, headdim) and headdim != dstate:
            initial_states = initial_states.transpose(-1, -2)
        else:
            raise ValueError(f"initial_states must be {canonical}, got "
                             f"{tuple(initial_states.shape)}")
    return initial_states


def mamba2_chunk_scan_recurrence(x, dt, A, B, C, D=None, z=None, dt_bias=None,
                                 dt_softplus=False, initial_states=None, dtype=F64):
    """Per-token SSD recurrence, the definition the chunk scan must reproduce.

    Restates ``cv/mamba2_chunk.py:681-723``: ``dt' = softplus(dt + dt_bias)``;
    ``s_t = exp(dt'_t A_h) s_{t-1} + dt'_t x_t (x) B_t``; ``y_t = <C_t, s_t> + D x_t``;
    ``y *= silu(z)``.  Shapes: ``x, z`` (b, L, H, P); ``dt`` (b, L, H); ``A,
    dt_bias`` (H,); ``B, C`` (b, L, G, N); ``D`` (H,) or (H, P); initial state
    (b, H, P, N).  Returns ``(y, final_state)`` in ``dtype``.
    """
    batch, length, nheads, headdim = x.shape
    ngroups, dstate = B.shape[2], B.shape[3]
    initial_states = normalize_initial_states(initial_states, batch, nheads, headdim, dstate)

    def cast(t):
        return None if t is None else t.to(dtype)

    x, dt, A, B, C, D, z, dt_bias, initial_states = map(
        cast, (x, dt, A, B, C, D, z, dt_bias, initial_states))
    rep = nheads // ngroups
    Bh = B.repeat_interleave(rep, dim=2)  # (b, L, H, N)
    Ch = C.repeat_interleave(rep, dim=2)
    if dt_bias is not None:
        dt = dt + dt_bias.view(1, 1, nheads)
    if dt_softplus:
        dt = softplus(dt)
    state = x.new_zeros(batch, nheads, headdim, dstate)
    if initial_states is not None:
        state = state + initial_states
    outs = []
    for t in range(length):
        step = dt[:, t]  # (b, H)
        state = torch.exp(step * A)[..., None, None] * state \
            + (step[..., None] * x[:, t])[..., None] * Bh[:, t][:, :, None, :]
        outs.append((state * Ch[:, t][:, :, None, :]).sum(-1))
    y = torch.stack(outs, dim=1) if outs else x.new_zeros(x.shape)
    if D is not None:
        y = y + x * (D.view(1, 1, nheads, 1) if D.dim() == 1 else D.view(1, 1, nheads, headdim))
    if z is not None:
        y = y * silu(z)
    return y, state


def mamba2_chunk_scan_composition(x, dt, A, B, C, chunk_size=64, D=None, z=None,
                                  dt_bias=None, dt_softplus=False, initial_states=None):
    """The chunked SSD matmul composition -- the reference's own CPU path.

    Restates ``cv/mamba2_chunk.py:447-533`` and ``:653-678``: per-chunk
    ``dcs = cumsum(dt A)`` in float32 (float64 for float64 input); chunk states
    ``B^T (x * dt exp(dcs_last - dcs))``; the closed-form chunk transfer (a causal
    ``(nchunks, nchunks)`` decay matrix applied to the flattened states plus the
    decayed initial state); the intra-chunk ``tril(exp(dcs_l - dcs_s) C_l.B_s dt_s) x``
    and inter-chunk ``exp(dcs_l) C_l . entering`` outputs; then skip, gate and
    slice.  Score and head-state products run in ``x.dtype`` as the reference does.
    Returns ``(y, final_state)`` in ``x.dtype``.  Differentiable.
    """
    batch, length, nheads, headdim = x.shape
    ngroups, dstate = B.shape[2], B.shape[3]
    initial_states = normalize_initial_states(initial_states, batch, nheads, headdim, dstate)
    acc = F64 if x.dtype == F64 else torch.float32
    Q = min(chunk_size, length)
    nchunks = -(-length // Q)
    padded = nchunks * Q
    pad = padded - length

    d = dt.transpose(1, 2).to(acc)
    if dt_bias is not None:
        d = d + dt_bias.to(acc).view(1, nheads, 1)
    if dt_softplus:
        d = softplus(d)
    if pad:
        d = F.pad(d, (0, pad))
        x = F.pad(x, (0, 0, 0, 0, 0, pad))
        B = F.pad(B, (0, 0, 0, 0, 0, pad))
        C = F.pad(C, (0, 0, 0, 0, 0, pad))
        if z is not None:
            z = F.pad(z, (0, 0, 0, 0, 0, pad))
    d = d.reshape(batch, nheads, nchunks, Q)
    dcs = torch.cumsum(d * A.to(acc).view(1, nheads, 1, 1), dim=-1)  # (b, H, c, Q)
    rep = nheads // ngroups

    # Chunk states, (b, H, c, N, P).
    w = (d * torch.exp(dcs[..., -1:] - dcs)).permute(0, 2, 3, 1)  # (b, c, Q, H)
    xw = x.view(batch, nchunks, Q, nheads, headdim) * w[..., None].to(x.dtype)
    xg = xw.view(batch, nchunks, Q, ngroups, rep, headdim).permute(0, 3, 4, 1, 2, 5)
    Bg = B.view(batch, nchunks, Q, ngroups, dstate).permute(0, 3, 1, 2, 4)  # (b,G,c,Q,N)
    states = torch.matmul(Bg.transpose(-1, -2).unsqueeze(2), xg)  # (b,G,rep,c,N,P)
    states = states.to(acc).reshape(batch, nheads, nchunks, dstate, headdim)

    # Closed-form chunk transfer.
    total = dcs[..., -1]  # (b, H, c)
    before = torch.cumsum(F.pad(total, (1, 0)), dim=-1)  # (b, H, c+1)
    diff = before[..., :-1, None] - before[..., None, 1:]  # (b, H, c, c)
    lower = torch.ones(nchunks, nchunks, dtype=torch.bool).tril(-1)
    transfer = torch.exp(diff.masked_fill(~lower, float("-inf")))
    entering = torch.matmul(transfer, states.reshape(batch, nheads, nchunks, dstate * headdim))
    if initial_states is not None:
        carry = torch.exp(before[..., :-1]).unsqueeze(-1)
        flat_init = initial_states.to(acc).transpose(-1, -2).reshape(
            batch, nheads, dstate * headdim)
        entering = entering + carry * flat_init.unsqueeze(2)
    entering = entering.reshape(batch, nheads, nchunks, dstate, headdim)
    final = states[:, :, -1] + torch.exp(total[:, :, -1])[..., None, None] * entering[:, :, -1]
    final = final.transpose(-1, -2)  # (b, H, P, N)

    # Outputs.
    tri = torch.ones(Q, Q, dtype=torch.bool).tril()
    decay = torch.exp((dcs[..., :, None] - dcs[..., None, :]).masked_fill(~tri, float("-inf")))
    out_decay = torch.exp(dcs)
    parts = []
    for g in range(ngroups):
        heads = slice(g * rep, (g + 1) * rep)
        Cg = C[:, :, g].reshape(batch, nchunks, Q, dstate)
        Bgg = B[:, :, g].reshape(batch, nchunks, Q, dstate)
        cb = torch.matmul(Cg, Bgg.transpose(-1, -2)).to(acc)  # (b, c, Q, Q)
        scores = (decay[:, heads] * cb[:, None] * d[:, heads][..., None, :]).to(x.dtype)
        xh = x[:, :, heads].view(batch, nchunks, Q, rep, headdim).permute(0, 3, 1, 2, 4)
        intra = torch.matmul(scores, xh)  # (b, rep, c, Q, P)
        prev = torch.matmul(Cg[:, None].to(x.dtype), entering[:, heads].to(x.dtype))
        prev = prev * out_decay[:, heads][..., None].to(x.dtype)
        parts.append((intra + prev).permute(0, 2, 3, 1, 4))  # (b, c, Q, rep, P)
    y = torch.cat(parts, dim=3).reshape(batch, padded, nheads, headdim)
    if D is not None:
        skip = D.to(x.dtype)
        y = y + x * (skip.view(1, 1, nheads, 1) if skip.dim() == 1
                     else skip.view(1, 1, nheads, headdim))
    if z is not None:
        y = y * F.silu(z)
    if pad:
        y = y[:, :length]
    return y, final.to(x.dtype)


def ssd_minimal_discrete(X, A, B, C, block_len, initial_states=None):
    """``ssd_minimal_discrete`` of state-spaces/mamba, as transcribed by the reference.

    Restates ``benchmarks/verify_mamba2_chunk.py:185-212``: ``X`` is the
    already-discretised input ``x * dt``, ``A`` is ``A * dt`` per token and head
    (b, L, H); ``B, C`` (b, L, G, N) with heads sharing groups by repetition; the
    length must be a multiple of ``block_len``.  Returns ``(y, final_state)`` with
    the final state in ``(b, H, P, N)`` order.
    """
    batch, length, nheads, headdim = X.shape
    ngroups, dstate = B.shape[2], B.shape[3]
    rep = nheads // ngroups
    nchunks = length // block_len
    Xc = X.reshape(batch, nchunks, block_len, nheads, headdim)
    Ac = A.reshape(batch, nchunks, block_len, nheads).permute(0, 3, 1, 2)  # (b,H,c,l)
    Bc = B.repeat_interleave(rep, dim=2).reshape(batch, nchunks, block_len, nheads, dstate)
    Cc = C.repeat_interleave(rep, dim=2).reshape(batch, nchunks, block_len, nheads, dstate)

    def segsum(v):
        # segsum(v)[..., i, j] = sum_{j < k <= i} v[..., k] for j <= i, -inf above.
        size = v.shape[-1]
        csum = torch.cumsum(v, dim=-1)
        out = csum[..., :, None] - csum[..., None, :]
        mask = torch.ones(size, size, dtype=torch.bool).tril()
        return out.masked_fill(~mask, float("-inf"))

    A_cumsum = torch.cumsum(Ac, dim=-1)
    L_mat = torch.exp(segsum(Ac))  # (b,H,c,l,s)
    # y_diag[b,c,l,h,p] = sum_s C[l].B[s] * L[l,s] * X[s,p]
    cb = torch.einsum("bclhn,bcshn->bhcls", Cc, Bc)
    y_diag = torch.einsum("bhcls,bcshp->bclhp", cb * L_mat, Xc)
    decay_states = torch.exp(A_cumsum[..., -1:] - A_cumsum)  # (b,H,c,l)
    states = torch.einsum("bclhn,bhcl,bclhp->bchpn", Bc, decay_states, Xc)
    if initial_states is None:
        initial_states = torch.zeros_like(states[:, :1])
    states = torch.cat([initial_states, states], dim=1)  # (b, c+1, H, P, N)
    chunk_tot = F.pad(A_cumsum[..., -1], (1, 0))  # (b, H, c+1)
    decay_chunk = torch.exp(segsum(chunk_tot))  # (b, H, c+1, c+1)
    new_states = torch.einsum("bhzc,bchpn->bzhpn", decay_chunk, states)
    states, final_state = new_states[:, :-1], new_states[:, -1]
    y_off = torch.einsum("bclhn,bchpn,bhcl->bclhp", Cc, states, torch.exp(A_cumsum))
    return (y_diag + y_off).reshape(batch, length, nheads, headdim), final_state


def mamba2_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                        dt_softplus=False, dtype=F64):
    """One Mamba-2 decode step, the definition the decode kernels are checked against.

    Restates ``cv/mamba2_state.py:822-849``: ``delta = softplus(dt + dt_bias)``;
    ``s' = exp(A_h delta) s + delta x B_g``; ``y = <s', C_g> + D x``; ``y *= silu(z)``.
    Shapes: ``state`` (b, H, P, N); ``x, z`` (b, H, P); ``dt`` (b, H) or (b, H, P);
    ``A, dt_bias`` (H,); ``B, C`` (b, G, N); ``D`` (H,) or (H, P).  Returns
    ``(y, new_state)`` in ``dtype``; ``state`` is not modified.
    """
    def cast(t):
        return None if t is None else t.to(dtype)

    state, x, dt, A, B, C, D, z, dt_bias = map(cast, (state, x, dt, A, B, C, D, z, dt_bias))
    if dt.dim() == 2:
        dt = dt.unsqueeze(-1)
    if D is not None and D.dim() == 1:
        D = D.unsqueeze(-1)
    if dt_bias is not None:
        dt = dt + dt_bias[None, :, None]
    if dt_softplus:
        dt = softplus(dt)
    nheads, groups = state.shape[1], B.shape[1]
    rep = nheads // groups
    Bh = B.repeat_interleave(rep, dim=1)
    Ch = C.repeat_interleave(rep, dim=1)
    decay = torch.exp(A[None, :, None, None] * dt[..., None])
    new_state = decay * state + (dt * x)[..., None] * Bh[:, :, None, :]
    y = (new_state * Ch[:, :, None, :]).sum(-1)
    if D is not None:
        y = y + x * D
    if z is not None:
        y = y * silu(z)
    return y, new_state


def inverse_softplus_uniform(gen, n, lo=1e-3, hi=1e-1):
    """``log(expm1(U(lo, hi)))``: the dt_bias initialisation the configs specify."""
    draw = lo + (hi - lo) * torch.rand(n, generator=gen)
    return torch.log(torch.expm1(draw))

