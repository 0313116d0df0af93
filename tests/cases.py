"""Seeded input builders shared by the oracle tests, the GPU parity tests and the bench.

Draw order and distributions follow the configs of the hot-path benchmark:
one CPU generator per problem, draws in the order listed, fp32 first and then
cast; ``dt_bias = log(expm1(U(1e-3, 1e-1)))``.
"""

from __future__ import annotations

import json
import os

import torch


def uniform(gen, shape, lo, hi):
    return lo + (hi - lo) * torch.rand(shape, generator=gen)


def inv_softplus_bias(gen, n):
    return torch.log(torch.expm1(uniform(gen, (n,), 1e-3, 1e-1)))


def mamba1_c1(seed=0):
    """Config 1: batch 2, d_inner 8, seqlen 64, d_state 16, ngroups 2, fp32."""
    g = torch.Generator().manual_seed(seed)
    b, d, l, n, grp = 2, 8, 64, 16, 2
    u = torch.randn(b, d, l, generator=g)
    dt = torch.randn(b, d, l, generator=g)
    dt_bias = inv_softplus_bias(g, d)
    A = -torch.arange(1, n + 1, dtype=torch.float32).expand(d, n).contiguous()
    B = torch.randn(b, grp, n, l, generator=g)
    C = torch.randn(b, grp, n, l, generator=g)
    D = torch.ones(d)
    z = torch.randn(b, d, l, generator=g)
    dy = torch.randn(b, d, l, generator=g)
    return dict(u=u, dt=dt, A=A, B=B, C=C, D=D, z=z, delta_bias=dt_bias), dy


def mamba1_layer(batch, dim, length, dstate=16, groups=1, seed=0, act=torch.bfloat16):
    """Configs 2-3: u/z/B/C in ``act``; dt, A, D, dt_bias fp32; A = -exp(log(1..N))."""
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(batch, dim, length, generator=g)
    dt = torch.randn(batch, dim, length, generator=g)
    dt_bias = inv_softplus_bias(g, dim)
    A = -torch.exp(torch.log(torch.arange(1, dstate + 1, dtype=torch.float32)))
    A = A.expand(dim, dstate).contiguous()
    B = torch.randn(batch, groups, dstate, length, generator=g)
    C = torch.randn(batch, groups, dstate, length, generator=g)
    D = 1.0 + 0.1 * torch.randn(dim, generator=g)
    z = torch.randn(batch, dim, length, generator=g)
    dy = torch.randn(batch, dim, length, generator=g)
    return dict(u=u.to(act), dt=dt, A=A, B=B.to(act), C=C.to(act), D=D, z=z.to(act),
                delta_bias=dt_bias), dy.to(act)


def ssd_problem(batch, length, nheads, headdim, ngroups, dstate, seed=0, act=torch.float32,
                init=True, d_per_head=False):
    """Config 4 draws: x, dt, dt_bias, A=-U(1,16), B, C, D=ones, z, initial states."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, length, nheads, headdim, generator=g)
    dt = torch.randn(batch, length, nheads, generator=g)
    dt_bias = inv_softplus_bias(g, nheads)
    A = -uniform(g, (nheads,), 1.0, 16.0)
    B = torch.randn(batch, length, ngroups, dstate, generator=g)
    C = torch.randn(batch, length, ngroups, dstate, generator=g)
    D = torch.ones(nheads, headdim) if d_per_head else torch.ones(nheads)
    z = torch.randn(batch, length, nheads, headdim, generator=g)
    initial = 0.1 * torch.randn(batch, nheads, headdim, dstate, generator=g) if init else None
    return dict(x=x.to(act), dt=dt, A=A, B=B.to(act), C=C.to(act), D=D, z=z.to(act),
                dt_bias=dt_bias, initial_states=None if initial is None else initial.to(act))


def ssd_matrix_inputs(shape, seed, options=("D", "z", "dt_bias", "initial_states"), d_row=False):
    """The SSD option/shape matrix's inputs (the reference verifier's ``_problem`` draws,
    benchmarks/verify_mamba2_chunk.py:113-147): x, dt, A = -exp(U), B, C ~ N(0, 1); D, z,
    dt_bias (x0.1) and initial states (x0.1) from a second generator; the upstream gradients
    dy and d final_state (float64) from a third."""
    batch, length, nheads, headdim, ngroups, dstate = shape
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, length, nheads, headdim, generator=g)
    dt = torch.randn(batch, length, nheads, generator=g)
    A = -torch.exp(torch.rand(nheads, generator=g))
    B = torch.randn(batch, length, ngroups, dstate, generator=g)
    C = torch.randn(batch, length, ngroups, dstate, generator=g)
    inputs = dict(x=x, dt=dt, A=A, B=B, C=C)
    g = torch.Generator().manual_seed(seed + 10)
    opt = dict(D=torch.randn(nheads, generator=g),
               z=torch.randn(batch, length, nheads, headdim, generator=g),
               dt_bias=torch.randn(nheads, generator=g) * 0.1,
               initial_states=torch.randn(batch, nheads, headdim, dstate, generator=g) * 0.1)
    if d_row:
        opt["D"] = torch.randn(nheads, headdim, generator=torch.Generator().manual_seed(seed + 20))
    inputs.update({k: opt[k] for k in options})
    g = torch.Generator().manual_seed(seed + 30)
    dy = torch.randn(batch, length, nheads, headdim, generator=g, dtype=torch.float64)
    dfinal = torch.randn(batch, nheads, headdim, dstate, generator=g, dtype=torch.float64)
    return inputs, dy, dfinal


def decode_problem(batch, nheads, headdim, dstate, ngroups, seed=0, act=torch.bfloat16,
                   state_dtype=torch.float32, dt_per_row=False):
    """Config 5 draws: state=0.1*N(0,1), x, dt, dt_bias, A=-U(1,16), B, C, D=ones, z."""
    g = torch.Generator().manual_seed(seed)
    state = 0.1 * torch.randn(batch, nheads, headdim, dstate, generator=g)
    x = torch.randn(batch, nheads, headdim, generator=g)
    dt = torch.randn(*((batch, nheads, headdim) if dt_per_row else (batch, nheads)), generator=g)
    dt_bias = inv_softplus_bias(g, nheads)
    A = -uniform(g, (nheads,), 1.0, 16.0)
    B = torch.randn(batch, ngroups, dstate, generator=g)
    C = torch.randn(batch, ngroups, dstate, generator=g)
    D = torch.ones(nheads)
    z = torch.randn(batch, nheads, headdim, generator=g)
    return dict(state=state.to(state_dtype), x=x.to(act), dt=dt, A=A, B=B.to(act),
                C=C.to(act), D=D, z=z.to(act), dt_bias=dt_bias)


def max_rel(actual, expected):
    """Max absolute error over the largest expected magnitude (the reference's metric)."""
    actual = actual.detach().double().cpu()
    expected = expected.detach().double().cpu()
    scale = max(expected.abs().max().item() if expected.numel() else 0.0, 1e-30)
    if actual.numel() == 0:
        return 0.0
    return (actual - expected).abs().max().item() / scale


def norm_rel(actual, expected):
    """Relative error of a gradient, normalised by that gradient's norm."""
    actual = actual.detach().double().cpu()
    expected = expected.detach().double().cpu()
    return (actual - expected).norm().item() / max(expected.norm().item(), 1e-30)


# Parity bars of the hot path: max relative error of outputs, and norm-relative error of
# gradients, by the dtype of the tensor compared (float16 follows the reference verifiers'
# 2e-3, benchmarks/verify_mamba2_chunk.py:62-64).
OUT_TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}
GRAD_TOL = {torch.float32: 1e-4, torch.float16: 2e-3, torch.bfloat16: 2e-2}


def record(case, quantity, err, tol):
    """Print one measured parity error and return it; with MKO_PARITY_LOG set, also append
    it to that file as one JSON line, so a run leaves a table of every error it asserted."""
    print(f"[parity] {case} {quantity}: {err:.3e} (bar {tol:g})", flush=True)
    path = os.environ.get("MKO_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"case": case, "quantity": quantity, "err": float(err),
                                "bar": float(tol)}) + "\n")
    return err
