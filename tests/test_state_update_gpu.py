"""Mamba-2 decode state update: HIP kernels against the float64 CPU oracle.

Case list, contracts, adjoint-None checks and determinism follow the reference
verifier (benchmarks/verify_mamba2_state.py:552-570, 196-302); tolerances are the
reference's decode tolerances: 1e-5 fp32, 5e-3 fp16, 3e-2 bf16.
"""

import pytest
import torch

import oracle
from cases import decode_problem, max_rel, norm_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("state", "x", "dt", "A", "B", "C", "D", "z", "dt_bias")
TOL = {torch.float32: 1e-5, torch.float16: 5e-3, torch.bfloat16: 3e-2}


def _api():
    from metal_kernelops.cv import mamba2_state_update
    return mamba2_state_update


def build(batch, nheads, dim, dstate, groups, dt_per_head=False, d_kind="head", use_z=True,
          use_bias=True, dtype=torch.float32, state_scale=1.0, seed=7):
    g = torch.Generator().manual_seed(seed)
    inputs = [
        torch.randn(batch, nheads, dim, dstate, generator=g) * state_scale,
        torch.randn(batch, nheads, dim, generator=g),
        (torch.rand(batch, nheads, dim, generator=g) if dt_per_head
         else torch.rand(batch, nheads, generator=g)) * 0.2,
        -torch.rand(nheads, generator=g) - 0.05,
        torch.randn(batch, groups, dstate, generator=g),
        torch.randn(batch, groups, dstate, generator=g),
        {"none": None, "head": torch.randn(nheads, generator=g),
         "head_dim": torch.randn(nheads, dim, generator=g)}[d_kind],
        torch.randn(batch, nheads, dim, generator=g) if use_z else None,
        torch.randn(nheads, generator=g) * 0.1 if use_bias else None,
    ]
    return [None if t is None else t.to(dtype) for t in inputs]


CASES = [
    ("decode-f32", torch.float32, (1, 16, 128, 128, 1), dict(softplus=True)),
    ("decode-batched", torch.float32, (4, 8, 64, 64, 2), {}),
    ("zero-state", torch.float32, (2, 4, 32, 64, 1), dict(state_scale=0.0)),
    ("carried-state", torch.float32, (3, 8, 16, 64, 2), {}),
    ("gqa-4", torch.float32, (2, 16, 32, 64, 4), {}),
    ("mha", torch.float32, (2, 6, 8, 16, 6), {}),
    ("dt-per-head", torch.float32, (2, 4, 16, 32, 2), {}),
    ("dt-per-element", torch.float32, (2, 4, 16, 32, 2), dict(dt_per_head=True)),
    ("head-dim-D", torch.float32, (2, 4, 16, 32, 2), dict(d_kind="head_dim")),
    ("no-D", torch.float32, (2, 4, 16, 32, 2), dict(d_kind="none")),
    ("no-gate", torch.float32, (2, 4, 16, 32, 2), dict(use_z=False)),
    ("bias-softplus", torch.float32, (2, 4, 16, 32, 2), dict(softplus=True)),
    ("softplus-no-bias", torch.float32, (2, 4, 16, 32, 2), dict(use_bias=False, softplus=True)),
    ("dstate-1", torch.float32, (2, 4, 8, 1, 1), {}),
    ("dstate-odd", torch.float32, (2, 4, 8, 13, 2), dict(softplus=True)),
    ("f16", torch.float16, (2, 4, 16, 32, 2), {}),
    ("bf16", torch.bfloat16, (2, 4, 16, 32, 2), {}),
    ("bf16-decode", torch.bfloat16, (1, 16, 128, 128, 1), {}),
]


@pytest.mark.parametrize("tag,dtype,shape,opts", CASES, ids=[c[0] for c in CASES])
def test_case(tag, dtype, shape, opts):
    opts = dict(opts)
    softplus = opts.pop("softplus", False)
    inputs = build(*shape, dtype=dtype, **opts)
    g = torch.Generator().manual_seed(1)
    wy = torch.randn(shape[0], shape[1], shape[2], generator=g, dtype=torch.float64) * 0.5
    ws = torch.randn(shape[0], shape[1], shape[2], shape[3], generator=g, dtype=torch.float64) * 0.5

    truth = [None if t is None else t.double().requires_grad_(True) for t in inputs]
    want_y, want_s = oracle.mamba2_state_update(*truth, dt_softplus=softplus)
    ((want_y * wy).sum() + (want_s * ws).sum()).backward()

    got = [None if t is None else t.to(DEV).requires_grad_(True) for t in inputs]
    y, s = _api()(*got, dt_softplus=softplus)
    ((y * wy.to(DEV, dtype)).sum() + (s * ws.to(DEV, dtype)).sum()).backward()
    torch.cuda.synchronize()

    assert y.dtype == dtype and s.dtype == dtype
    fwd_err = max((y.detach().double().cpu() - want_y.detach()).abs().max().item(),
                  (s.detach().double().cpu() - want_s.detach()).abs().max().item())
    scale = max(want_y.abs().max().item(), want_s.abs().max().item())
    assert fwd_err <= TOL[dtype] * max(scale, 1.0), f"{tag}: forward |err| {fwd_err:.3e}"
    for name, t, w in zip(NAMES, got, truth):
        if t is None:
            continue
        assert t.grad is not None and t.grad.dtype == dtype, name
        e = norm_rel(t.grad, w.grad)
        assert e <= TOL[dtype], f"{tag}: grad {name} rel {e:.3e}"


def test_config5_shape_batch_subset():
    # Config 5 geometry (nheads 80, headdim 64, dstate 128, fp32 state, bf16 x/B/C/z);
    # rows of different batches are independent, so a batch slice checks exactly.
    p = decode_problem(16, 80, 64, 128, 1, seed=0)
    ys, ss = _api()(*(p[k].to(DEV) for k in ("state", "x", "dt", "A", "B", "C")),
                    D=p["D"].to(DEV), z=p["z"].to(DEV), dt_bias=p["dt_bias"].to(DEV), dt_softplus=True)
    wy, ws = oracle.mamba2_state_update(**p, dt_softplus=True)
    assert max_rel(ys, wy) <= 1e-5
    assert max_rel(ss, ws) <= 1e-5


def test_in_place_decode_loop_matches_recurrence():
    p = decode_problem(4, 8, 16, 32, 2, seed=3)
    g = torch.Generator().manual_seed(4)
    steps = 24
    xs = torch.randn(steps, 4, 8, 16, generator=g).bfloat16()
    dts = torch.randn(steps, 4, 8, generator=g)
    Bs = torch.randn(steps, 4, 2, 32, generator=g).bfloat16()
    Cs = torch.randn(steps, 4, 2, 32, generator=g).bfloat16()
    state = p["state"].to(DEV).clone()
    ref_state = p["state"].double()
    fn = _api()
    for t in range(steps):
        y, out = fn(state, xs[t].to(DEV), dts[t].to(DEV), p["A"].to(DEV), Bs[t].to(DEV), Cs[t].to(DEV),
                    D=p["D"].to(DEV), dt_bias=p["dt_bias"].to(DEV), dt_softplus=True, out_state=state)
        assert out.data_ptr() == state.data_ptr()
        wy, ref_state = oracle.mamba2_state_update(ref_state, xs[t], dts[t], p["A"], Bs[t], Cs[t],
                                                   D=p["D"], dt_bias=p["dt_bias"], dt_softplus=True)
        assert max_rel(y, wy) <= 1e-5
    assert max_rel(state, ref_state) <= 1e-5


def test_contracts_and_errors():
    fn = _api()
    inputs = build(2, 4, 6, 16, 2)
    state, x, dt, A, B, C, D, z, bias = [t.to(DEV) for t in inputs]
    kept = state.clone()
    y, new_state = fn(state, x, dt, A, B, C, D, z, bias)
    torch.cuda.synchronize()
    assert torch.equal(state, kept)
    assert new_state.data_ptr() != state.data_ptr()
    out = torch.empty_like(state)
    _, staged = fn(state, x, dt, A, B, C, D, z, bias, out_state=out)
    assert torch.equal(out, new_state)
    assert staged.untyped_storage().data_ptr() == out.untyped_storage().data_ptr()
    assert torch.equal(state, kept)
    buffer = state.clone()
    _, updated = fn(buffer, x, dt, A, B, C, D, z, bias, out_state=buffer)
    assert torch.equal(buffer, new_state)
    assert updated.untyped_storage().data_ptr() == buffer.untyped_storage().data_ptr()

    bad_B = torch.randn(2, 3, 16, device=DEV)
    errors = [
        lambda: fn(*(t.cpu() for t in (state, x, dt, A, B, C))),
        lambda: fn(state, x, dt, A, bad_B, bad_B.clone()),
        lambda: fn(state, x, dt, A, B, C, out_state=torch.empty_like(y)),
        lambda: fn(state.int(), x.int(), dt.int(), A, B.int(), C.int()),
        lambda: fn(state, x, dt, A, B, C, out_state=torch.empty_like(state).requires_grad_(True)),
    ]
    for call in errors:
        with pytest.raises(ValueError):
            call()

    wide_x = torch.randn(2, 4, 12, device=DEV)
    wide_z = torch.randn(2, 4, 12, device=DEV)
    y1, s1 = fn(state, wide_x[:, :, ::2], dt, A, B, C, D, wide_z[:, :, ::2], bias)
    y2, s2 = fn(state, wide_x[:, :, ::2].contiguous(), dt, A, B, C, D, wide_z[:, :, ::2].contiguous(), bias)
    assert torch.equal(y1, y2) and torch.equal(s1, s2)


@pytest.mark.parametrize("use_y,use_state", [(True, False), (False, True)])
def test_adjoint_none(use_y, use_state):
    inputs = build(2, 4, 6, 16, 2)
    g = torch.Generator().manual_seed(5)
    wy = torch.randn(2, 4, 6, generator=g, dtype=torch.float64)
    ws = torch.randn(2, 4, 6, 16, generator=g, dtype=torch.float64)

    def loss(y, s):
        total = 0
        if use_y:
            total = total + (y * wy.to(y.device, y.dtype)).sum()
        if use_state:
            total = total + (s * ws.to(s.device, s.dtype)).sum()
        return total

    truth = [t.double().requires_grad_(True) for t in inputs]
    loss(*oracle.mamba2_state_update(*truth)).backward()
    got = [t.to(DEV).requires_grad_(True) for t in inputs]
    loss(*_api()(*got)).backward()
    for name, t, w in zip(NAMES, got, truth):
        if w.grad is None:
            continue
        assert norm_rel(t.grad, w.grad) <= 1e-5, name


@pytest.mark.parametrize("shape", [(4, 8, 64, 64, 2), (1, 16, 128, 128, 1)])
def test_backward_is_deterministic(shape):
    inputs = build(*shape)
    wy = torch.randn(*shape[:3], device=DEV)
    ws = torch.randn(*shape[:4], device=DEV)
    got = [t.to(DEV).requires_grad_(True) for t in inputs]
    runs = []
    for _ in range(3):
        for t in got:
            t.grad = None
        y, s = _api()(*got)
        ((y * wy).sum() + (s * ws).sum()).backward()
        runs.append([t.grad.clone() for t in got])
    for name, vals in zip(NAMES, zip(*runs)):
        assert all(torch.equal(vals[0], v) for v in vals[1:]), name
        assert vals[0].abs().max().item() > 0, name
