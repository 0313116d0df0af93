"""Mamba-2 decode state update: HIP kernels against the float64 CPU oracle.

Case list, contracts, adjoint-None checks and determinism follow the reference
verifier (benchmarks/verify_mamba2_state.py:552-570, 196-302).  Tolerances: the reference's
decode tolerances for fp32 and fp16 (1e-5, 5e-3); bf16 is held to 2e-2, tighter than the
reference's 3e-2, since the kernels' bf16 errors measure under 1e-2 on every case here.
"""

import pytest
import torch

import oracle
from cases import decode_problem, max_rel, norm_rel, record

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("state", "x", "dt", "A", "B", "C", "D", "z", "dt_bias")
TOL = {torch.float32: 1e-5, torch.float16: 5e-3, torch.bfloat16: 2e-2}


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
    ("dstate-640", torch.float32, (2, 4, 8, 640, 2), dict(softplus=True)),  # 16 states per lane
    ("dstate-24", torch.float32, (2, 4, 40, 24, 2), {}),  # two vectors per lane, 4 lanes per row
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
    fwd_bar = TOL[dtype] * max(scale, 1.0)
    record(f"decode {tag}", "y, new_state (max abs)", fwd_err, fwd_bar)
    assert fwd_err <= fwd_bar, f"{tag}: forward |err| {fwd_err:.3e}"
    for name, t, w in zip(NAMES, got, truth):
        if t is None:
            continue
        assert t.grad is not None and t.grad.dtype == dtype, name
        e = record(f"decode {tag}", "d" + name, norm_rel(t.grad, w.grad), TOL[dtype])
        assert e <= TOL[dtype], f"{tag}: grad {name} rel {e:.3e}"


C5 = (256, 80, 64, 128, 1)  # config 5: batch, nheads, headdim, dstate, ngroups


def _c5_ring(steps=8):
    """Per-step x, dt, B, C, z of config 5 from a seeded ring of 8 (the bench's draws)."""
    batch, nheads, headdim, dstate, _ = C5
    ring = []
    for i in range(steps):
        g = torch.Generator().manual_seed(100 + i)
        ring.append({"x": torch.randn(batch, nheads, headdim, generator=g).bfloat16(),
                     "dt": torch.randn(batch, nheads, generator=g),
                     "B": torch.randn(batch, 1, dstate, generator=g).bfloat16(),
                     "C": torch.randn(batch, 1, dstate, generator=g).bfloat16(),
                     "z": torch.randn(batch, nheads, headdim, generator=g).bfloat16()})
    return ring


def test_config5_full_batch_step():
    # Config 5 at full size (256 x 80 x 64 x 128 fp32 state, bf16 x/B/C/z): one step on
    # the GPU; batches are independent, so the oracle checks the first and last two.
    p = decode_problem(*C5, seed=0)
    ys, ss = _api()(*(p[k].to(DEV) for k in ("state", "x", "dt", "A", "B", "C")),
                    D=p["D"].to(DEV), z=p["z"].to(DEV), dt_bias=p["dt_bias"].to(DEV), dt_softplus=True)
    rows = torch.tensor([0, 1, 254, 255])
    sub = {k: (v[rows] if v.dim() >= 2 else v) for k, v in p.items()}
    wy, ws = oracle.mamba2_state_update(**sub, dt_softplus=True)
    e_y = record("c5 full step", "y", max_rel(ys[rows.to(DEV)], wy), 1e-5)
    e_s = record("c5 full step", "new_state", max_rel(ss[rows.to(DEV)], ws), 1e-5)
    assert e_y <= 1e-5 and e_s <= 1e-5
    assert torch.isfinite(ys).all() and torch.isfinite(ss).all()


def test_config5_1024_in_place_steps():
    # The workload the decode metric is quoted on: 1024 in-place steps (out_state=state)
    # at full size with per-step inputs from a seeded ring of 8.  The oracle steps two
    # batch rows through the same 1024 steps in float64.
    p = decode_problem(*C5, seed=0)
    ring = _c5_ring()
    ring_dev = [{k: v.to(DEV) for k, v in r.items()} for r in ring]
    A, D, bias = p["A"], p["D"], p["dt_bias"]
    state = p["state"].to(DEV)
    rows = torch.tensor([0, 255])
    ref_state = p["state"][rows].double()
    fn = _api()
    worst_y = 0.0
    for t in range(1024):
        r, rd = ring[t % 8], ring_dev[t % 8]
        y, out = fn(state, rd["x"], rd["dt"], A.to(DEV), rd["B"], rd["C"], D=D.to(DEV), z=rd["z"],
                    dt_bias=bias.to(DEV), dt_softplus=True, out_state=state)
        assert out.data_ptr() == state.data_ptr()
        wy, ref_state = oracle.mamba2_state_update(ref_state, r["x"][rows], r["dt"][rows], A, r["B"][rows],
                                                   r["C"][rows], D=D, z=r["z"][rows], dt_bias=bias,
                                                   dt_softplus=True)
        if t % 64 == 63:
            worst_y = max(worst_y, max_rel(y[rows.to(DEV)], wy))
    e_y = record("c5 1024 in-place steps", "y (every 64th step)", worst_y, 1e-5)
    e_s = record("c5 1024 in-place steps", "final state", max_rel(state[rows.to(DEV)], ref_state), 1e-5)
    assert e_y <= 1e-5 and e_s <= 1e-5
    assert torch.isfinite(state).all()


def test_config5_backward_batch_slice():
    # The decode backward at config-5 geometry, full batch on the GPU.  With the upstream
    # gradients zero outside batch rows 0 and 1, the parameter gradients (summed over the
    # batch) only see those rows, so the float64 oracle runs on them alone.
    p = decode_problem(*C5, seed=2)
    names = ("state", "x", "dt", "A", "B", "C", "D", "z", "dt_bias")
    g = torch.Generator().manual_seed(3)
    wy = torch.zeros(C5[0], C5[1], C5[2])
    ws = torch.zeros(C5[0], C5[1], C5[2], C5[3])
    wy[:2] = torch.randn(2, C5[1], C5[2], generator=g)
    ws[:2] = torch.randn(2, C5[1], C5[2], C5[3], generator=g)
    got = {k: p[k].to(DEV).requires_grad_(True) for k in names}
    y, s = _api()(*(got[k] for k in names[:6]), D=got["D"], z=got["z"], dt_bias=got["dt_bias"],
                  dt_softplus=True)
    ((y.float() * wy.to(DEV)).sum() + (s * ws.to(DEV)).sum()).backward()
    sub = {k: (p[k][:2] if k in ("state", "x", "dt", "B", "C", "z") else p[k]).double().requires_grad_(True)
           for k in names}
    ry, rs = oracle.mamba2_state_update(**sub, dt_softplus=True)
    ((ry * wy[:2].double()).sum() + (rs * ws[:2].double()).sum()).backward()
    for k in names:
        gk = got[k].grad
        if k in ("state", "x", "dt", "B", "C", "z"):
            assert torch.count_nonzero(gk[2:]) == 0, k
            gk = gk[:2]
        tol = TOL[got[k].dtype]
        e = record("c5 backward rows 0-1", "d" + k, norm_rel(gk, sub[k].grad), tol)
        assert e <= tol, f"d{k} {e:.3e}"


@pytest.mark.parametrize("x_dtype,z_dtype", [(torch.bfloat16, torch.float32),
                                             (torch.float32, torch.bfloat16),
                                             (torch.float16, torch.bfloat16)],
                         ids=["x-bf16-z-f32", "x-f32-z-bf16", "x-f16-z-bf16"])
def test_mixed_x_and_z_dtypes(x_dtype, z_dtype):
    # A float32 state with x and z of different dtypes: the reference casts both to the
    # state's dtype (exact here), so the oracle sees the rounded values in float64.
    p = decode_problem(3, 8, 16, 32, 2, seed=5, state_dtype=torch.float32)
    p["x"], p["z"] = p["x"].float().to(x_dtype), p["z"].float().to(z_dtype)
    names = ("state", "x", "dt", "A", "B", "C", "D", "z", "dt_bias")
    got = {k: p[k].to(DEV).requires_grad_(True) for k in names}
    y, s = _api()(*(got[k] for k in names[:6]), D=got["D"], z=got["z"], dt_bias=got["dt_bias"],
                  dt_softplus=True)
    g = torch.Generator().manual_seed(6)
    wy = torch.randn(y.shape, generator=g)
    ((y * wy.to(DEV)).sum() + s.square().sum()).backward()
    ref = {k: p[k].double().requires_grad_(True) for k in names}
    ry, rs = oracle.mamba2_state_update(**ref, dt_softplus=True)
    ((ry * wy.double()).sum() + rs.square().sum()).backward()
    case = f"mixed x {x_dtype} z {z_dtype}"
    assert y.dtype == torch.float32
    e = record(case, "y", max_rel(y, ry), 1e-5)
    assert e <= 1e-5
    for k in names:
        assert got[k].grad.dtype == got[k].dtype, k
        tol = TOL[got[k].dtype]
        e = record(case, "d" + k, norm_rel(got[k].grad, ref[k].grad), tol)
        assert e <= tol, f"d{k} {e:.3e}"


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
