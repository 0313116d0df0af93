"""The package's exported pure-torch twins against the pinned float64 oracle (CPU only).

``scan_reference`` / ``reference.selective_scan`` restate the reference's
``reference.py:5-49`` and ``scan.py:326-329``; ``mamba2_state_update_reference``
restates ``cv/mamba2_state.py:822-849``; ``mamba2_chunk_scan_reference`` restates
``cv/mamba2_chunk.py:681-723``.  They are API a caller can run on any device, so
each is checked here against the oracle function that the oracle tests pin
independently (the literal Mamba-1 loop, the decode closed form, the per-token SSD
recurrence), in float64 to round-off and in float32 / bfloat16 to those dtypes' bars.
"""

import pytest
import torch

import oracle
from cases import decode_problem, mamba1_c1, max_rel, norm_rel, ssd_problem
from metal_kernelops import reference, scan_reference
from metal_kernelops.cv import mamba2_chunk_scan_reference, mamba2_state_update_reference

F64 = torch.float64


def _mamba1_bare(seed=0, groups=2):
    inputs, _ = mamba1_c1(seed)
    args = {k: inputs[k] for k in ("u", "dt", "A", "B", "C")}
    args["dt"] = torch.nn.functional.softplus(args["dt"] + inputs["delta_bias"][:, None])
    if groups != 2:
        args["B"], args["C"] = args["B"][:, :groups].contiguous(), args["C"][:, :groups].contiguous()
    return args


@pytest.mark.parametrize("groups", [1, 2])
def test_scan_reference_matches_literal_loop(groups):
    args = _mamba1_bare(groups=groups)
    want = oracle.selective_scan_loop(*(args[k] for k in ("u", "dt", "A", "B", "C")))
    got64 = scan_reference(*(args[k].double() for k in ("u", "dt", "A", "B", "C")))
    assert got64.dtype == F64
    assert max_rel(got64, want) <= 1e-12
    got32 = reference.selective_scan(*(args[k] for k in ("u", "dt", "A", "B", "C")))
    assert got32.dtype == torch.float32
    assert max_rel(got32, want) <= 1e-5


def test_scan_reference_gradients_match_oracle():
    args = _mamba1_bare()
    names = ("u", "dt", "A", "B", "C")
    dy = torch.randn(args["u"].shape, generator=torch.Generator().manual_seed(4), dtype=F64)
    mine = {k: args[k].double().requires_grad_(True) for k in names}
    (scan_reference(*(mine[k] for k in names)) * dy).sum().backward()
    theirs = {k: args[k].double().requires_grad_(True) for k in names}
    (oracle.selective_scan(*(theirs[k] for k in names)) * dy).sum().backward()
    for k in names:
        assert norm_rel(mine[k].grad, theirs[k].grad) <= 1e-12, k


def test_scan_reference_contracts():
    args = _mamba1_bare()
    u = args["u"][:, :, :0]
    out = scan_reference(u, args["dt"][:, :, :0], args["A"], args["B"][..., :0], args["C"][..., :0])
    assert out.shape == (2, 8, 0)
    with pytest.raises(ValueError):
        scan_reference(args["u"], args["dt"], args["A"], args["B"][:, :1].repeat(1, 3, 1, 1),
                       args["C"][:, :1].repeat(1, 3, 1, 1))
    # bf16 inputs: computed in the inputs' dtype, returned in u's
    got = scan_reference(*(args[k].bfloat16() for k in ("u", "dt", "A", "B", "C")))
    assert got.dtype == torch.bfloat16
    want = oracle.selective_scan_loop(*(args[k].bfloat16() for k in ("u", "dt", "A", "B", "C")))
    assert max_rel(got, want) <= 5e-2


DECODE_CASES = [
    dict(),
    dict(dt_per_row=True),
    dict(d_row=True),
    dict(no_z=True, no_bias=True),
    dict(softplus=False),
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=lambda c: "-".join(c) or "default")
def test_state_update_reference_matches_oracle(case):
    p = decode_problem(3, 8, 6, 16, 2, seed=8, act=torch.float32, dt_per_row=case.get("dt_per_row", False))
    if case.get("d_row"):
        p["D"] = torch.randn(8, 6, generator=torch.Generator().manual_seed(9))
    if case.get("no_z"):
        p["z"] = None
    if case.get("no_bias"):
        p["dt_bias"] = None
    softplus = case.get("softplus", True)
    if not softplus:
        p["dt"] = p["dt"].abs() * 0.3
    kept = p["state"].clone()
    wy, ws = oracle.mamba2_state_update(**p, dt_softplus=softplus)
    y64, s64 = mamba2_state_update_reference(**{k: (None if v is None else v.double()) for k, v in p.items()},
                                             dt_softplus=softplus)
    assert max_rel(y64, wy) <= 1e-12 and max_rel(s64, ws) <= 1e-12
    y32, s32 = mamba2_state_update_reference(**p, dt_softplus=softplus)
    assert torch.equal(p["state"], kept)
    assert y32.dtype == torch.float32 and s32.dtype == torch.float32
    assert max_rel(y32, wy) <= 1e-5 and max_rel(s32, ws) <= 1e-5


def test_state_update_reference_gradients_match_oracle():
    p = decode_problem(2, 4, 6, 8, 2, seed=10, act=torch.float32)
    names = tuple(p)
    g = torch.Generator().manual_seed(11)
    wy = torch.randn(2, 4, 6, generator=g, dtype=F64)
    ws = torch.randn(2, 4, 6, 8, generator=g, dtype=F64)
    mine = {k: p[k].double().requires_grad_(True) for k in names}
    y, s = mamba2_state_update_reference(**mine, dt_softplus=True)
    ((y * wy).sum() + (s * ws).sum()).backward()
    theirs = {k: p[k].double().requires_grad_(True) for k in names}
    y, s = oracle.mamba2_state_update(**theirs, dt_softplus=True)
    ((y * wy).sum() + (s * ws).sum()).backward()
    for k in names:
        assert norm_rel(mine[k].grad, theirs[k].grad) <= 1e-12, k


def test_chunk_scan_reference_matches_recurrence():
    p = ssd_problem(2, 37, 4, 6, 2, 5, seed=12)
    names = ("x", "dt", "A", "B", "C")
    opts = {k: p[k] for k in ("D", "z", "dt_bias", "initial_states")}
    wy, ws = oracle.mamba2_chunk_scan_recurrence(*(p[k] for k in names), **opts, dt_softplus=True)
    y, s = mamba2_chunk_scan_reference(*(p[k].double() for k in names), chunk_size=8,
                                       **{k: v.double() for k, v in opts.items()}, dt_softplus=True)
    assert max_rel(y, wy) <= 1e-12 and max_rel(s, ws) <= 1e-12
