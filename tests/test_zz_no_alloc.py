"""mko_state_update_bwd_static (the decode backward with its partials in the library's
static scratch array) against mko_state_update_bwd (partials in a caller workspace).

Both run the same kernels on the same inputs, so every gradient must match bit for
bit.  Two calls in a row, the second smaller than the first, show that the array's
leftover contents from one call never leak into the next.  Every call goes through
the C ABI.
"""

import ctypes

import pytest
import torch

from cases import decode_problem

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _grads(entry, p, use_workspace, softplus=True):
    """Run one backward entry point; returns its float32 gradients by name."""
    from metal_kernelops import _native as nat
    from metal_kernelops.cv.mamba2_state import _params
    state, x, dt, A, B, C = (p[k] for k in ("state", "x", "dt", "A", "B", "C"))
    D, z, bias = p.get("D"), p.get("z"), p.get("dt_bias")
    f32 = dict(dtype=torch.float32, device=DEV)
    g = torch.Generator(device="cpu").manual_seed(21)
    dy = torch.randn(x.shape, generator=g).to(DEV)
    dnew = torch.randn(state.shape, generator=g).to(DEV)
    out = {"state": torch.empty(state.shape, **f32), "x": torch.empty(x.shape, **f32),
           "dt": torch.empty(dt.shape, **f32), "A": torch.empty(A.shape, **f32),
           "B": torch.empty(B.shape, **f32), "C": torch.empty(C.shape, **f32)}
    if D is not None:
        out["D"] = torch.empty(D.shape, **f32)
    if z is not None:
        out["z"] = torch.empty(z.shape, **f32)
    if bias is not None:
        out["dt_bias"] = torch.empty(bias.shape, **f32)
    prm = _params(state, x, dt, A, B, C, D, z, bias, softplus)
    prm.dy, prm.dnew_state = dy.data_ptr(), dnew.data_ptr()
    prm.grad_state, prm.dx, prm.ddt = out["state"].data_ptr(), out["x"].data_ptr(), out["dt"].data_ptr()
    prm.dA, prm.dB, prm.dC = out["A"].data_ptr(), out["B"].data_ptr(), out["C"].data_ptr()
    prm.dD = out["D"].data_ptr() if D is not None else None
    prm.dz = out["z"].data_ptr() if z is not None else None
    prm.ddt_bias = out["dt_bias"].data_ptr() if bias is not None else None
    lib = nat.lib()
    ws = None
    if use_workspace:
        ws = nat.workspace(lib.mko_state_update_bwd_workspace_size(ctypes.byref(prm)), state.device)
        prm.workspace, prm.workspace_bytes = ws.data_ptr(), ws.numel()
    status = getattr(lib, entry)(ctypes.byref(prm), nat.stream_of(state.device))
    nat.check(status, entry)
    torch.cuda.synchronize()
    return out


def _problem(shape, seed, **kw):
    p = decode_problem(*shape, seed=seed, **kw)
    return {k: v.to(DEV) for k, v in p.items()}


@pytest.mark.parametrize("second", [
    dict(shape=(3, 8, 16, 32, 2)),
    dict(shape=(2, 4, 8, 13, 1), dt_per_row=True),
], ids=["grouped", "dt-per-row-odd-dstate"])
def test_static_scratch_matches_workspace_twice(second):
    print(f"[no-alloc] first call (64, 80, 64, 128, 1), then {second}", flush=True)
    first = _problem((64, 80, 64, 128, 1), seed=31)
    small = _problem(second["shape"], seed=32, dt_per_row=second.get("dt_per_row", False))
    small["D"] = torch.randn(small["A"].shape[0], small["x"].shape[-1],
                             generator=torch.Generator().manual_seed(33)).to(DEV)  # per-row D
    for p in (first, small):
        ref = _grads("mko_state_update_bwd", p, use_workspace=True)
        got = _grads("mko_state_update_bwd_static", p, use_workspace=False)
        for name, want in ref.items():
            assert torch.equal(got[name], want), name
            assert torch.isfinite(want).all(), name


def test_static_scratch_rejects_a_problem_beyond_its_size():
    from metal_kernelops import _native as nat
    from metal_kernelops.cv.mamba2_state import _params
    p = _problem((4, 8, 16, 32, 2), seed=34)
    prm = _params(p["state"], p["x"], p["dt"], p["A"], p["B"], p["C"], None, None, None, False)
    prm.batch = 1 << 16  # sizes only: the call must refuse before it reads a pointer
    sink = torch.empty(1, device=DEV)
    prm.grad_state = prm.dx = prm.ddt = prm.dA = prm.dB = prm.dC = sink.data_ptr()
    lib = nat.lib()
    assert lib.mko_state_update_bwd_workspace_size(ctypes.byref(prm)) > nat.STATIC_SCRATCH_BYTES
    assert lib.mko_state_update_bwd_static(ctypes.byref(prm), nat.stream_of(p["state"].device)) == 4
    assert b"static scratch" in lib.mko_last_error()
