"""Gated RMSNorm: oracle pins on the CPU, HIP parity on the GPU.

Cases follow the reference's verifier (``benchmarks/verify_gated_norm.py``): the
forward grid of shapes, groups, bias, gate and eps (:78-117), the gradient grid
(:119-166), central differences of the kernel's own forward (:169-220), non-contiguous
and empty inputs, narrow and wide feature axes around the register cut-offs
(:255-343), a float32 weight on float16 activations (:345-371) and an Adam step
(:374-397).  Tolerances are the verifier's (:52-53): forward max-abs error float32
2e-5, float16 5e-3, bfloat16 4e-2 (plus the output dtype's own rounding, half an ulp
of the value); gradients, relative error of the global norm, float32 1e-6, float16
2e-3, bfloat16 2e-2.
"""

import pytest
import torch
import torch.nn.functional as F

import oracle

DEV = "cuda"
FWD_TOL = {torch.float32: 2e-5, torch.float16: 5e-3, torch.bfloat16: 4e-2}
GRAD_TOL = {torch.float32: 1e-6, torch.float16: 2e-3, torch.bfloat16: 2e-2}
HALF_ULP = {torch.float32: 2.0 ** -24, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def make(shape, seed, scale=1.0, dtype=torch.float64):
    return (torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64) * scale).to(dtype)


def rel(actual, expected):
    a, e = actual.detach().double().cpu(), expected.detach().double().cpu()
    d = e.norm().item()
    return (a - e).norm().item() / d if d else (a - e).norm().item()


def fwd_error(out, ref64):
    """Max-abs error beyond the output dtype's rounding of the float64 value."""
    a, e = out.detach().double().cpu(), ref64.detach().double().cpu()
    return ((a - e).abs() - HALF_ULP[out.dtype] * e.abs()).max().item()


# --------------------------------------------------------------------------- CPU: oracle pins


@pytest.mark.parametrize("group", [None, 4, 16])
def test_oracle_equals_library_rms_norm(group):
    """Without z and bias the oracle is torch's rms_norm over each group, then the weight."""
    x, w = make((5, 3, 32), 1), make((32,), 2)
    out, rstd = oracle.rmsnorm_gated(x, w, eps=1e-5, group_size=group)
    g = 32 if group is None else group
    want = F.rms_norm(x.reshape(5, 3, 32 // g, g), (g,), eps=1e-5).reshape(5, 3, 32) * w
    assert (out - want).abs().max() < 1e-12
    assert rstd.shape == (5, 3, 32 // g)


def test_oracle_gate_special_cases():
    x, w, b, z = make((6, 24), 3), make((24,), 4), make((24,), 5), make((6, 24), 6)
    plain, _ = oracle.rmsnorm_gated(x, w, b, eps=0.0, group_size=8)
    # a gate before the norm that is a positive constant cancels when eps = 0:
    # silu(40) is 40 in float64 and rms_norm(40 x) = rms_norm(x)
    const, _ = oracle.rmsnorm_gated(x, w, b, torch.full_like(x, 40.0), eps=0.0, group_size=8, norm_before_gate=False)
    assert (const - plain).abs().max() < 1e-12
    # the gate after the norm multiplies the shifted output by torch's silu(z)
    after, _ = oracle.rmsnorm_gated(x, w, b, z, eps=0.0, group_size=8, norm_before_gate=True)
    assert (after - plain * F.silu(z)).abs().max() < 1e-12


@pytest.mark.parametrize("gate", ["none", "before", "after"])
@pytest.mark.parametrize("group", [None, 6])
def test_oracle_backward_equals_autograd(gate, group):
    """The analytic backward equals torch autograd through the forward composition."""
    x = make((4, 3, 18), 7).requires_grad_(True)
    w, b = make((18,), 8).requires_grad_(True), make((18,), 9).requires_grad_(True)
    z = make((4, 3, 18), 10).requires_grad_(True) if gate != "none" else None
    dy = make((4, 3, 18), 11)
    out, _ = oracle.rmsnorm_gated(x, w, b, z, eps=1e-3, group_size=group, norm_before_gate=gate != "before")
    leaves = [t for t in (x, w, b, z) if t is not None]
    want = torch.autograd.grad((out * dy).sum(), leaves)
    dx, dw, db, dz = oracle.rmsnorm_gated_bwd(dy, x.detach(), w.detach(), b.detach(),
                                              None if z is None else z.detach(), eps=1e-3, group_size=group,
                                              norm_before_gate=gate != "before")
    got = [dx, dw, db] + ([dz] if z is not None else [])
    for g_, w_ in zip(got, want):
        assert (g_ - w_).abs().max() < 1e-12


@pytest.mark.parametrize("before", [False, True])
def test_oracle_backward_equals_central_differences(before):
    """The analytic dx and dz against central differences of sum(out * dy) in float64."""
    x, w, b, z, dy = make((2, 12), 12), make((12,), 13), make((12,), 14), make((2, 12), 15), make((2, 12), 16)
    dx, _, _, dz = oracle.rmsnorm_gated_bwd(dy, x, w, b, z, eps=1e-4, group_size=4, norm_before_gate=not before)

    def loss(xx, zz):
        return (oracle.rmsnorm_gated(xx, w, b, zz, eps=1e-4, group_size=4, norm_before_gate=not before)[0] * dy).sum()

    h = 1e-6
    for i in range(0, 24, 5):
        e = torch.zeros(24, dtype=torch.float64)
        e[i] = h
        e = e.reshape(2, 12)
        nx = (loss(x + e, z) - loss(x - e, z)) / (2 * h)
        nz = (loss(x, z + e) - loss(x, z - e)) / (2 * h)
        assert abs(nx - dx.reshape(-1)[i]) < 1e-7 * max(1.0, abs(nx))
        assert abs(nz - dz.reshape(-1)[i]) < 1e-7 * max(1.0, abs(nz))


def test_reference_twin_matches_oracle():
    from metal_kernelops.cv import rmsnorm_gated_reference
    x, w, b, z = make((7, 40), 17, dtype=torch.float32), make((40,), 18), make((40,), 19), make((7, 40), 20)
    for before in (False, True):
        got = rmsnorm_gated_reference(x, w, b, z, eps=1e-5, group_size=10, norm_before_gate=before)
        want, _ = oracle.rmsnorm_gated(x, w, b, z, eps=1e-5, group_size=10, norm_before_gate=before)
        assert got.dtype == torch.float32 and got.device.type == "cpu"
        assert (got.double() - want).abs().max() < 1e-6


def test_errors_on_the_host():
    from metal_kernelops.cv import rmsnorm_gated
    x, w = torch.randn(4, 300), torch.ones(300)
    with pytest.raises(ValueError, match="groups of"):
        rmsnorm_gated(x, w, group_size=7)
    with pytest.raises(ValueError, match="weight"):
        rmsnorm_gated(x, torch.ones(299))
    with pytest.raises(ValueError, match="z should have shape"):
        rmsnorm_gated(x, w, z=torch.randn(4, 299))
    with pytest.raises(ValueError, match="feature axis"):
        rmsnorm_gated(torch.randn(()), w)
    with pytest.raises(ValueError, match="ROCm GPU"):
        rmsnorm_gated(x, w)
    # an empty feature axis returns a copy before any device check, as in the reference
    empty = torch.randn(5, 0)
    out = rmsnorm_gated(empty, torch.ones(0))
    assert out.shape == (5, 0) and out.dtype == empty.dtype


# --------------------------------------------------------------------------- GPU: HIP parity

# shape, group_size, bias, gate, norm_before_gate, eps (the verifier's forward grid)
FWD_CASES = [
    ((512, 300), None, True, True, True, 1e-5),
    ((512, 300), 60, True, True, True, 1e-5),
    ((512, 300), 100, True, True, True, 1e-6),
    ((512, 300), 150, True, True, False, 1e-5),
    ((512, 300), None, False, True, True, 1e-5),
    ((512, 300), None, True, False, True, 1e-5),
    ((512, 300), 60, True, True, False, 1e-5),
    ((512, 300), None, True, True, True, 1.0),
    ((4, 8, 300), 100, True, True, True, 1e-5),
    ((3, 5, 7, 128), 32, True, True, True, 1e-5),
    ((1, 64), 16, True, True, False, 1e-5),
    ((7, 4096), 1024, True, True, True, 1e-5),
    ((2, 3, 8192), None, True, True, True, 1e-5),
    ((64, 16384), 4096, True, True, True, 1e-5),
    ((16, 32768), None, True, True, True, 1e-5),
    ((8, 40000), 20000, True, True, False, 1e-5),
    # this build's own path boundaries: a streamed forward group, an unaligned wide one
    ((4, 65536), None, True, True, False, 1e-5),
    ((3, 4100), None, True, True, True, 1e-5),
    ((300, 2560), None, True, True, True, 1e-5),
]


def _fid(c):
    shape, group, bias, gate, before, eps = c
    return f"{'x'.join(map(str, shape))}-g{group}-b{int(bias)}-z{int(gate)}-{'before' if before else 'after'}-eps{eps}"


def _inputs(shape, bias, gate, dtype, seed):
    x = make(shape, seed, 1.0, dtype)
    w = make(shape[-1:], seed + 1, 1.0, dtype)
    b = make(shape[-1:], seed + 2, 1.0, dtype) if bias else None
    z = make(shape, seed + 3, 1.0, dtype) if gate else None
    return x, w, b, z


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", FWD_CASES, ids=_fid)
def test_forward(case, dtype):
    from metal_kernelops.cv import rmsnorm_gated
    shape, group, bias, gate, before, eps = case
    x, w, b, z = _inputs(shape, bias, gate, dtype, seed=len(shape) + shape[-1])
    dev = [t.to(DEV) if t is not None else None for t in (x, w, b, z)]
    with torch.no_grad():
        out = rmsnorm_gated(*dev, eps=eps, group_size=group, norm_before_gate=before)
    torch.cuda.synchronize()
    want, _ = oracle.rmsnorm_gated(x, w, b, z, eps=eps, group_size=group, norm_before_gate=before)
    assert out.dtype == dtype and out.shape == x.shape and out.device.type == "cuda"
    err = fwd_error(out, want)
    assert err <= FWD_TOL[dtype], err


# shape, group_size, bias, gate, norm_before_gate (the verifier's gradient grid)
GRAD_CASES = [
    ((256, 300), None, True, True, True),
    ((256, 300), 60, True, True, True),
    ((256, 300), 100, True, True, False),
    ((256, 300), None, False, True, True),
    ((256, 300), None, True, False, True),
    ((4, 6, 128), 32, True, True, False),
    ((8, 4096), 1024, True, True, True),
    ((16, 32768), None, True, True, True),
    ((8, 40000), 20000, True, True, False),
    # the backward's own boundaries: the widest register group, the first streamed
    # one, an unaligned wide one, many row blocks
    ((64, 8192), None, True, True, False),
    ((16, 8200), None, True, True, True),
    ((5, 4100), None, True, True, True),
    ((4096, 768), None, True, True, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("case", GRAD_CASES, ids=lambda c: _fid(c + (1e-5,)))
def test_gradients(case, dtype):
    from metal_kernelops.cv import rmsnorm_gated
    shape, group, bias, gate, before = case
    x, w, b, z = _inputs(shape, bias, gate, dtype, seed=100 + shape[-1])
    dy = make(shape, 7, 1.0, dtype)
    leaves = [t.to(DEV).requires_grad_(True) if t is not None else None for t in (x, w, b, z)]
    out = rmsnorm_gated(*leaves, group_size=group, norm_before_gate=before)
    out.backward(dy.to(DEV))
    torch.cuda.synchronize()
    dx, dw, db, dz = oracle.rmsnorm_gated_bwd(dy, x, w, b, z, eps=1e-5, group_size=group, norm_before_gate=before)
    for name, leaf, want in (("x", leaves[0], dx), ("weight", leaves[1], dw), ("bias", leaves[2], db),
                             ("z", leaves[3], dz)):
        if leaf is None:
            continue
        assert leaf.grad is not None and leaf.grad.dtype == dtype, name
        assert rel(leaf.grad, want) <= GRAD_TOL[dtype], (name, rel(leaf.grad, want))


@pytest.mark.gpu
def test_bench_shape_full_size():
    """The bench's shape at full size (8192 x 2560 bf16, z and bias, gate after the norm, as
    ``benchmarks/verify_gated_norm.py:518-555`` times it): every row of the output and of dx,
    dz, and the weight and bias gradients summed over all 8192 rows."""
    from metal_kernelops.cv import rmsnorm_gated
    shape = (8192, 2560)
    x, w, b, z = _inputs(shape, True, True, torch.bfloat16, seed=500)
    dy = make(shape, 501, 1.0, torch.bfloat16)
    leaves = [t.to(DEV).requires_grad_(True) for t in (x, w, b, z)]
    out = rmsnorm_gated(*leaves, norm_before_gate=True)
    out.backward(dy.to(DEV))
    torch.cuda.synchronize()
    want, _ = oracle.rmsnorm_gated(x, w, b, z, norm_before_gate=True)
    assert fwd_error(out, want) <= FWD_TOL[torch.bfloat16]
    dx, dw, db, dz = oracle.rmsnorm_gated_bwd(dy, x, w, b, z, eps=1e-5, norm_before_gate=True)
    for name, leaf, ref in (("x", leaves[0], dx), ("weight", leaves[1], dw), ("bias", leaves[2], db),
                            ("z", leaves[3], dz)):
        assert rel(leaf.grad, ref) <= GRAD_TOL[torch.bfloat16], (name, rel(leaf.grad, ref))


@pytest.mark.gpu
@pytest.mark.parametrize("shape,group,before", [((4, 300), 100, True), ((4, 128), 32, False)])
def test_central_differences_of_the_kernel(shape, group, before):
    """The kernels' analytic dx and dz against central differences of their own forward."""
    from metal_kernelops.cv import rmsnorm_gated
    x, w, b, z, dy = (make(s, 11 + i, 1.0, torch.float32).to(DEV)
                      for i, s in enumerate((shape, shape[-1:], shape[-1:], shape, shape)))

    def objective(xx, zz):
        return (rmsnorm_gated(xx, w, b, zz, group_size=group, norm_before_gate=before) * dy).sum()

    xg, zg = x.clone().requires_grad_(True), z.clone().requires_grad_(True)
    objective(xg, zg).backward()
    step = 1e-2
    for pos in torch.randperm(x.numel(), generator=torch.Generator().manual_seed(3))[:12].tolist():
        for base, grad, is_x in ((x, xg.grad, True), (z, zg.grad, False)):
            plus, minus = base.flatten().clone(), base.flatten().clone()
            plus[pos] += step
            minus[pos] -= step
            args_p = (plus.view(shape), z) if is_x else (x, plus.view(shape))
            args_m = (minus.view(shape), z) if is_x else (x, minus.view(shape))
            numeric = float((objective(*args_p) - objective(*args_m)) / (2 * step))
            exact = float(grad.flatten()[pos])
            assert abs(numeric - exact) / max(abs(numeric), abs(exact), 1e-2) < 2e-2


@pytest.mark.gpu
def test_non_contiguous_inputs():
    from metal_kernelops.cv import rmsnorm_gated
    base = torch.randn(64, 129, device=DEV)
    for x in (base.t(), torch.randn(64, 258, device=DEV)[:, ::2]):
        assert not x.is_contiguous()
        w = torch.randn(x.shape[-1], device=DEV)
        with torch.no_grad():
            out = rmsnorm_gated(x, w)
        want, _ = oracle.rmsnorm_gated(x.cpu(), w.cpu())
        assert fwd_error(out, want) < 2e-5
        xg, wg = x.detach().clone().requires_grad_(True), w.detach().clone().requires_grad_(True)
        dy = torch.randn(x.shape, device=DEV)
        gx, gw = torch.autograd.grad((rmsnorm_gated(xg, wg) * dy).sum(), (xg, wg))
        dx, dw, _, _ = oracle.rmsnorm_gated_bwd(dy.cpu(), x.cpu(), w.cpu())
        assert rel(gx, dx) < 1e-6 and rel(gw, dw) < 1e-6


@pytest.mark.gpu
def test_empty_and_narrow_inputs():
    from metal_kernelops.cv import rmsnorm_gated
    for shape in ((0, 300), (5, 0), (0,), (2, 0, 7)):
        x = torch.empty(*shape, device=DEV)
        out = rmsnorm_gated(x, torch.empty(shape[-1] if shape else 0, device=DEV))
        assert out.shape == x.shape and out.numel() == 0 and out.dtype == x.dtype
    leaf = torch.empty(0, 300, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    w = torch.ones(300, device=DEV, requires_grad=True)
    out = rmsnorm_gated(leaf, w)
    assert out.dtype == torch.bfloat16
    out.sum().backward()
    assert leaf.grad.shape == (0, 300) and torch.equal(w.grad, torch.zeros_like(w))
    for features in (1, 2, 31, 33):
        x, w = torch.randn(4, features, device=DEV), torch.randn(features, device=DEV)
        with torch.no_grad():
            out = rmsnorm_gated(x, w)
        want, _ = oracle.rmsnorm_gated(x.cpu(), w.cpu())
        assert fwd_error(out, want) < 2e-5, features


@pytest.mark.gpu
def test_mixed_weight_and_gate_dtypes():
    """A float32 weight on float16 activations, and a gate of another dtype than x."""
    from metal_kernelops.cv import rmsnorm_gated
    x = make((64, 512), 30, 1.0, torch.float16)
    w, b = make((512,), 31, 1.0, torch.float32), make((512,), 32, 1.0, torch.float32)
    z = make((64, 512), 33, 1.0, torch.float16)
    leaves = [t.to(DEV).requires_grad_(True) for t in (x, w, b, z)]
    out = rmsnorm_gated(*leaves)
    out.sum().backward()
    want, _ = oracle.rmsnorm_gated(x, w, b, z)
    assert fwd_error(out, want) < 5e-3
    assert [t.grad.dtype for t in leaves] == [torch.float16, torch.float32, torch.float32, torch.float16]
    _, dw, _, _ = oracle.rmsnorm_gated_bwd(torch.ones(64, 512, dtype=torch.float64), x, w, b, z)
    assert rel(leaves[1].grad, dw) < 2e-3
    # a float32 gate on bfloat16 activations: the kernel runs both in float32
    xb = make((16, 256), 34, 1.0, torch.bfloat16)
    zf = make((16, 256), 35, 1.0, torch.float32)
    wb = make((256,), 36, 1.0, torch.bfloat16)
    with torch.no_grad():
        outb = rmsnorm_gated(xb.to(DEV), wb.to(DEV), z=zf.to(DEV), norm_before_gate=False)
    wantb, _ = oracle.rmsnorm_gated(xb, wb, None, zf, norm_before_gate=False)
    assert outb.dtype == torch.bfloat16 and fwd_error(outb, wantb) < 4e-2
    # bfloat16 parameters on float32 activations (read as 4-element, 8-byte vectors), and
    # float64 parameters (made float32 for the kernel); gradients come back in their dtype
    for pdtype in (torch.bfloat16, torch.float64):
        x4, z4 = make((48, 640), 37, 1.0, torch.float32), make((48, 640), 38, 1.0, torch.float32)
        w4, b4 = make((640,), 39, 1.0, pdtype), make((640,), 40, 1.0, pdtype)
        dy = make((48, 640), 41, 1.0, torch.float32)
        leaves = [t.to(DEV).requires_grad_(True) for t in (x4, w4, b4, z4)]
        out4 = rmsnorm_gated(*leaves, group_size=160, norm_before_gate=False)
        out4.backward(dy.to(DEV))
        want4, _ = oracle.rmsnorm_gated(x4, w4, b4, z4, group_size=160, norm_before_gate=False)
        assert fwd_error(out4, want4) <= 2e-5
        grads = oracle.rmsnorm_gated_bwd(dy, x4, w4, b4, z4, group_size=160, norm_before_gate=False)
        for leaf, want in zip(leaves, (grads[0], grads[1], grads[2], grads[3])):
            assert leaf.grad.dtype == leaf.dtype
            # the parameter gradients are float32 sums rounded once to the parameter dtype
            tol = 1e-6 if leaf.dtype != torch.bfloat16 else 2 ** -8
            assert rel(leaf.grad, want) <= tol, (pdtype, leaf.dtype, rel(leaf.grad, want))


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(4096, 768), (8, 40000)])
def test_backward_deterministic(shape):
    from metal_kernelops.cv import rmsnorm_gated
    x, w, b, z = (make(s, 40 + i, 1.0, torch.float32).to(DEV)
                  for i, s in enumerate((shape, shape[-1:], shape[-1:], shape)))
    runs = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_(True) for t in (x, w, b, z)]
        rmsnorm_gated(*leaves).square().sum().backward()
        runs.append([t.grad for t in leaves])
    for a, c in zip(*runs):
        assert torch.equal(a, c)


@pytest.mark.gpu
def test_adam_step_lowers_the_loss():
    from metal_kernelops.cv import rmsnorm_gated
    torch.manual_seed(0)
    target, x, z = (torch.randn(256, 512, device=DEV) for _ in range(3))
    weight = torch.ones(512, device=DEV, requires_grad=True)
    bias = torch.zeros(512, device=DEV, requires_grad=True)
    opt = torch.optim.Adam([weight, bias], lr=1e-2)
    losses = []
    for _ in range(5):
        opt.zero_grad()
        loss = (rmsnorm_gated(x, weight, bias, z) - target).pow(2).mean()
        loss.backward()
        losses.append(float(loss.detach()))
        opt.step()
    assert losses[-1] < losses[0]
    assert not torch.equal(weight.detach(), torch.ones_like(weight))
    assert not torch.equal(bias.detach(), torch.zeros_like(bias))
