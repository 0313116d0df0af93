"""Four-path 2D selective scan (ss2d): oracle pins on the CPU, HIP parity on the GPU.

Cases follow the reference's verifier (``benchmarks/verify_path_scan.py``): the
cumulative-sum ordering check (:125-159), the step-wise formulation (:162-188),
central differences in float64 (:191-215), degenerate extents and state counts
(:218-238), the state limit (:241-250), strided inputs (:253-277) and its
forward/backward shapes (:502-507), with its tolerances: 1e-5 on the output and
1e-4 on gradient norms for float32.
"""

import pytest
import torch

import oracle
from cases import max_rel, norm_rel

DEV = "cuda"
NAMES = ("u", "dt", "A", "B", "C")


def _build(batch, channels, groups, states, height, width, seed, dtype=torch.float32):
    """Inputs drawn as in verify_path_scan.py:69-84: dt in [0.05, 0.25], A in [-1.1, -0.1]."""
    g = torch.Generator().manual_seed(seed)
    shape = (batch, channels, height, width)
    u = torch.randn(shape, generator=g, dtype=dtype)
    dt = torch.rand(shape, generator=g, dtype=dtype) * 0.2 + 0.05
    A = -(torch.rand((channels, states), generator=g, dtype=dtype) + 0.1)
    B = torch.randn((batch, groups, states, height, width), generator=g, dtype=dtype)
    C = torch.randn((batch, groups, states, height, width), generator=g, dtype=dtype)
    return dict(u=u, dt=dt, A=A, B=B, C=C)


def _cumsum_expected(values, height, width):
    """A = 0, dt = 1, B = C = 1: every path is a running sum in its own order."""
    expected = torch.zeros_like(values)
    for order in oracle.ss2d_path_orders(height, width):
        idx = torch.tensor(order)
        seq = values.index_select(0, idx).cumsum(0)
        back = torch.empty_like(seq)
        back[idx] = seq
        expected += back
    return expected


ORDER_MAPS = ((4, 3), (1, 6), (6, 1), (5, 5))


# --------------------------------------------------------------------------- CPU: oracle pins


@pytest.mark.parametrize("hw", ORDER_MAPS, ids=lambda s: f"{s[0]}x{s[1]}")
def test_oracle_cumsum_degeneration(hw):
    height, width = hw
    values = torch.randn(height * width, generator=torch.Generator().manual_seed(height * 31 + width),
                         dtype=torch.float64)
    ones = torch.ones(1, 1, height, width, dtype=torch.float64)
    got = oracle.ss2d_scan(values.reshape(1, 1, height, width), ones, torch.zeros(1, 1, dtype=torch.float64),
                           ones.reshape(1, 1, 1, height, width), ones.reshape(1, 1, 1, height, width))
    assert max_rel(got.reshape(-1), _cumsum_expected(values, height, width)) < 1e-12


def test_oracle_orders_match_views():
    """The index lists agree with the transposed/flipped views the package builds."""
    from metal_kernelops.cv.path_scan import path_orders
    for height, width in ORDER_MAPS + ((3, 7),):
        lists = oracle.ss2d_path_orders(height, width)
        views = path_orders(height, width)
        for a, b in zip(lists, views):
            assert a == b.tolist()


def test_oracle_equals_literal_loops():
    """Each path equals the literal per-index Mamba-1 loop on the permuted sequence."""
    args = _build(2, 4, 2, 3, 3, 4, seed=5, dtype=torch.float64)
    got = oracle.ss2d_scan(**args)
    batch, channels, height, width = args["u"].shape
    length = height * width
    flat = {k: args[k].reshape(*args[k].shape[:-2], length) for k in ("u", "dt", "B", "C")}
    total = []
    for order in oracle.ss2d_path_orders(height, width):
        idx = torch.tensor(order)
        y = oracle.selective_scan_loop(flat["u"][..., idx], flat["dt"][..., idx], args["A"],
                                       flat["B"][..., idx], flat["C"][..., idx])
        back = torch.zeros(batch, channels, length, dtype=torch.float64)
        back[..., idx] = y
        total.append(back)
    want = ((total[0] + total[2]) + (total[1] + total[3])).reshape(got.shape)
    assert max_rel(got, want) < 1e-12


@pytest.mark.parametrize("merge", ["sum", "mean"])
def test_oracle_gradcheck(merge):
    """Central differences in float64 on a two-by-two map (verify_path_scan.py:191-215)."""
    args = _build(1, 2, 1, 2, 2, 2, seed=13, dtype=torch.float64)
    leaves = tuple(args[k].requires_grad_(True) for k in NAMES)
    assert torch.autograd.gradcheck(lambda *a: oracle.ss2d_scan(*a, merge=merge), leaves, eps=1e-6, atol=1e-8)


def test_reference_twin_matches_oracle():
    from metal_kernelops.cv import ss2d_scan_reference
    for shape in ((2, 8, 2, 4, 6, 5), (1, 3, 3, 2, 5, 7)):
        args = _build(*shape, seed=3, dtype=torch.float64)
        for merge in ("sum", "mean"):
            assert max_rel(ss2d_scan_reference(**args, merge=merge), oracle.ss2d_scan(**args, merge=merge)) < 1e-12


def test_errors_on_the_host():
    from metal_kernelops.cv import ss2d_scan, ss2d_scan_reference
    args = _build(1, 4, 1, 3, 3, 3, seed=1)
    with pytest.raises(ValueError, match="merge"):
        ss2d_scan_reference(**args, merge="max")
    bad = dict(args, B=args["B"][:, :, :2], C=args["C"][:, :, :2])
    with pytest.raises(ValueError, match="states"):
        ss2d_scan_reference(**bad)
    with pytest.raises(ValueError, match="divide"):
        ss2d_scan_reference(**_build(1, 4, 3, 3, 3, 3, seed=1))
    with pytest.raises(ValueError, match="ROCm GPU"):
        ss2d_scan(**args)  # CPU tensors: the HIP path refuses them


# --------------------------------------------------------------------------- GPU: HIP parity


def _gpu_case(shape, merge="sum", seed=1, tol=1e-5, gradient_tol=1e-4, dtype=torch.float32):
    from metal_kernelops.cv import ss2d_scan
    args = _build(*shape, seed=seed)
    g = torch.Generator().manual_seed(seed + 1000)
    dy = torch.randn(shape[0], shape[1], shape[4], shape[5], generator=g)
    leaves = {k: (v.to(dtype) if k in ("u", "B", "C") else v).to(DEV).requires_grad_(True) for k, v in args.items()}
    out = ss2d_scan(**leaves, merge=merge)
    out.backward(dy.to(DEV).to(out.dtype))
    torch.cuda.synchronize()
    ref = {k: v.double().requires_grad_(True) for k, v in args.items()}
    want = oracle.ss2d_scan(**ref, merge=merge)
    want.backward(dy.double())
    assert out.shape == want.shape and out.dtype == leaves["u"].dtype
    assert max_rel(out, want) <= tol, f"forward {max_rel(out, want):.2e}"
    for k in NAMES:
        got_grad = leaves[k].grad
        assert got_grad is not None and got_grad.dtype == leaves[k].dtype and got_grad.shape == leaves[k].shape
        err = norm_rel(got_grad, ref[k].grad)
        assert err <= gradient_tol, f"d{k} {err:.2e}"


SHAPES = [
    (2, 8, 2, 4, 6, 5),
    (2, 16, 1, 8, 8, 8),
    (1, 3, 3, 2, 5, 7),
    (1, 4, 4, 3, 3, 5),     # per-channel groups
    (1, 1, 1, 3, 3, 3),     # one channel
    (1, 8, 1, 16, 9, 11),   # sixteen states
    (1, 4, 2, 32, 5, 7),    # thirty-two states
    (1, 6, 2, 5, 13, 3),    # five states
    (1, 4, 1, 3, 1, 1),     # single pixel
    (1, 4, 1, 3, 1, 7),     # single row
    (1, 4, 1, 3, 7, 1),     # single column
    (2, 64, 1, 16, 8, 12),  # a full 64-channel wavefront per group
    (1, 8, 1, 16, 28, 28),  # 784 steps: 49 chunks, chained by a wavefront per (row, state)
]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_forward_backward(shape):
    _gpu_case(shape)


@pytest.mark.gpu
def test_mean_merge():
    _gpu_case((1, 4, 1, 3, 4, 5), merge="mean")


@pytest.mark.gpu
def test_bf16_activations():
    _gpu_case((2, 16, 1, 8, 8, 8), tol=2e-2, gradient_tol=2e-2, dtype=torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("hw", ORDER_MAPS, ids=lambda s: f"{s[0]}x{s[1]}")
def test_traversal_order(hw):
    from metal_kernelops.cv import ss2d_scan
    height, width = hw
    values = torch.randn(height * width, generator=torch.Generator().manual_seed(height * 31 + width))
    ones = torch.ones(1, 1, height, width, device=DEV)
    got = ss2d_scan(values.reshape(1, 1, height, width).to(DEV), ones, torch.zeros(1, 1, device=DEV),
                    ones.reshape(1, 1, 1, height, width), ones.reshape(1, 1, 1, height, width))
    assert max_rel(got.reshape(-1), _cumsum_expected(values.double(), height, width)) < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1, 4, 1, 3, 0, 5), (1, 4, 1, 3, 5, 0), (2, 0, 0, 4, 3, 3),
                                   (1, 4, 1, 0, 3, 3), (0, 4, 1, 3, 3, 3)],
                         ids=["zero-height", "zero-width", "no-channels", "no-states", "batch-of-zero"])
def test_degenerate_extents(shape):
    from metal_kernelops.cv import ss2d_scan
    args = {k: v.to(DEV).requires_grad_(True) for k, v in _build(*shape, seed=2).items()}
    out = ss2d_scan(**args)
    assert tuple(out.shape) == (shape[0], shape[1], shape[4], shape[5])
    assert not out.any()
    out.sum().backward()
    for k in NAMES:
        assert args[k].grad is not None and not args[k].grad.any()


@pytest.mark.gpu
def test_state_limit_and_devices():
    from metal_kernelops.cv import ss2d_scan
    args = {k: v.to(DEV) for k, v in _build(1, 4, 1, 33, 3, 3, seed=3).items()}
    with pytest.raises(ValueError, match="32"):
        ss2d_scan(**args)


@pytest.mark.gpu
def test_strided_inputs():
    from metal_kernelops.cv import ss2d_scan
    g = torch.Generator().manual_seed(91)
    stored = dict(u=torch.randn(2, 4, 5, 6, generator=g), dt=torch.rand(2, 4, 5, 6, generator=g) * 0.2 + 0.05,
                  A=-(torch.rand(3, 4, generator=g) + 0.1), B=torch.randn(2, 2, 3, 5, 6, generator=g),
                  C=torch.randn(2, 2, 3, 5, 6, generator=g))
    dims = dict(u=(2, 3), dt=(2, 3), A=(0, 1), B=(3, 4), C=(3, 4))
    views = {k: stored[k].transpose(*dims[k]) for k in stored}
    dev = {k: stored[k].to(DEV).transpose(*dims[k]) for k in stored}  # strided views of device storage
    assert not any(v.is_contiguous() for v in dev.values())
    got = ss2d_scan(**dev)
    want = oracle.ss2d_scan(**{k: v.double() for k, v in views.items()})
    assert max_rel(got, want) < 1e-5


@pytest.mark.gpu
def test_deterministic():
    from metal_kernelops.cv import ss2d_scan
    args = _build(2, 64, 1, 16, 8, 12, seed=4)
    runs = []
    for _ in range(2):
        leaves = {k: v.to(DEV).requires_grad_(True) for k, v in args.items()}
        out = ss2d_scan(**leaves)
        out.square().sum().backward()
        runs.append([out.detach()] + [leaves[k].grad for k in NAMES])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
