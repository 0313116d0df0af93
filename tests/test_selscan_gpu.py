"""Mamba-1 selective scan: HIP kernels against the float64 CPU oracle.

Bars, by the dtype of the tensor compared (north star): outputs fp32 <= 1e-5 max
relative error (max abs error over the largest reference magnitude), bf16 <= 2e-2,
fp16 <= 2e-3; gradient norms fp32 <= 1e-4 relative, bf16 2e-2, fp16 2e-3.  The
kernels widen 16-bit inputs exactly and compute in float32, so a float32 gradient
(of delta, A, D, delta_bias) is held to 1e-4 also when the activations are 16-bit.
Every measured error is printed (and logged to $MKO_PARITY_LOG when set).
"""

import os

import numpy as np
import pytest
import torch

import oracle
from cases import GRAD_TOL, OUT_TOL, mamba1_c1, mamba1_layer, max_rel, norm_rel, record

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("u", "dt", "A", "B", "C", "D", "z", "delta_bias")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "mamba1_c1.npz")


def _selective_scan():
    from metal_kernelops import selective_scan
    return selective_scan


def _gpu(inputs, dy, softplus=True):
    leaves = {k: (None if v is None else v.to(DEV).requires_grad_(True)) for k, v in inputs.items()}
    out = _selective_scan()(**leaves, delta_softplus=softplus)
    out.backward(dy.to(DEV))
    torch.cuda.synchronize()
    return out.detach(), {k: (None if v is None else v.grad) for k, v in leaves.items()}


def _ref(inputs, dy, softplus=True):
    leaves = {k: (None if v is None else v.double().requires_grad_(True)) for k, v in inputs.items()}
    out = oracle.selective_scan(**leaves, delta_softplus=softplus)
    out.backward(dy.double())
    return out.detach(), {k: (None if v is None else v.grad) for k, v in leaves.items()}


def _compare(inputs, dy, softplus, case):
    """Forward and every gradient against the oracle, each at the bar of its own dtype."""
    out, grads = _gpu(inputs, dy, softplus)
    ref, rgrads = _ref(inputs, dy, softplus)
    assert out.dtype == inputs["u"].dtype
    tol = OUT_TOL[out.dtype]
    err = record(case, "out", max_rel(out, ref), tol)
    assert err <= tol, f"forward max rel {err:.3e}"
    for name in NAMES:
        if inputs.get(name) is None:
            continue
        assert grads[name] is not None and grads[name].dtype == inputs[name].dtype, name
        tol = GRAD_TOL[grads[name].dtype]
        e = record(case, "d" + name, norm_rel(grads[name], rgrads[name]), tol)
        assert e <= tol, f"grad {name}: norm rel {e:.3e}"


def test_config1_fp32_forward_backward():
    inputs, dy = mamba1_c1()
    _compare(inputs, dy, True, "c1")


def test_config1_matches_golden_fixture():
    data = np.load(GOLDEN)
    inputs = {k: torch.from_numpy(data["in_" + k]).float() for k in NAMES}
    dy = torch.from_numpy(data["dy"]).float()
    out, grads = _gpu(inputs, dy, True)
    assert max_rel(out, torch.from_numpy(data["out"])) <= 1e-5
    for k in NAMES:
        assert norm_rel(grads[k], torch.from_numpy(data["grad_" + k])) <= 1e-4, k


def _random_problem(batch, dim, length, dstate, groups, seed, act=torch.float32, d=True, z=True,
                    bias=True):
    g = torch.Generator().manual_seed(seed)
    inputs = dict(
        u=torch.randn(batch, dim, length, generator=g).to(act),
        dt=torch.randn(batch, dim, length, generator=g),
        A=-torch.rand(dim, dstate, generator=g) * 4 - 0.05,
        B=torch.randn(batch, groups, dstate, length, generator=g).to(act),
        C=torch.randn(batch, groups, dstate, length, generator=g).to(act),
        D=torch.randn(dim, generator=g) if d else None,
        z=torch.randn(batch, dim, length, generator=g).to(act) if z else None,
        delta_bias=0.5 * torch.randn(dim, generator=g) - 1.0 if bias else None,
    )
    dy = torch.randn(batch, dim, length, generator=g).to(act)
    return inputs, dy


SHAPES = [
    (2, 8, 64, 16, 2),      # config 1 geometry, lanes span groups (atomic dB/dC path)
    (2, 128, 200, 16, 2),   # one 64-channel wavefront per group, ragged length
    (1, 256, 300, 16, 1),   # four wavefronts per workgroup, several coarse chunks
    (2, 64, 97, 5, 1),      # dstate padded to 16
    (1, 128, 130, 32, 2),   # dstate 32
    (3, 24, 77, 20, 3),     # dstate 20, ragged everything
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_shapes_fp32(shape):
    inputs, dy = _random_problem(*shape, seed=sum(shape))
    _compare(inputs, dy, True, "x".join(map(str, shape)))


@pytest.mark.parametrize("opts", [dict(d=False), dict(z=False), dict(bias=False),
                                  dict(d=False, z=False, bias=False)],
                         ids=["noD", "noz", "nobias", "bare"])
@pytest.mark.parametrize("softplus", [True, False])
def test_options(opts, softplus):
    inputs, dy = _random_problem(2, 128, 150, 16, 1, seed=7, **opts)
    if not softplus:  # raw steps must stay positive without the softplus
        inputs["dt"] = torch.rand(inputs["dt"].shape) * 0.3
        if inputs["delta_bias"] is not None:
            inputs["delta_bias"] = inputs["delta_bias"].abs() * 0.1
    _compare(inputs, dy, softplus, f"options {opts} softplus={softplus}")


def test_bf16_activations():
    inputs, dy = _random_problem(2, 256, 512, 16, 1, seed=9, act=torch.bfloat16)
    _compare(inputs, dy, True, "2x256x512 bf16")


def test_bf16_delta_and_fp16():
    inputs, dy = _random_problem(1, 128, 200, 16, 1, seed=10, act=torch.float16)
    _compare(inputs, dy, True, "1x128x200 fp16")
    inputs, dy = _random_problem(1, 128, 200, 16, 1, seed=11, act=torch.bfloat16)
    inputs["dt"] = inputs["dt"].bfloat16()
    _compare(inputs, dy, True, "1x128x200 bf16 with bf16 delta")


# At 6144 channels (batch x dim) and more, dstate <= 16 and whole 16-step blocks, the forward
# runs one lane per (channel, state) over the whole sequence; its saved states feed the backward.
LANE_SHAPES = [
    (2, 3072, 64, 16, 1),   # the smallest lane-path problem
    (2, 3072, 48, 12, 2),   # dstate 12 (lanes 12..15 idle), two groups
    (1, 6200, 32, 16, 2),   # a ragged last workgroup, two groups of 3100 channels
    (2, 3072, 16, 16, 1),   # one 16-step block: the backward's load ahead re-reads block 0
]


def _forward_kernels(inputs, softplus):
    """The library's kernels that one forward launches (its per-kernel timing names)."""
    from metal_kernelops import _native as nat
    from metal_kernelops import selective_scan
    dev = {k: (v.to(DEV) if v is not None else None) for k, v in inputs.items()}
    nat.kernel_timing_reset()
    nat.kernel_timing(True)
    try:
        with torch.no_grad():
            selective_scan(**dev, delta_softplus=softplus)
        return set(nat.kernel_times())
    finally:
        nat.kernel_timing(False)


@pytest.mark.parametrize("shape", LANE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_lane_forward_shapes_fp32(shape):
    inputs, dy = _random_problem(*shape, seed=sum(shape))
    assert "selscan_fwd_lane" in _forward_kernels(inputs, True)
    _compare(inputs, dy, True, "lane " + "x".join(map(str, shape)))


def _backward_kernels(inputs, dy, softplus=True):
    """The library's kernels that one backward launches (their timing names)."""
    from metal_kernelops import _native as nat
    leaves = {k: (v.to(DEV).requires_grad_(True) if v is not None else None) for k, v in inputs.items()}
    out = _selective_scan()(**leaves, delta_softplus=softplus)
    torch.cuda.synchronize()
    nat.kernel_timing_reset()
    nat.kernel_timing(True)
    try:
        out.backward(dy.to(DEV))
        torch.cuda.synchronize()
        return set(nat.kernel_times())
    finally:
        nat.kernel_timing(False)


@pytest.mark.parametrize("shape", [(2, 3072, 64, 16, 1), (1, 6200, 32, 16, 2), (2, 3072, 48, 12, 3),
                                   (2, 3072, 16, 16, 1)],
                         ids=["groups-of-3072", "groups-of-3100", "dstate-12-groups-of-1024", "one-16-step-block"])
def test_lane_backward_kernel_is_taken_and_deterministic(shape):
    # 6144+ channel rows, whole 16-step blocks, dstate <= 16 and groups a multiple of 4
    # channels wide: one lane per (channel, state) walks the sequence backwards. Groups of a
    # multiple of 16 channels add their dB/dC in 16-channel workgroup partials, others in
    # 4-channel wavefront partials; both orders are fixed.
    inputs, dy = _random_problem(*shape, seed=sum(shape) + 1)
    assert "selscan_bwd_lane" in _backward_kernels(inputs, dy)
    _compare(inputs, dy, True, "lane bwd " + "x".join(map(str, shape)))
    runs = [_gpu(inputs, dy, True) for _ in range(2)]
    for k in NAMES:
        assert torch.equal(runs[0][1][k], runs[1][1][k]), k


def test_lane_backward_where_the_gate_is_zero():
    # Where silu(z) is exactly zero (z = 0, or z so negative that sigmoid underflows) the
    # pre-gate output cannot come back from out / silu(z): those blocks sum C x over the
    # states instead.  Spread such elements over a few blocks and channels.
    inputs, dy = _random_problem(2, 3072, 64, 16, 1, seed=41, act=torch.bfloat16)
    z = inputs["z"].clone()
    z[0, 5, 17] = 0.0
    z[1, 3000, 63] = -200.0
    z[0, 100:104, 32:48] = 0.0
    inputs["z"] = z
    _compare(inputs, dy, True, "lane bwd, zero gates")


def test_lane_backward_without_the_forward_output():
    # A C-ABI caller may leave out NULL in the backward: dz then comes from the summed C x
    # in every block, to the same result within rounding.
    from metal_kernelops.scan import selscan_bwd_impl, selscan_fwd_impl
    inputs, dy = _random_problem(2, 3072, 32, 16, 1, seed=43)
    dev = {k: v.to(DEV) for k, v in inputs.items()}
    args = [dev[k] for k in ("u", "dt", "A", "B", "C", "D", "z", "delta_bias")]
    out, states = selscan_fwd_impl(*args, True)
    with_out = selscan_bwd_impl(dy.to(DEV), *args, True, states, out)
    without = selscan_bwd_impl(dy.to(DEV), *args, True, states, None)
    for name, a, b in zip(("du", "ddelta", "dA", "dB", "dC", "dD", "dz", "dbias"), with_out, without):
        e = record("lane bwd with/without out", name, norm_rel(a, b), 1e-5)
        assert e <= 1e-5, name


def test_unaligned_groups_take_the_chunked_forward():
    """Groups of 1550 channels (not a multiple of the 4 a lane-path wavefront shares): the
    chunked forward runs instead, to the same result."""
    inputs, dy = _random_problem(1, 6200, 32, 16, 4, seed=6252)
    kernels = _forward_kernels(inputs, True)
    assert "selscan_fwd_lane" not in kernels and "selscan_fwd_replay" in kernels
    _compare(inputs, dy, True, "1x6200x32 G4")


@pytest.mark.parametrize("opts", [dict(d=False), dict(z=False), dict(bias=False),
                                  dict(d=False, z=False, bias=False)],
                         ids=["noD", "noz", "nobias", "bare"])
@pytest.mark.parametrize("softplus", [True, False])
def test_lane_forward_options(opts, softplus):
    inputs, dy = _random_problem(2, 3072, 32, 16, 1, seed=17, **opts)
    if not softplus:
        inputs["dt"] = torch.rand(inputs["dt"].shape) * 0.3
        if inputs["delta_bias"] is not None:
            inputs["delta_bias"] = inputs["delta_bias"].abs() * 0.1
    _compare(inputs, dy, softplus, f"lane options {opts} softplus={softplus}")


def test_lane_forward_16bit():
    inputs, dy = _random_problem(2, 3072, 64, 16, 1, seed=19, act=torch.bfloat16)
    _compare(inputs, dy, True, "lane 2x3072x64 bf16")
    inputs, dy = _random_problem(2, 3072, 64, 16, 1, seed=20, act=torch.float16)
    _compare(inputs, dy, True, "lane 2x3072x64 fp16")
    # 16-bit u and z with float32 B and C
    inputs, dy = _random_problem(2, 3072, 64, 16, 1, seed=21, act=torch.bfloat16)
    inputs["B"], inputs["C"] = inputs["B"].float(), inputs["C"].float()
    _compare(inputs, dy, True, "lane 2x3072x64 bf16 u/z, fp32 B/C")


@pytest.mark.parametrize("shape", [(1, 64, 2000, 16, 1), (2, 24, 1500, 20, 3)],
                         ids=lambda s: "x".join(map(str, s)))
def test_long_sequences_few_channels(shape):
    # Few rows and 16-step chunks: 125 (94) chunks, more than 32, so the chunk chains run
    # a wavefront per (row, state) with the chunks split into runs across its lanes.
    inputs, dy = _random_problem(*shape, seed=sum(shape))
    _compare(inputs, dy, True, "long " + "x".join(map(str, shape)))


def test_partial_reductions_whole_batches_and_tail():
    # One group of 2304 channels: 9 blocks of 256 channels feed each dB/dC value (a batch
    # of eight partials plus one), and the 256 steps run as 16 chunks of 16, so each
    # dA/dD/ddelta_bias value sums 16 chunks x 2 batches = 32 partials in whole batches.
    inputs, dy = _random_problem(2, 2304, 256, 16, 1, seed=23)
    _compare(inputs, dy, True, "2x2304x256")


@pytest.mark.parametrize("shape", [(2, 256, 300, 16, 1), (2, 8, 64, 16, 2), (1, 384, 784, 16, 4),
                                   (3, 24, 77, 20, 3)],
                         ids=["groups-of-256", "c1-groups-of-4", "groups-of-96", "groups-of-8-dstate-20"])
def test_deterministic_backward(shape):
    # Bit-identical reruns for every group width: 64-multiple groups, and groups narrower or
    # wider than a wavefront whose rows meet several wavefronts (the c1 geometry, 4 channels a
    # group; the ss2d bench's 96).
    inputs, dy = _random_problem(*shape, seed=12)
    runs = [_gpu(inputs, dy, True) for _ in range(3)]
    for r in runs[1:]:
        assert torch.equal(runs[0][0], r[0])
        for k in NAMES:
            assert torch.equal(runs[0][1][k], r[1][k]), k
    _compare(inputs, dy, True, "determinism " + "x".join(map(str, shape)))


def _layer_channel_subset(case, batch, dim, length, stride):
    """A BASELINE layer shape at full size on the GPU, checked on a channel subset.

    Channels are independent in the forward; with the upstream gradient zero outside
    the subset, the dB/dC sums over channels only see the subset, so the oracle only
    needs those channels.  bf16 tensors (out, du, dz, dB, dC) are held to 2e-2, the
    float32 gradients (delta, A, D, delta_bias) to 1e-4."""
    inputs, dy = mamba1_layer(batch, dim, length, seed=0)
    sel = torch.arange(0, dim, stride)
    mask = torch.zeros(dim, dtype=torch.bool)
    mask[sel] = True
    dy = dy * mask[None, :, None].to(dy.dtype)
    out, grads = _gpu(inputs, dy, True)
    assert torch.isfinite(out).all()
    sub = {k: (v[:, sel] if k in ("u", "dt", "z") else v[sel] if k in ("A", "D", "delta_bias") else v)
           for k, v in inputs.items()}
    ref, rgrads = _ref(sub, dy[:, sel], True)
    err = record(case, "out", max_rel(out[:, sel], ref), OUT_TOL[out.dtype])
    assert err <= OUT_TOL[out.dtype], f"out {err:.3e}"
    for k in NAMES:
        g = grads[k]
        got = g[:, sel] if k in ("u", "dt", "z") else g[sel] if k in ("A", "D", "delta_bias") else g
        tol = GRAD_TOL[g.dtype]
        e = record(case, "d" + k, norm_rel(got, rgrads[k]), tol)
        assert e <= tol, f"d{k} {e:.3e} > {tol}"


def test_config2_full_size_channel_subset():
    # Config 2 (130M layer): 8 x 1536 x 2048, 64 channels spread over the width
    _layer_channel_subset("c2 8x1536x2048", 8, 1536, 2048, 24)


def test_config3_full_size_channel_subset():
    # Config 3 (2.8B layer): 4 x 5120 x 4096, 64 channels spread over the width
    _layer_channel_subset("c3 4x5120x4096", 4, 5120, 4096, 80)


def test_empty_inputs():
    ss = _selective_scan()
    for shape in ((2, 8, 0), (0, 8, 16)):
        b, d, length = shape
        u = torch.zeros(b, d, length, device=DEV, requires_grad=True)
        A = (-torch.ones(d, 4, device=DEV)).requires_grad_(True)
        B = torch.zeros(b, 2, 4, length, device=DEV, requires_grad=True)
        out = ss(u, torch.zeros_like(u), A, B, B.detach().clone(), D=torch.ones(d, device=DEV))
        assert out.shape == shape
        out.sum().backward()
        assert torch.equal(A.grad, torch.zeros_like(A))


def test_errors():
    from metal_kernelops import scan_mps
    ss = _selective_scan()
    inputs, _ = mamba1_c1()
    cpu = [inputs[k] for k in ("u", "dt", "A", "B", "C")]
    cpu[1] = torch.nn.functional.softplus(cpu[1])  # the bare scan takes positive steps
    with pytest.raises(ValueError):
        ss(*cpu)
    gpu = [t.to(DEV) for t in cpu]
    with pytest.raises(ValueError):
        ss(gpu[0], gpu[1], gpu[2], gpu[3][:, :1].repeat(1, 3, 1, 1), gpu[4][:, :1].repeat(1, 3, 1, 1))
    with pytest.raises(ValueError):
        ss(gpu[0], gpu[1], torch.zeros(8, 40, device=DEV), gpu[3], gpu[4])
    with pytest.raises(ValueError):
        scan_mps(gpu[0].transpose(0, 1).contiguous().transpose(0, 1), *gpu[1:])
    y = scan_mps(*gpu)
    ref = oracle.selective_scan(*cpu)
    assert max_rel(y, ref) <= 1e-5
