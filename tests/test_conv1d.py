"""Causal depthwise conv1d: oracle pins on the CPU, HIP parity on the GPU.

Cases follow the reference's verifier (``benchmarks/verify_causal_conv1d.py:170-193``):
decode-length and prefill forwards with and without an initial state, a narrow k=8 case
without activation, the k=1 edge, the gradient check with a seeded loss over the output
and the final state (:238-276), and the decode updates including q = 4 and a wide state
(:308-333).  Tolerances: float32 1e-5, float16 2e-3, bfloat16 2e-2, on the relative error
of the global norm (the verifier's metric, :73-79).
"""

import pytest
import torch
import torch.nn.functional as F

import oracle

DEV = "cuda"


def rel(actual, expected):
    a, e = actual.detach().double().cpu(), expected.detach().double().cpu()
    d = e.norm().item()
    return (a - e).norm().item() / d if d else (a - e).norm().item()


def make(shape, seed, scale=1.0, dtype=torch.float64):
    return (torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64) * scale).to(dtype)


# --------------------------------------------------------------------------- CPU: oracle pins


@pytest.mark.parametrize("width", [1, 2, 4, 8])
@pytest.mark.parametrize("with_state", [False, True])
def test_oracle_equals_library_conv1d(width, with_state):
    """The window sum equals torch's grouped conv1d on cat(state or zeros, x)."""
    x, w, b = make((2, 5, 19), 1), make((5, 1, width), 2), make((5,), 3)
    init = make((2, 5, width - 1), 4) if with_state else None
    out, final = oracle.causal_conv1d(x, w, b, "silu", init)
    lead = init if with_state else x.new_zeros(2, 5, width - 1)
    joined = torch.cat([lead, x], dim=-1)
    want = F.silu(F.conv1d(joined, w, b, groups=5))
    assert (out - want).abs().max() < 1e-12
    assert torch.equal(final, joined[..., 19:])


def test_oracle_special_cases():
    x = make((1, 3, 10), 5)
    identity = torch.zeros(3, 4, dtype=torch.float64)
    identity[:, -1] = 1.0  # the last tap reads the current step
    out, _ = oracle.causal_conv1d(x, identity)
    assert torch.equal(out, x)
    shift = torch.zeros(3, 4, dtype=torch.float64)
    shift[:, 0] = 1.0  # the first tap reads three steps back
    out, _ = oracle.causal_conv1d(x, shift)
    assert torch.equal(out[..., 3:], x[..., :-3]) and not out[..., :3].any()


def test_oracle_update_equals_prefill():
    """q single-token updates from a state equal one prefill from that initial state."""
    x, w, b = make((2, 4, 6), 6), make((4, 4), 7), make((4,), 8)
    state = make((2, 4, 3), 9)
    want, final = oracle.causal_conv1d(x, w, b, "silu", state)
    outs = []
    for t in range(6):
        o, state = oracle.causal_conv1d_update(state, x[..., t:t + 1], w, b, "silu")
        outs.append(o)
    assert (torch.cat(outs, dim=-1) - want).abs().max() < 1e-12
    assert (state - final).abs().max() < 1e-12


def test_oracle_gradcheck():
    x = make((1, 2, 7), 10).requires_grad_(True)
    w = make((2, 1, 3), 11, 0.5).requires_grad_(True)
    b = make((2,), 12).requires_grad_(True)
    init = make((1, 2, 2), 13).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda *a: oracle.causal_conv1d(*a[:3], "silu", a[3])[0], (x, w, b, init))


def test_reference_twin_matches_oracle():
    from metal_kernelops.cv import causal_conv1d_ref
    x, w, b, init = make((2, 5, 13), 14), make((5, 1, 4), 15), make((5,), 16), make((2, 5, 3), 17)
    out, final = causal_conv1d_ref(x, w, b, "silu", init, True)
    want, wfinal = oracle.causal_conv1d(x, w, b, "silu", init)
    assert (out - want).abs().max() < 1e-12 and torch.equal(final, wfinal)


def test_errors_on_the_host():
    from metal_kernelops.cv import causal_conv1d_fn, causal_conv1d_update
    x, w = make((1, 4, 8), 1, dtype=torch.float32), make((4, 1, 4), 2, dtype=torch.float32)
    with pytest.raises(ValueError, match="depthwise"):
        causal_conv1d_fn(x, w.reshape(2, 2, 4))
    with pytest.raises(NotImplementedError):
        causal_conv1d_fn(x, w, activation="gelu")
    with pytest.raises(ValueError, match="channels"):
        causal_conv1d_fn(x[:, :3], w)
    with pytest.raises(ValueError, match="initial_state"):
        causal_conv1d_fn(x, w, initial_state=torch.zeros(1, 4, 2))
    with pytest.raises(ValueError, match="ROCm GPU"):
        causal_conv1d_fn(x, w)
    with pytest.raises(ValueError, match="stride 1"):
        causal_conv1d_update(x[..., 0], torch.zeros(1, 4, 6)[..., ::2], w)
    with pytest.raises(ValueError, match="at least"):
        causal_conv1d_update(x[..., 0], torch.zeros(1, 4, 2), w)
    with pytest.raises(RuntimeError, match="autograd"):
        causal_conv1d_update(x[..., 0].requires_grad_(True), torch.zeros(1, 4, 3), w)


# --------------------------------------------------------------------------- GPU: HIP parity

TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}

# name, batch, channels, length, width, activation, initial_state, dtype
CASES = [
    ("decode-1x2048", 1, 2048, 1, 4, "silu", True, torch.float32),
    ("decode-16x1536-fp16", 16, 1536, 1, 4, "silu", True, torch.float16),
    ("short-2x256x16", 2, 256, 16, 4, "silu", False, torch.float32),
    ("prefill-1x768x4096", 1, 768, 4096, 4, "silu", True, torch.float32),
    ("prefill-2x512x2048", 2, 512, 2048, 4, "silu", False, torch.float32),
    ("prefill-4x768x1024-fp16", 4, 768, 1024, 4, "silu", True, torch.float16),
    ("prefill-4x256x1000-bf16", 4, 256, 1000, 4, "swish", True, torch.bfloat16),
    ("narrow-4x128x200-k8", 4, 128, 200, 8, None, False, torch.float32),
    ("k1-2x64x33", 2, 64, 33, 1, None, True, torch.float32),
    ("ragged-3x40x37-k3", 3, 40, 37, 3, "silu", True, torch.float32),
    ("wide-2x16x90-k20", 2, 16, 90, 20, "silu", True, torch.float32),
    # this build's own boundaries: rows longer than one interleaved wavefront's span in both
    # directions (the carry crosses segments), aligned and ragged, and width 8
    ("long-2x64x9000-k4", 2, 64, 9000, 4, "silu", True, torch.float32),
    ("long-2x32x12288-k8-bf16", 2, 32, 12288, 8, "silu", True, torch.bfloat16),
]


def _inputs(batch, channels, length, width, has_state, dtype, seed=0):
    w = make((channels, 1, width), seed + 1, 0.5, dtype)
    b = make((channels,), seed + 2, 1.0, dtype)
    x = make((batch, channels, length), seed + 3, 1.0, dtype)
    s = make((batch, channels, width - 1), seed + 4, 1.0, dtype) if has_state else None
    return x, w, b, s


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_forward(case):
    from metal_kernelops.cv import causal_conv1d_fn
    _, batch, channels, length, width, act, has_state, dtype = case
    x, w, b, s = _inputs(batch, channels, length, width, has_state, dtype)
    with torch.no_grad():
        out, final = causal_conv1d_fn(x.to(DEV), w.to(DEV), b.to(DEV), act, None if s is None else s.to(DEV), True)
        plain = causal_conv1d_fn(x.to(DEV), w.to(DEV), b.to(DEV), act, None if s is None else s.to(DEV))
    torch.cuda.synchronize()
    want, wfinal = oracle.causal_conv1d(x, w, b, act, s)
    assert out.dtype == dtype and out.shape == x.shape
    assert rel(out, want) <= TOL[dtype], rel(out, want)
    assert rel(final, wfinal) == 0.0
    assert torch.equal(out, plain)


@pytest.mark.gpu
@pytest.mark.parametrize("case", [c for c in CASES if c[3] > 1], ids=lambda c: c[0])
def test_gradients(case):
    from metal_kernelops.cv import causal_conv1d_fn
    _, batch, channels, length, width, act, has_state, dtype = case
    x, w, b, s = _inputs(batch, channels, length, width, has_state, dtype, seed=10)
    seed_out = make((batch, channels, length), 15, 1.0, dtype)
    seed_final = make((batch, channels, width - 1), 16, 1.0, dtype)
    leaves = [t.to(DEV).requires_grad_(True) if t is not None else None for t in (x, w, b, s)]
    out, final = causal_conv1d_fn(leaves[0], leaves[1], leaves[2], act, leaves[3], True)
    ((out * seed_out.to(DEV)).sum() + (final * seed_final.to(DEV)).sum()).backward()
    torch.cuda.synchronize()
    ref = [t.double().requires_grad_(True) if t is not None else None for t in (x, w, b, s)]
    rout, rfinal = oracle.causal_conv1d(ref[0], ref[1], ref[2], act, ref[3])
    ((rout * seed_out.double()).sum() + (rfinal * seed_final.double()).sum()).backward()
    tol = 1e-4 if dtype == torch.float32 else 10 * TOL[dtype]
    for name, got, want in zip(("x", "weight", "bias", "initial_state"), leaves, ref):
        if got is None:
            continue
        assert got.grad is not None and got.grad.dtype == got.dtype, name
        assert rel(got.grad, want.grad) <= tol, (name, rel(got.grad, want.grad))


@pytest.mark.gpu
def test_bench_shape_full_size_channel_subset():
    """The bench's prefill shape at full size (4 x 5120 x 4096, width 4, bf16, SiLU).  Channels
    are independent in the output, dx and the tap and bias gradients, so the full-size run is
    checked on 64 channels spread over the width against the oracle."""
    from metal_kernelops.cv import causal_conv1d_fn
    batch, channels, length, width = 4, 5120, 4096, 4
    g = torch.Generator().manual_seed(50)
    x = torch.randn(batch, channels, length, generator=g).bfloat16()
    w = (0.5 * torch.randn(channels, width, generator=g)).bfloat16()
    b = torch.randn(channels, generator=g).bfloat16()
    dy = torch.randn(batch, channels, length, generator=g).bfloat16()
    leaves = [t.to(DEV).requires_grad_(True) for t in (x, w, b)]
    out = causal_conv1d_fn(leaves[0], leaves[1], leaves[2], activation="silu")
    out.backward(dy.to(DEV))
    torch.cuda.synchronize()
    sel = torch.arange(0, channels, 80)
    xs, ws, bs = (t.double().requires_grad_(True) for t in (x[:, sel], w[sel], b[sel]))
    want, _ = oracle.causal_conv1d(xs, ws, bs, "silu")
    want.backward(dy[:, sel].double())
    on = sel.to(DEV)
    assert rel(out.detach()[:, on], want) <= TOL[torch.bfloat16]
    for name, got, ref in (("x", leaves[0].grad[:, on], xs.grad), ("weight", leaves[1].grad[on], ws.grad),
                           ("bias", leaves[2].grad[on], bs.grad)):
        assert rel(got, ref) <= 10 * TOL[torch.bfloat16], (name, rel(got, ref))


@pytest.mark.gpu
def test_backward_deterministic():
    from metal_kernelops.cv import causal_conv1d_fn
    x, w, b, s = _inputs(4, 256, 777, 4, True, torch.float32, seed=30)
    runs = []
    for _ in range(2):
        leaves = [t.to(DEV).requires_grad_(True) for t in (x, w, b, s)]
        causal_conv1d_fn(leaves[0], leaves[1], leaves[2], "silu", leaves[3]).square().sum().backward()
        runs.append([t.grad for t in leaves])
    for a, c in zip(*runs):
        assert torch.equal(a, c)


@pytest.mark.gpu
def test_mixed_dtypes_and_empty():
    from metal_kernelops.cv import causal_conv1d_fn
    x = make((2, 32, 50), 40, 1.0, torch.bfloat16)
    w = make((32, 4), 41, 0.5, torch.float32)  # arithmetic follows the weight, result x's dtype
    out = causal_conv1d_fn(x.to(DEV), w.to(DEV), activation="silu")
    want, _ = oracle.causal_conv1d(x.float(), w, None, "silu")
    assert out.dtype == torch.bfloat16 and rel(out, want) <= 1e-2
    empty = causal_conv1d_fn(torch.zeros(0, 32, 50, device=DEV), w.to(DEV))
    assert empty.shape == (0, 32, 50)
    leaf = torch.zeros(2, 32, 0, device=DEV, requires_grad=True)
    out, final = causal_conv1d_fn(leaf, w.to(DEV), return_final_state=True)
    assert out.shape == (2, 32, 0) and final.shape == (2, 32, 3)


# name, batch, channels, q, width, activation, state columns, dtype
UPDATES = [
    ("update-1x2048x1", 1, 2048, 1, 4, "silu", 3, torch.float32),
    ("update-64x2048x1", 64, 2048, 1, 4, "silu", 3, torch.float32),
    ("update-1x2048x4", 1, 2048, 4, 4, "silu", 3, torch.float32),
    ("update-8x2048x1-wide", 8, 2048, 1, 4, "silu", 8, torch.float32),
    ("update-16x1536x1-fp16", 16, 1536, 1, 4, "silu", 3, torch.float16),
    ("update-4x512x6-bf16", 4, 512, 6, 4, None, 5, torch.bfloat16),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", UPDATES, ids=lambda c: c[0])
def test_update(case):
    from metal_kernelops.cv import causal_conv1d_update
    _, batch, channels, q, width, act, cols, dtype = case
    w, b = make((channels, 1, width), 21, 0.5, dtype), make((channels,), 22, 1.0, dtype)
    x, state = make((batch, channels, q), 23, 1.0, dtype), make((batch, channels, cols), 24, 1.0, dtype)
    dev_state = state.to(DEV)
    out = causal_conv1d_update(x.to(DEV), dev_state, w.to(DEV), b.to(DEV), act)
    torch.cuda.synchronize()
    want, wstate = oracle.causal_conv1d_update(state, x, w, b, act)
    assert out.shape == x.shape and out.dtype == dtype
    assert rel(out, want) <= TOL[dtype]
    assert rel(dev_state, wstate) == 0.0
    if q == 1:  # a (batch, channels) token comes back in the same rank
        out2 = causal_conv1d_update(x[..., 0].to(DEV), state.to(DEV), w.to(DEV), b.to(DEV), act)
        assert out2.shape == (batch, channels)


@pytest.mark.gpu
def test_update_in_a_cache_slice():
    """The state is a strided slice of a larger cache; only its columns change."""
    from metal_kernelops.cv import causal_conv1d_update
    cache = make((3, 64, 10), 50, 1.0, torch.float32).to(DEV)
    before = cache.clone()
    view = cache[:, 8:40, 2:6]  # strides (640, 10, 1)
    w, b, x = make((32, 4), 51, 0.5, torch.float32), make((32,), 52), make((3, 32, 2), 53)
    out = causal_conv1d_update(x.float().to(DEV), view, w.to(DEV), b.float().to(DEV), "silu")
    want, wstate = oracle.causal_conv1d_update(before[:, 8:40, 2:6].cpu(), x, w, b, "silu")
    assert rel(out, want) <= 1e-5 and rel(cache[:, 8:40, 2:6], wstate) <= 1e-7
    mask = torch.ones_like(cache, dtype=torch.bool)
    mask[:, 8:40, 2:6] = False
    assert torch.equal(cache[mask], before[mask])


@pytest.mark.gpu
def test_decode_steps_equal_prefill():
    from metal_kernelops.cv import causal_conv1d_fn, causal_conv1d_update
    x, w, b, s = _inputs(2, 128, 12, 4, True, torch.float32, seed=60)
    x, w, b, s = (t.float().to(DEV) for t in (x, w, b, s))
    with torch.no_grad():
        want, final = causal_conv1d_fn(x, w, b, "silu", s, True)
    state = s.clone()
    outs = [causal_conv1d_update(x[..., t], state, w, b, "silu") for t in range(12)]
    assert rel(torch.stack(outs, dim=-1), want) <= 1e-6
    assert torch.equal(state, final)
