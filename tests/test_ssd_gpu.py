"""Mamba-2 SSD chunk scan: HIP kernels against the float64 CPU oracle.

Option/shape matrix follows the reference verifier (benchmarks/verify_mamba2_chunk.py:
113-179, 237-290): grouped heads, D (H,) and (H,P), z, dt_bias, softplus,
initial states, ragged lengths, chunk sizes larger than the sequence.
Tolerances (reference and north star): fp32 1e-5, fp16 2e-3, bf16 2e-2 max
relative error; gradient norms 1e-4 (fp32).
"""

import json
import math
import numpy as np
import os
import pytest
import torch

import oracle
from cases import max_rel, norm_rel, record, ssd_matrix_inputs, ssd_problem

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ssd_small.npz")


def _api():
    from metal_kernelops.cv import mamba2_chunk_scan
    return mamba2_chunk_scan


def _problem(batch, length, nheads, headdim, ngroups, dstate, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, length, nheads, headdim, generator=g)
    dt = torch.randn(batch, length, nheads, generator=g)
    A = -torch.exp(torch.rand(nheads, generator=g))
    B = torch.randn(batch, length, ngroups, dstate, generator=g)
    C = torch.randn(batch, length, ngroups, dstate, generator=g)
    return [t.to(dtype) for t in (x, dt, A, B, C)]


def _options(batch, length, nheads, headdim, dstate, seed=1):
    g = torch.Generator().manual_seed(seed)
    return dict(D=torch.randn(nheads, generator=g),
                z=torch.randn(batch, length, nheads, headdim, generator=g),
                dt_bias=torch.randn(nheads, generator=g) * 0.1,
                initial_states=torch.randn(batch, nheads, headdim, dstate, generator=g) * 0.1)


SHAPES = [
    (2, 13, 4, 6, 2, 5),
    (1, 16, 4, 4, 1, 4),
    (2, 9, 4, 3, 4, 3),
    (1, 5, 2, 2, 1, 3),
    (2, 300, 4, 64, 1, 128),   # two 128-token chunks, ragged tail
    (1, 1100, 2, 80, 2, 72),   # 256-token chunks, P and N not multiples of 64
    (1, 1100, 3, 64, 1, 128),  # 256-token chunks at the c4 head shape, ragged tail
    (1, 1030, 4, 60, 2, 128),  # 256-token chunks at d_state 128 with element-wise d_head rows
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_forward_option_matrix(shape, dtype):
    seed = sum(shape)
    args = [t.to(DEV, dtype) for t in _problem(*shape, seed=seed, dtype=dtype)]
    options = {k: v.to(DEV, dtype) for k, v in _options(*shape[:4], shape[5], seed=seed + 10).items()}
    cpu = [t.cpu().double() for t in args]
    cpu_opt = {k: v.cpu().double() for k, v in options.items()}
    y_ref, s_ref = oracle.mamba2_chunk_scan_recurrence(*cpu, **cpu_opt, dt_softplus=True)
    y, s = _api()(*args, 64, **options, dt_softplus=True)
    assert y.dtype == dtype and s.dtype == dtype
    assert y.shape == y_ref.shape and s.shape == s_ref.shape
    case = f"fwd {'x'.join(map(str, shape))} {dtype}"
    assert record(case, "y", max_rel(y, y_ref), TOL[dtype]) <= TOL[dtype], f"y {max_rel(y, y_ref):.3e}"
    assert record(case, "final_state", max_rel(s, s_ref), TOL[dtype]) <= TOL[dtype], \
        f"state {max_rel(s, s_ref):.3e}"


def test_defaults_and_each_option_alone():
    args = [t.to(DEV) for t in _problem(2, 9, 4, 6, 2, 5, seed=7)]
    cpu = [t.cpu().double() for t in args]
    options = _options(2, 9, 4, 6, 5, seed=17)
    dp = torch.randn(4, 6, generator=torch.Generator().manual_seed(3))
    for extra in ({}, {"D": options["D"]}, {"D": dp}, {"dt_bias": options["dt_bias"]},
                  {"initial_states": options["initial_states"]}, {"z": options["z"]}):
        y_ref, s_ref = oracle.mamba2_chunk_scan_recurrence(*cpu, **{k: v.double() for k, v in extra.items()})
        y, s = _api()(*args, 4, **{k: v.to(DEV) for k, v in extra.items()})
        assert max_rel(y, y_ref) <= 1e-5, list(extra)
        assert max_rel(s, s_ref) <= 1e-5, list(extra)


def test_layout_contracts():
    from metal_kernelops.cv import last_path
    args = [t.to(DEV) for t in _problem(2, 13, 4, 6, 2, 5, seed=11)]
    wide = torch.zeros(2, 13, 4, 12, device=DEV)
    wide[:, :, :, ::2] = args[0]
    y_strided, _ = _api()(wide[:, :, :, ::2], *args[1:], 5)
    y_plain, _ = _api()(*args, 5)
    assert torch.equal(y_strided, y_plain)
    assert last_path() == "hip"
    state0 = torch.randn(2, 4, 6, 5, generator=torch.Generator().manual_seed(12)).to(DEV)
    y_a, s_a = _api()(*args, 5, initial_states=state0)
    y_b, s_b = _api()(*args, 5, initial_states=state0.transpose(-1, -2))
    y_c, s_c = _api()(*args, 5, initial_states=state0[:, None])
    assert torch.equal(y_a, y_b) and torch.equal(y_a, y_c) and torch.equal(s_a, s_c)
    with pytest.raises(ValueError):
        _api()(*args, 5, initial_states=torch.zeros(2, 4, 5, 5, device=DEV))
    with pytest.raises(ValueError):
        _api()(*(t.cpu() for t in args), 5)
    with pytest.raises(ValueError):
        _api()(*args, 0)


def test_config4_shape_batch_slice():
    # Config 4 geometry (H64 P64 N128, L 4096, bf16); batches are independent, so
    # the oracle runs on one batch of the full-size problem.
    p = ssd_problem(4, 4096, 64, 64, 1, 128, seed=0, act=torch.bfloat16, init=False)
    dev = {k: (None if v is None else v.to(DEV)) for k, v in p.items()}
    y, s = _api()(dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"], 256, D=dev["D"], z=dev["z"],
                  dt_bias=dev["dt_bias"], dt_softplus=True)
    one = {k: (None if v is None else (v[:1] if v.dim() >= 3 else v)) for k, v in p.items()}
    y_ref, s_ref = oracle.mamba2_chunk_scan_composition(
        one["x"].double(), one["dt"].double(), one["A"].double(), one["B"].double(), one["C"].double(),
        chunk_size=256, D=one["D"].double(), z=one["z"].double(), dt_bias=one["dt_bias"].double(),
        dt_softplus=True)
    assert record("c4 fwd batch 0", "y", max_rel(y[:1], y_ref), 2e-2) <= 2e-2
    assert record("c4 fwd batch 0", "final_state", max_rel(s[:1], s_ref), 2e-2) <= 2e-2
    assert torch.isfinite(y).all() and torch.isfinite(s).all()


# ---------------------------------------------------------------- backward

# Gradient norm-relative tolerances against the float64 oracle run on the same (rounded)
# inputs: 1e-4 for fp32 (the reference's gradient bar); half precision rounds the
# matrix-core operands as the reference's composition does, so every gradient of a
# half-precision problem (the float32 ones of dt, A, D and dt_bias included) is held to
# the half-precision output bars, 2e-2 for bf16, and 1e-2 for fp16.
GRAD_TOL = {torch.float32: 1e-4, torch.float16: 1e-2, torch.bfloat16: 2e-2}
ACTS = ("x", "B", "C", "z", "initial_states")
NAMES = ("x", "dt", "A", "B", "C")


def _leaves(tensors, device, dtype=None):
    out = {}
    for k, v in tensors.items():
        t = v.detach().to(device)
        if dtype is not None and k in ACTS:
            t = t.to(dtype)
        out[k] = t.requires_grad_(True)
    return out


def _run_grad(fn, leaves, dy, dfinal, softplus, double=False):
    kw = {k: v for k, v in leaves.items() if k not in NAMES}
    y, s = fn(*(leaves[k] for k in NAMES), **kw, dt_softplus=softplus)
    loss = (y.double() * dy).sum() if dy is not None else 0
    if dfinal is not None:
        loss = loss + (s.double() * dfinal).sum()
    loss.backward()
    return {k: v.grad for k, v in leaves.items()}


def _oracle_grads(inputs, dy, dfinal, softplus, dtype=torch.float64):
    """float64 oracle gradients on the inputs rounded to the kernel's activation dtype."""
    leaves = _leaves({k: (v.to(dtype) if k in ACTS else v).double() for k, v in inputs.items()}, "cpu")
    return _run_grad(oracle.mamba2_chunk_scan_recurrence, leaves, dy, dfinal, softplus)


def _gpu_grads(inputs, dy, dfinal, softplus, dtype):
    leaves = _leaves(inputs, DEV, dtype)
    api = lambda x, dt, A, B, C, **kw: _api()(x, dt, A, B, C, 64, **kw)
    return _run_grad(api, leaves, None if dy is None else dy.to(DEV), None if dfinal is None else dfinal.to(DEV),
                     softplus)


def _inputs(shape, seed, options=("D", "z", "dt_bias", "initial_states"), d_row=False):
    return ssd_matrix_inputs(shape, seed, options, d_row)


def _compare(got, ref, tol, what):
    for k, r in ref.items():
        gk = got[k]
        if r is None:  # the loss does not depend on this input
            assert gk is None or torch.count_nonzero(gk) == 0, f"{what}: nonzero gradient for {k}"
            continue
        assert gk is not None, f"{what}: no gradient for {k}"
        assert gk.shape == r.shape, f"{what}: {k} shape {tuple(gk.shape)} vs {tuple(r.shape)}"
        assert torch.isfinite(gk).all(), f"{what}: {k} not finite"
        err = record(what, "d" + k, norm_rel(gk, r), tol)
        assert err <= tol, f"{what}: d{k} norm-relative error {err:.3e} > {tol}"


# The 16-bit gradient bars come from the reference's own arithmetic: the norm-relative error of
# its bf16 / fp16 torch composition's autograd (oracle.mamba2_chunk_scan_composition) against
# float64 on the same rounded inputs, measured by tests/golden/make_ssd_half_bars.py.  Each
# gradient of a 16-bit case is held to 1.5x that error.  On the matrix's small cases a
# gradient has few elements (dA one per head, ddt 72 on 2x9x4), so one case's error is a noisy
# sample (the composition's bf16 dA spans 0.8e-3 to 6e-3 over the rows): there the bar is 1.5x
# the larger of the case's error and the root-mean-square error of that gradient over the
# matrix's rows of the dtype.  The config-4 cases are held to their own error, except dA: the
# kernels round u = step x, C.B^T and K = C.B^T e^{cs_l - cs_s} to the input dtype for the
# matrix cores, where the composition keeps its decays and C.B^T products in fp32 and folds
# the step into one rounded score, and with 64 heads that shows in dA.  The fixture holds the
# dA error those rounding points imply (make_ssd_half_bars.kernel_rounding_dA, a float64
# restatement of where the kernels round, which the GPU's own per-token sums match): 3.9e-3
# on the causal prefix and 8.1e-3 on batch 0, against the composition's 1.9e-3 and 2.3e-3.
# The config-4 dA is held to 1.1x that, so it must do exactly what its rounding design says.
C4_DA_FACTOR = 1.1
HALF_BARS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "ssd_half_composition_errors.json")))["cases"]
HALF_NAME = {torch.bfloat16: "bf16", torch.float16: "fp16"}


def _half_bars(case, dtype, quantities):
    name = HALF_NAME[dtype]
    own = HALF_BARS[case]
    rows = [v for k, v in HALF_BARS.items() if k.startswith(f"matrix {name} ")]
    bars = {}
    for q in quantities:
        if q not in own:
            continue
        base = own[q]
        if not case.startswith("c4 "):
            vals = [v[q] for v in rows if q in v]
            base = max(base, math.sqrt(sum(e * e for e in vals) / len(vals)))
        if q == "dA" and case.startswith("c4 "):
            bars[q] = C4_DA_FACTOR * own["dA kernel rounding"]
        else:
            bars[q] = 1.5 * base
    return bars


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_backward_option_matrix(shape, dtype):
    inputs, dy, dfinal = _inputs(shape, seed=sum(shape) + 3)
    ref = _oracle_grads(inputs, dy, dfinal, True, dtype)
    got = _gpu_grads(inputs, dy, dfinal, True, dtype)
    if dtype == torch.float32:
        _compare(got, ref, GRAD_TOL[dtype], f"{shape} {dtype}")
        return
    case = f"matrix {HALF_NAME[dtype]} " + "x".join(map(str, shape))
    bars = _half_bars(case, dtype, ["d" + k for k in ref])
    for k, r in ref.items():
        _compare({k: got[k]}, {k: r}, bars.get("d" + k, 0.0), f"{shape} {dtype}")


def test_reference_gradient_case():
    """The reference's own gradient check (benchmarks/verify_mamba2_chunk.py:269-290):
    (2, 21, 4, 4, 2, 5), chunk 8, every option, loss sum(y^2) + sum(state^2), fp32
    gradients against float64 autograd of the recurrence, max-relative error 1e-5."""
    shape = (2, 21, 4, 4, 2, 5)
    x, dt, A, B, C = _problem(*shape, seed=13)
    opt = _options(2, 21, 4, 4, 5, seed=14)

    def grads(device, dtype, fn):
        leaves = [t.to(device, dtype).requires_grad_(True) for t in (x, dt, A, B, C)]
        kw = {k: v.to(device, dtype).requires_grad_(True) for k, v in opt.items()}
        y, s = fn(*leaves, D=kw["D"], z=kw["z"], dt_bias=kw["dt_bias"], dt_softplus=True,
                  initial_states=kw["initial_states"])
        loss = (y * y).sum() + (s * s).sum()
        return torch.autograd.grad(loss, (*leaves, kw["D"], kw["z"], kw["dt_bias"], kw["initial_states"]))

    fast = grads(DEV, torch.float32, lambda *a, **k: _api()(*a[:5], 8, **k))
    slow = grads("cpu", torch.float64, oracle.mamba2_chunk_scan_recurrence)
    for name, got, ref in zip(("x", "dt", "A", "B", "C", "D", "z", "dt_bias", "init"), fast, slow):
        err = record("reference gradient case", "d" + name + " (max rel)", max_rel(got, ref), 1e-5)
        assert err <= 1e-5, f"grad {name}: {err:.3e}"


@pytest.mark.parametrize("case", [
    dict(options=()),
    dict(options=("D",), d_row=True),
    dict(options=("z",)),
    dict(options=("dt_bias",), softplus=False),
    dict(options=("initial_states",), dfinal=False),
    dict(options=("D", "z"), dy=False),
    dict(options=("D", "z", "dt_bias", "initial_states"), d_row=True, softplus=False),
], ids=lambda c: "-".join(c["options"]) + ("-row" if c.get("d_row") else "") +
       ("-nosp" if c.get("softplus") is False else "") + ("-nodfin" if c.get("dfinal") is False else "") +
       ("-nody" if c.get("dy") is False else ""))
def test_backward_each_option(case):
    shape = (2, 150, 4, 5, 2, 3)
    inputs, dy, dfinal = _inputs(shape, seed=5, options=case["options"], d_row=case.get("d_row", False))
    if not case.get("softplus", True):
        inputs["dt"] = inputs["dt"].abs() * 0.2 + 0.3
    dy = dy if case.get("dy", True) else None
    dfinal = dfinal if case.get("dfinal", True) else None
    ref = _oracle_grads(inputs, dy, dfinal, case.get("softplus", True))
    got = _gpu_grads(inputs, dy, dfinal, case.get("softplus", True), torch.float32)
    _compare(got, ref, 1e-4, str(case))


@pytest.mark.parametrize("shape", [(2, 300, 8, 64, 2, 64),     # 128-token chunks, one d_state tile
                                   (1, 1100, 4, 64, 1, 128)],  # 256-token chunks at d_state 128
                         ids=lambda s: "x".join(map(str, s)))
def test_backward_deterministic_and_graph_free_outputs(shape):
    inputs, dy, dfinal = _inputs(shape, seed=9)
    a = _gpu_grads(inputs, dy, dfinal, True, torch.bfloat16)
    b = _gpu_grads(inputs, dy, dfinal, True, torch.bfloat16)
    for k in a:
        assert torch.equal(a[k], b[k]), k


TWO_STREAM_SHAPES = [(2, 300, 8, 64, 2, 64), (1, 1100, 4, 64, 1, 128)]


def test_backward_from_two_host_threads():
    """Two host threads run the backward at once, each on its own torch stream, three times
    each.  They share the library's second stream of the device (the C.B^T adjoint runs there),
    and every run matches that problem's single-thread gradients bit for bit."""
    import threading
    cases = [_inputs(s, seed=20 + i) for i, s in enumerate(TWO_STREAM_SHAPES)]
    serial = [_gpu_grads(*c, True, torch.bfloat16) for c in cases]
    torch.cuda.synchronize()
    results, errors = [None, None], []

    def work(i):
        try:
            st = torch.cuda.Stream()
            with torch.cuda.stream(st):
                runs = [_gpu_grads(*cases[i], True, torch.bfloat16) for _ in range(3)]
            st.synchronize()
            results[i] = runs
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not errors, errors
    for i, runs in enumerate(results):
        assert runs is not None, f"thread {i} did not finish"
        for r, got in enumerate(runs):
            for k, v in serial[i].items():
                assert torch.equal(got[k], v), f"{TWO_STREAM_SHAPES[i]} run {r}: d{k}"


def test_backward_under_graph_capture():
    """A forward and backward captured into a graph: under capture the library keeps the whole
    backward on the capturing stream.  Each of three replays, with eager runs of the same step
    in between, gives the eager gradients bit for bit."""
    inputs, dy, dfinal = _inputs(TWO_STREAM_SHAPES[1], seed=11)
    leaves = _leaves(inputs, DEV, torch.bfloat16)
    dyd, dfd = dy.to(DEV).to(torch.bfloat16), dfinal.to(DEV).to(torch.bfloat16)
    kw = {k: v for k, v in leaves.items() if k not in NAMES}
    order = list(leaves.values())

    def step():
        y, s = _api()(*(leaves[k] for k in NAMES), 64, **kw, dt_softplus=True)
        return torch.autograd.grad((y, s), order, (dyd, dfd))

    eager = [g.clone() for g in step()]
    warm = torch.cuda.Stream()
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(warm)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        again = step()
        torch.cuda.synchronize()
        for name, g, e, a in zip(leaves, captured, eager, again):
            assert torch.equal(g, e), f"replay {r}: d{name}"
            assert torch.equal(a, e), f"eager run after replay {r}: d{name}"


def test_backward_empty_sequence():
    inputs, dy, dfinal = _inputs((2, 0, 4, 6, 2, 5), seed=1)
    got = _gpu_grads(inputs, dy, dfinal, True, torch.float32)
    assert torch.equal(got["initial_states"].cpu(), dfinal.float())
    for k in ("A", "D", "dt_bias"):
        assert torch.count_nonzero(got[k]) == 0, k
    assert got["x"].shape == (2, 0, 4, 6)



NOGATE = (1, 1100, 2, 80, 2, 72)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
def test_backward_without_gate(dtype):
    """Without z, gy is dy itself and the d cs row and column sums (gy . y~ and u . du) carry the
    whole chunk output: the case where two kernels rounding u = step x differently (one of them
    through a single-rounding mixed-precision multiply-add) put the float16 dA 50x above the
    composition's own error.  Every gradient is held to the 16-bit bars (1.5x the composition's
    error on this case, pooled with the matrix's as for the small matrix cases)."""
    inputs, dy, dfinal = _inputs(NOGATE, seed=sum(NOGATE) + 3, options=("D", "dt_bias", "initial_states"))
    ref = _oracle_grads(inputs, dy, dfinal, True, dtype)
    got = _gpu_grads(inputs, dy, dfinal, True, dtype)
    bars = _half_bars(f"nogate {HALF_NAME[dtype]} " + "x".join(map(str, NOGATE)), dtype, ["d" + k for k in ref])
    for k, r in ref.items():
        _compare({k: got[k]}, {k: r}, bars.get("d" + k, 0.0), f"no gate {NOGATE} {dtype}")

def test_config4_backward_prefix():
    """Config 4 geometry (b4 L4096 H64 P64 N128, bf16) with dy zero after 384 tokens and
    no final-state gradient: by causality the exact gradients of the first 384 tokens
    (and of A, D, dt_bias) are those of the 384-token problem, which the oracle runs,
    and every per-token gradient after the prefix is zero."""
    batch, length, nheads, headdim, ngroups, dstate = 4, 4096, 64, 64, 1, 128
    cut = 384
    p = ssd_problem(batch, length, nheads, headdim, ngroups, dstate, seed=4, act=torch.bfloat16, init=False)
    p.pop("initial_states")
    g = torch.Generator().manual_seed(44)
    dy = torch.zeros(batch, length, nheads, headdim, dtype=torch.float64)
    dy[:1, :cut] = torch.randn(1, cut, nheads, headdim, generator=g, dtype=torch.float64)
    leaves = {k: v.detach().to(DEV).requires_grad_(True) for k, v in p.items()}
    kw = {k: leaves[k] for k in ("D", "z", "dt_bias")}
    y, _ = _api()(leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], 256, **kw, dt_softplus=True)
    (y.double() * dy.to(DEV)).sum().backward()
    got = {k: v.grad for k, v in leaves.items()}
    pre = {k: (v[:1, :cut] if k in ("x", "dt", "B", "C", "z") else v).detach().double().requires_grad_(True)
           for k, v in p.items()}
    yr, _ = oracle.mamba2_chunk_scan_composition(
        pre["x"], pre["dt"], pre["A"], pre["B"], pre["C"], chunk_size=128, D=pre["D"], z=pre["z"],
        dt_bias=pre["dt_bias"], dt_softplus=True)
    (yr * dy[:1, :cut]).sum().backward()
    bars = _half_bars("c4 prefix 384", torch.bfloat16, ["d" + k for k in pre])
    over = []
    for k, v in pre.items():
        gk = got[k]
        if k in ("x", "dt", "B", "C", "z"):
            assert torch.count_nonzero(gk[:, cut:]) == 0 and torch.count_nonzero(gk[1:]) == 0, k
            gk = gk[:1, :cut]
        err = record("c4 bwd prefix 384", "d" + k, norm_rel(gk, v.grad), bars["d" + k])
        if err > bars["d" + k]:
            over.append(f"d{k} {err:.3e} > {bars['d' + k]:.3e}")
    assert not over, over


def test_config4_backward_full():
    """Config 4 (b4 L4096 H64 P64 N128, bf16) with the upstream gradient on batch 0 over all
    4096 tokens and a final-state gradient: the whole state-adjoint chain over the 16 chunks
    and the d_final path, against float64 autograd of the composition on batch 0 (batches are
    independent, so the other batches' per-token gradients must be exactly zero and A, D and
    dt_bias take only batch 0's terms)."""
    batch, length, nheads, headdim, ngroups, dstate = 4, 4096, 64, 64, 1, 128
    p = ssd_problem(batch, length, nheads, headdim, ngroups, dstate, seed=4, act=torch.bfloat16, init=False)
    p.pop("initial_states")
    g = torch.Generator().manual_seed(45)
    dy = torch.zeros(batch, length, nheads, headdim, dtype=torch.float64)
    dfinal = torch.zeros(batch, nheads, headdim, dstate, dtype=torch.float64)
    dy[:1] = torch.randn(1, length, nheads, headdim, generator=g, dtype=torch.float64)
    dfinal[:1] = torch.randn(1, nheads, headdim, dstate, generator=g, dtype=torch.float64)
    leaves = {k: v.detach().to(DEV).requires_grad_(True) for k, v in p.items()}
    kw = {k: leaves[k] for k in ("D", "z", "dt_bias")}
    y, s = _api()(leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], 256, **kw, dt_softplus=True)
    ((y.double() * dy.to(DEV)).sum() + (s.double() * dfinal.to(DEV)).sum()).backward()
    got = {k: v.grad for k, v in leaves.items()}
    one = {k: (v[:1] if k in ("x", "dt", "B", "C", "z") else v).detach().double().requires_grad_(True)
           for k, v in p.items()}
    yr, sr = oracle.mamba2_chunk_scan_composition(
        one["x"], one["dt"], one["A"], one["B"], one["C"], chunk_size=256, D=one["D"], z=one["z"],
        dt_bias=one["dt_bias"], dt_softplus=True)
    ((yr * dy[:1]).sum() + (sr * dfinal[:1]).sum()).backward()
    bars = _half_bars("c4 batch 0", torch.bfloat16, ["d" + k for k in one])
    over = []
    for k, v in one.items():
        gk = got[k]
        if k in ("x", "dt", "B", "C", "z"):
            assert torch.count_nonzero(gk[1:]) == 0, k
            gk = gk[:1]
        err = record("c4 bwd batch 0 full", "d" + k, norm_rel(gk, v.grad), bars["d" + k])
        if err > bars["d" + k]:
            over.append(f"d{k} {err:.3e} > {bars['d' + k]:.3e}")
    assert not over, over

def _composition_grads(inputs, dy, dfinal, softplus, dtype):
    """float64 gradients of the oracle's chunked composition (pinned to the recurrence by
    tests/test_oracle.py) on the inputs rounded to the kernel's activation dtype: the
    recurrence's autograd would hold a state per token, too much at these head counts."""
    leaves = _leaves({k: (v.to(dtype) if k in ACTS else v).double() for k, v in inputs.items()}, "cpu")
    fn = lambda x, dt, A, B, C, **kw: oracle.mamba2_chunk_scan_composition(x, dt, A, B, C, 256, **kw)
    return _run_grad(fn, leaves, dy, dfinal, softplus)


# Many heads: at least 256 (batch, head, 64-wide d_head tile) pairs of 16-bit inputs with
# 256-token chunks, two d_head tiles, a ragged state tile, grouped heads and a ragged tail.
MANY_HEAD_SHAPES = [
    (1, 1100, 128, 128, 2, 96),
    (2, 1024, 128, 64, 1, 128),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", MANY_HEAD_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_backward_many_heads(shape, dtype):
    """Every option with the initial-state and final-state gradients at head counts past the
    small matrix, against float64 autograd of the composition; bit-identical run to run."""
    inputs, dy, dfinal = _inputs(shape, seed=sum(shape) + 5, d_row=shape[3] == 64)
    got = _gpu_grads(inputs, dy, dfinal, True, dtype)
    ref = _composition_grads(inputs, dy, dfinal, True, dtype)
    _compare(got, ref, GRAD_TOL[dtype], f"many heads {shape} {dtype}")
    again = _gpu_grads(inputs, dy, dfinal, True, dtype)
    for k in got:
        assert torch.equal(got[k], again[k]), k


# ---------------------------------------------------------------- float64

F64_TOL = 1e-10  # both sides compute in float64; the sums differ only in their order


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_float64_forward_and_backward(shape):
    """float64 inputs, which the reference's composition takes (cv/mamba2_chunk.py:439-440):
    every option, forward and every gradient against the float64 recurrence at 1e-10."""
    inputs, dy, dfinal = _inputs(shape, seed=sum(shape) + 7, d_row=shape[3] % 2 == 0)
    inputs = {k: v.double() for k, v in inputs.items()}
    leaves = _leaves(inputs, DEV)
    kw = {k: leaves[k] for k in leaves if k not in NAMES}
    y, s = _api()(*(leaves[k] for k in NAMES), 64, **kw, dt_softplus=True)
    assert y.dtype == torch.float64 and s.dtype == torch.float64
    ref_leaves = _leaves(inputs, "cpu")
    rkw = {k: ref_leaves[k] for k in ref_leaves if k not in NAMES}
    yr, sr = oracle.mamba2_chunk_scan_recurrence(*(ref_leaves[k] for k in NAMES), **rkw, dt_softplus=True)
    what = f"{shape} float64"
    assert record(what, "y", max_rel(y, yr), F64_TOL) <= F64_TOL
    assert record(what, "final_state", max_rel(s, sr), F64_TOL) <= F64_TOL
    ((y * dy.to(DEV)).sum() + (s * dfinal.to(DEV)).sum()).backward()
    ((yr * dy).sum() + (sr * dfinal).sum()).backward()
    for k in leaves:
        g, r = leaves[k].grad, ref_leaves[k].grad
        assert g.dtype == torch.float64, k
        err = record(what, "d" + k, norm_rel(g, r), F64_TOL)
        assert err <= F64_TOL, f"{what}: d{k} {err:.3e}"


def test_float64_ssd_minimal():
    """The reference verifier's float64 case (benchmarks/verify_mamba2_chunk.py:214-233):
    the scan against the literal ssd_minimal_discrete, chunk 4, with an initial state."""
    import torch.nn.functional as F
    batch, length, nheads, headdim, ngroups, dstate = 1, 16, 2, 3, 1, 4
    g = lambda s: torch.Generator().manual_seed(s)
    x = torch.randn(batch, length, nheads, headdim, generator=g(5), dtype=torch.float64)
    dt = F.softplus(torch.randn(batch, length, nheads, generator=g(6), dtype=torch.float64) - 2)
    A = -torch.exp(torch.rand(nheads, generator=g(7), dtype=torch.float64))
    B = torch.randn(batch, length, ngroups, dstate, generator=g(8), dtype=torch.float64)
    C = torch.randn(batch, length, ngroups, dstate, generator=g(9), dtype=torch.float64)
    init = torch.randn(batch, nheads, headdim, dstate, generator=g(10), dtype=torch.float64) * 0.1
    y_min, s_min = oracle.ssd_minimal_discrete(x * dt.unsqueeze(-1), A * dt, B, C, 4, init[:, None])
    y, s = _api()(*(t.to(DEV) for t in (x, dt, A, B, C)), 4, initial_states=init.to(DEV))
    assert record("ssd_minimal float64", "y", max_rel(y, y_min), F64_TOL) <= F64_TOL
    assert record("ssd_minimal float64", "final_state", max_rel(s, s_min), F64_TOL) <= F64_TOL


def test_float64_errors_and_empty():
    """float64 x takes float64 step sizes and parameters (the wrapper converts them), refuses
    d_state above 256, and an empty sequence returns the initial state."""
    x, dt, A, B, C = (t.double().to(DEV) for t in _problem(1, 8, 2, 4, 1, 300))
    with pytest.raises(RuntimeError, match="d_state"):
        _api()(x, dt, A, B, C)
    x, dt, A, B, C = (t.double().to(DEV) for t in _problem(2, 0, 2, 4, 1, 8))
    init = torch.randn(2, 2, 4, 8, dtype=torch.float64, device=DEV)
    y, s = _api()(x, dt.float(), A.float(), B, C, initial_states=init)
    assert y.shape == x.shape and torch.equal(s, init)


def test_double_backward_is_refused():
    """The backward is hand-written: a second derivative through it raises RuntimeError
    (the reference differentiates its composition, which allows it)."""
    inputs, dy, dfinal = _inputs((1, 40, 2, 8, 1, 8), seed=3)
    leaves = _leaves(inputs, DEV, torch.float32)
    kw = {k: leaves[k] for k in leaves if k not in NAMES}
    y, s = _api()(*(leaves[k] for k in NAMES), 64, **kw, dt_softplus=True)
    (gx,) = torch.autograd.grad((y * dy.to(DEV).float()).sum(), leaves["x"], create_graph=True)
    with pytest.raises(RuntimeError):
        gx.sum().backward()
