"""Measure the reference's own 16-bit SSD arithmetic, the bars of the 16-bit GPU gradient tests.

Run from the repository root: ``python tests/golden/make_ssd_half_bars.py``; writes
``tests/golden/ssd_half_composition_errors.json``.

The reference computes a bf16 (fp16) ``mamba2_chunk_scan`` as a torch composition in that
dtype with float32 step sizes, decay exponents and C.B^T (``cv/mamba2_chunk.py:447-533``) and
takes its gradients by autograd through it (``:653-678``).  ``oracle.mamba2_chunk_scan_composition`` is
that composition, restated and pinned to the float64 recurrence by ``tests/test_oracle.py``.
For each 16-bit gradient case of ``tests/test_ssd_gpu.py`` -- the bf16 and fp16 rows of the
option / shape matrix, one case without the gate, the config-4 causal prefix, and config 4's
batch 0 over all 4096 tokens with a final-state gradient -- this runs the composition in the 16-bit dtype on the case's
inputs (rounded to it where the kernels take it) and records the norm-relative error of every
gradient against float64 autograd on the same rounded inputs: of the recurrence, or at config
4's full length of the float64 composition (which tests/test_oracle.py pins to the
recurrence; the recurrence's autograd would hold 4096 states).  The GPU tests then hold each gradient to a multiple of this error: the error the
reference's own arithmetic makes on the same problem.  For the two config-4 cases it also
records the dA error that the HIP kernels' own rounding points imply (``kernel_rounding_dA``,
a float64 restatement of where csrc/ssd_bwd.hip rounds), which the config-4 dA bar uses.
"""

import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
from cases import norm_rel, ssd_matrix_inputs, ssd_problem  # noqa: E402

OUT = os.path.join(HERE, "ssd_half_composition_errors.json")
ACTS = ("x", "B", "C", "z", "initial_states")  # the tensors the kernels take in the input dtype
NAMES = ("x", "dt", "A", "B", "C")

# the bf16 rows of SHAPES in tests/test_ssd_gpu.py and their seeds (sum(shape) + 3)
MATRIX = [
    (2, 13, 4, 6, 2, 5),
    (1, 16, 4, 4, 1, 4),
    (2, 9, 4, 3, 4, 3),
    (1, 5, 2, 2, 1, 3),
    (2, 300, 4, 64, 1, 128),
    (1, 1100, 2, 80, 2, 72),
    (1, 1100, 3, 64, 1, 128),
    (1, 1030, 4, 60, 2, 128),
]


NOGATE = (1, 1100, 2, 80, 2, 72)


def _grads(fn, inputs, dy, dfinal):
    leaves = {k: v.detach().clone().requires_grad_(True) for k, v in inputs.items()}
    kw = {k: v for k, v in leaves.items() if k not in NAMES}
    y, s = fn(*(leaves[k] for k in NAMES), **kw)
    loss = 0
    if dy is not None:
        loss = loss + (y.double() * dy).sum()
    if dfinal is not None:
        loss = loss + (s.double() * dfinal).sum()
    loss.backward()
    return {k: v.grad for k, v in leaves.items()}


def errors(inputs, dy, dfinal, chunk, dtype=torch.bfloat16, reference="recurrence"):
    """Norm-relative errors of the 16-bit composition's gradients against float64 autograd of
    the recurrence (or the composition), both on the inputs rounded to ``dtype``."""
    rounded = {k: (v.to(dtype) if k in ACTS else v.float()) for k, v in inputs.items()}
    low = _grads(lambda *a, **kw: oracle.mamba2_chunk_scan_composition(*a, chunk, **kw, dt_softplus=True),
                 rounded, dy, dfinal)
    if reference == "recurrence":
        ref = lambda *a, **kw: oracle.mamba2_chunk_scan_recurrence(*a, **kw, dt_softplus=True)
    else:
        ref = lambda *a, **kw: oracle.mamba2_chunk_scan_composition(*a, chunk, **kw, dt_softplus=True)
    f64 = _grads(ref, {k: v.double() for k, v in rounded.items()}, dy, dfinal)
    return {"d" + k: norm_rel(low[k], f64[k]) for k in f64}


def kernel_rounding_dA(inp, dy, dfinal, q, dtype):
    """dA as the HIP kernels' rounding points determine it, in float64 elsewhere.

    The 16-bit SSD backward of csrc/ssd_bwd.hip rounds to ``dtype`` exactly these values (each
    an fp32 value in the kernels, exact here): u = step x, C.B^T, K = C.B^T e^{cs_l - cs_s},
    the local states and their operand e^{T - cs_s} step x, the entering states S_in,
    gy = dy silu(z), the local adjoint and its operand e^{cs_l} gy, and the state adjoints G.
    From them it forms, per token, ya = gy . y~ and ut = u . du (row and column sums of the
    same rounded operands), tau = u . du_state and dT = e^T <G, S_in>, and dA = sum step *
    (reverse cumulative sum of ya - ut, with sum tau + dT at each chunk's last token).  The
    GPU's workspace values match this restatement token for token, so the difference between
    its dA and the reference's is the kernels' rounding design, not a defect."""
    f64 = torch.float64
    R = lambda t: t.to(dtype).to(f64)
    x, B, C, z = inp["x"], inp["B"], inp["C"], inp.get("z")
    b, L, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    nc = -(-L // q)
    pad = lambda t: torch.cat([t, t.new_zeros(t.shape[0], nc * q - L, *t.shape[2:])], 1)
    dl = pad(torch.nn.functional.softplus(inp["dt"] + inp["dt_bias"]))
    cs = (dl * inp["A"]).view(b, nc, q, H).cumsum(2)
    T = cs[:, :, -1]
    X = pad(x).view(b, nc, q, H, P)
    Bc = pad(B).repeat_interleave(H // G, 2).view(b, nc, q, H, N)
    Cc = pad(C).repeat_interleave(H // G, 2).view(b, nc, q, H, N)
    step = dl.view(b, nc, q, H)
    u = R(step[..., None] * X)
    w = torch.exp(T[:, :, None] - cs)
    local = R(torch.einsum("bclhp,bclhn->bchpn", R(w[..., None] * X * step[..., None]), Bc))
    S = torch.zeros(b, nc + 1, H, P, N, dtype=f64)
    if inp.get("initial_states") is not None:
        S[:, 0] = inp["initial_states"]
    for c in range(nc):
        S[:, c + 1] = torch.exp(T[:, c])[..., None, None] * S[:, c] + local[:, c]
    S = R(S)
    cst = cs.permute(0, 1, 3, 2)
    tri = torch.tril(torch.ones(q, q, dtype=torch.bool))
    K = R(torch.where(tri, torch.exp(cst[..., :, None] - cst[..., None, :]) * R(torch.einsum("bclhn,bcshn->bchls", Cc, Bc)), 0.0))
    yt = torch.einsum("bchls,bcshp->bclhp", K, u) + torch.exp(cs)[..., None] * torch.einsum("bclhn,bchpn->bclhp", Cc, S[:, :nc])
    dyc = pad(dy).view(b, nc, q, H, P)
    gy = R(dyc * pad(z).view(b, nc, q, H, P) * torch.sigmoid(pad(z).view(b, nc, q, H, P))) if z is not None else dyc
    adj = R(torch.einsum("bclhp,bclhn->bchpn", R(torch.exp(cs)[..., None] * gy), Cc))
    Gs = torch.zeros(b, nc, H, P, N, dtype=f64)
    dT = torch.zeros(b, nc, H, dtype=f64)
    g = dfinal.clone() if dfinal is not None else torch.zeros(b, H, P, N, dtype=f64)
    for c in reversed(range(nc)):
        Gs[:, c] = g
        dT[:, c] = torch.exp(T[:, c]) * (g * S[:, c]).sum((-1, -2))
        g = adj[:, c] + torch.exp(T[:, c])[..., None, None] * g
    du_state = w[..., None] * torch.einsum("bcshn,bchpn->bcshp", Bc, R(Gs))
    du = torch.einsum("bchls,bclhp->bcshp", K, gy) + du_state
    dcs = (gy * yt).sum(-1) - (u * du).sum(-1)
    dcs[:, :, -1] += (u * du_state).sum(-1).sum(2) + dT
    rcs = dcs.flip(2).cumsum(2).flip(2)
    return (step * rcs).sum((0, 1, 2))


def _dA_ref(inputs, dy, dfinal, chunk, dtype, reference):
    rounded = {k: (v.to(dtype) if k in ACTS else v.float()).double() for k, v in inputs.items()}
    if reference == "recurrence":
        ref = lambda *a, **kw: oracle.mamba2_chunk_scan_recurrence(*a, **kw, dt_softplus=True)
    else:
        ref = lambda *a, **kw: oracle.mamba2_chunk_scan_composition(*a, chunk, **kw, dt_softplus=True)
    return rounded, _grads(ref, rounded, dy, dfinal)["A"]


def kernel_rounding_error(inputs, dy, dfinal, chunk, dtype=torch.bfloat16, reference="recurrence"):
    """Norm-relative error of kernel_rounding_dA against the float64 reference's dA, with the
    upstream gradient rounded to ``dtype`` as the kernels receive it."""
    rounded, ref = _dA_ref(inputs, dy, dfinal, chunk, dtype, reference)
    got = kernel_rounding_dA(rounded, dy.to(dtype).double(), dfinal, chunk, dtype)
    return norm_rel(got, ref)


def main():
    torch.set_num_threads(os.cpu_count() or 1)
    table = {}
    for dtype, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        for shape in MATRIX:
            inputs, dy, dfinal = ssd_matrix_inputs(shape, seed=sum(shape) + 3)
            key = f"matrix {name} " + "x".join(map(str, shape))
            table[key] = errors(inputs, dy, dfinal, 64, dtype)
            print(key, table[key], flush=True)
    # without the gate (test_backward_without_gate): gy is dy itself, the case whose float16 dA a
    # kernel rounding u differently on the two sides of the d cs cancellation put at 50x this error
    for dtype, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        shape = NOGATE
        inputs, dy, dfinal = ssd_matrix_inputs(shape, seed=sum(shape) + 3, options=("D", "dt_bias", "initial_states"))
        key = f"nogate {name} " + "x".join(map(str, shape))
        table[key] = errors(inputs, dy, dfinal, 64, dtype)
        print(key, table[key], flush=True)
    # the config-4 causal prefix of test_config4_backward_prefix: batch 0, 384 tokens
    p = ssd_problem(4, 4096, 64, 64, 1, 128, seed=4, act=torch.bfloat16, init=False)
    p.pop("initial_states")
    g = torch.Generator().manual_seed(44)
    cut = 384
    dy = torch.randn(1, cut, 64, 64, generator=g, dtype=torch.float64)
    pre = {k: (v[:1, :cut] if k in ("x", "dt", "B", "C", "z") else v) for k, v in p.items()}
    table["c4 prefix 384"] = errors(pre, dy, None, 256)
    table["c4 prefix 384"]["dA kernel rounding"] = kernel_rounding_error(pre, dy, None, 256)
    print("c4 prefix", table["c4 prefix 384"], flush=True)
    # config 4, batch 0, all 4096 tokens, with a final-state gradient (test_config4_backward_full)
    g = torch.Generator().manual_seed(45)
    dy = torch.randn(1, 4096, 64, 64, generator=g, dtype=torch.float64)
    dfinal = torch.randn(1, 64, 64, 128, generator=g, dtype=torch.float64)
    one = {k: (v[:1] if k in ("x", "dt", "B", "C", "z") else v) for k, v in p.items()}
    table["c4 batch 0"] = errors(one, dy, dfinal, 256, reference="composition")
    table["c4 batch 0"]["dA kernel rounding"] = kernel_rounding_error(one, dy, dfinal, 256, reference="composition")
    print("c4 batch 0", table["c4 batch 0"], flush=True)
    with open(OUT, "w") as f:
        json.dump({"source": "tests/golden/make_ssd_half_bars.py", "metric": "norm-relative gradient error of "
                   "the 16-bit composition (oracle.mamba2_chunk_scan_composition) against float64 autograd of "
                   "the recurrence, on the same bf16-rounded inputs; 'dA kernel rounding': the same error of the dA "
                   "that the HIP kernels' rounding points imply (kernel_rounding_dA)", "cases": table}, f, indent=1, sort_keys=True)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
