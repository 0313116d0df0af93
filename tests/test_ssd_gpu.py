"""Mamba-2 SSD chunk scan: HIP kernels against the float64 CPU oracle.

Option/shape matrix follows the reference verifier (benchmarks/verify_mamba2_chunk.py:
113-179, 237-290): grouped heads, D (H,) and (H,P), z, dt_bias, softplus,
initial states, ragged lengths, chunk sizes larger than the sequence.
Tolerances (reference and north star): fp32 1e-5, fp16 2e-3, bf16 2e-2 max
relative error; gradient norms 1e-4 (fp32).
"""

import numpy as np
import os
import pytest
import torch

import oracle
from cases import max_rel, norm_rel, ssd_problem

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
    assert max_rel(y, y_ref) <= TOL[dtype], f"y {max_rel(y, y_ref):.3e}"
    assert max_rel(s, s_ref) <= TOL[dtype], f"state {max_rel(s, s_ref):.3e}"


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
    assert max_rel(y[:1], y_ref) <= 2e-2
    assert max_rel(s[:1], s_ref) <= 2e-2
    assert torch.isfinite(y).all() and torch.isfinite(s).all()
