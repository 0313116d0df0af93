"""The measurements behind the 16-bit SSD gradient bars (tests/golden/make_ssd_half_bars.py).

The bars of the 16-bit GPU tests are multiples of errors that the generator measured and
committed in ssd_half_composition_errors.json.  Here the generator's pieces are pinned on the
CPU: its restatement of the kernels' rounding points reduces to the exact gradient when no
rounding happens (float64), and a fixture row is reproduced from scratch.
"""
import importlib.util
import json
import os

import pytest
import torch

import oracle
from cases import norm_rel, ssd_matrix_inputs

HERE = os.path.dirname(os.path.abspath(__file__))
spec = importlib.util.spec_from_file_location("make_ssd_half_bars", os.path.join(HERE, "golden", "make_ssd_half_bars.py"))
bars = importlib.util.module_from_spec(spec)
spec.loader.exec_module(bars)
FIXTURE = json.load(open(os.path.join(HERE, "golden", "ssd_half_composition_errors.json")))


@pytest.mark.parametrize("shape,q", [((1, 40, 3, 5, 1, 6), 16), ((2, 37, 4, 3, 2, 4), 8)])
@pytest.mark.parametrize("with_z,with_final,with_init", [(True, True, True), (False, True, False), (True, False, False)])
def test_kernel_rounding_dA_without_rounding_is_the_exact_gradient(shape, q, with_z, with_final, with_init):
    """With float64 'rounding' (none), the restated kernel decomposition -- row and column
    sums ya - ut, tau and dT at each chunk's end, the reverse cumulative sum -- gives the
    float64 recurrence's dA: the decomposition itself is exact, so what it reports at 16 bits
    is the rounding alone.  Ragged tails (40 = 2 x 16 + 8, 37 = 4 x 8 + 5), gate on and off,
    final-state gradient and initial state on and off."""
    opts = ("D", "dt_bias") + (("z",) if with_z else ()) + (("initial_states",) if with_init else ())
    inputs, dy, dfinal = ssd_matrix_inputs(shape, seed=sum(shape), options=opts)
    inputs = {k: v.double() for k, v in inputs.items()}
    leaves = {k: v.clone().requires_grad_(True) for k, v in inputs.items()}
    kw = {k: leaves[k] for k in leaves if k not in ("x", "dt", "A", "B", "C")}
    y, s = oracle.mamba2_chunk_scan_recurrence(leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"],
                                               **kw, dt_softplus=True)
    loss = (y * dy).sum() + ((s * dfinal).sum() if with_final else 0)
    loss.backward()
    got = bars.kernel_rounding_dA(inputs, dy, dfinal if with_final else None, q, torch.float64)
    assert norm_rel(got, leaves["A"].grad) < 1e-10


def test_kernel_rounding_dA_sees_a_dropped_rounding():
    """At bf16 the restatement's dA differs from the exact one, and by more when C.B^T is
    rounded than when it is not -- a rounding point that the restatement silently skipped
    would fail this."""
    shape = (1, 64, 4, 8, 1, 16)
    inputs, dy, dfinal = ssd_matrix_inputs(shape, seed=5, options=("D", "z", "dt_bias"))
    exact = bars.kernel_rounding_dA({k: v.double() for k, v in inputs.items()}, dy, dfinal, 32, torch.float64)
    half = bars.kernel_rounding_dA({k: v.double() for k, v in inputs.items()}, dy, dfinal, 32, torch.bfloat16)
    assert 1e-5 < norm_rel(half, exact) < 5e-2


def test_fixture_row_is_reproduced():
    """The smallest bf16 matrix row of the committed fixture, measured again."""
    shape = (1, 5, 2, 2, 1, 3)
    inputs, dy, dfinal = ssd_matrix_inputs(shape, seed=sum(shape) + 3)
    got = bars.errors(inputs, dy, dfinal, 64, torch.bfloat16)
    want = FIXTURE["cases"]["matrix bf16 " + "x".join(map(str, shape))]
    assert set(got) == set(want)
    for k, v in want.items():
        assert abs(got[k] - v) <= 1e-12 + 1e-9 * v, k
