"""Write the golden fixtures under tests/golden/ from the float64 CPU oracle.

Run from the repository root: ``python tests/golden/make_golden.py``.  Each
fixture holds the seeded inputs (as float32, exactly what the GPU tests feed the
kernels), the upstream gradient, and the oracle's float64 outputs and input
gradients.  The reference repository ships no fixtures for this path, so these
freeze the oracle's answers (pinned by tests/test_oracle.py) for the GPU tests.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
from cases import decode_problem, mamba1_c1, ssd_problem  # noqa: E402

F64 = torch.float64


def _grads(fn, inputs, seeds):
    leaves = {k: (None if v is None else v.double().requires_grad_(True)) for k, v in inputs.items()}
    outs = fn(leaves)
    outs = outs if isinstance(outs, tuple) else (outs,)
    loss = sum((o * s.double()).sum() for o, s in zip(outs, seeds))
    loss.backward()
    return [o.detach() for o in outs], {k: v.grad for k, v in leaves.items() if v is not None}


def mamba1():
    inputs, dy = mamba1_c1()
    outs, grads = _grads(lambda t: oracle.selective_scan(**t, delta_softplus=True), inputs, [dy])
    data = {"in_" + k: v.numpy().astype(np.float32) for k, v in inputs.items()}
    data["dy"] = dy.numpy().astype(np.float32)
    data["out"] = outs[0].numpy()
    data.update({"grad_" + k: v.numpy() for k, v in grads.items()})
    np.savez_compressed(os.path.join(HERE, "mamba1_c1.npz"), **data)


def ssd():
    inputs = ssd_problem(2, 13, 4, 6, 2, 5, seed=3)
    g = torch.Generator().manual_seed(4)
    dy = torch.randn(2, 13, 4, 6, generator=g)
    dfinal = torch.randn(2, 4, 6, 5, generator=g)
    outs, grads = _grads(lambda t: oracle.mamba2_chunk_scan_recurrence(**t, dt_softplus=True),
                         inputs, [dy, dfinal])
    data = {"in_" + k: v.numpy().astype(np.float32) for k, v in inputs.items()}
    data.update(dy=dy.numpy(), dfinal=dfinal.numpy(), y=outs[0].numpy(), final_state=outs[1].numpy())
    data.update({"grad_" + k: v.numpy() for k, v in grads.items()})
    np.savez_compressed(os.path.join(HERE, "ssd_small.npz"), **data)


def decode():
    inputs = decode_problem(2, 4, 6, 16, 2, seed=5, act=torch.float32)
    g = torch.Generator().manual_seed(6)
    dy = torch.randn(2, 4, 6, generator=g)
    dstate = torch.randn(2, 4, 6, 16, generator=g)
    outs, grads = _grads(lambda t: oracle.mamba2_state_update(**t, dt_softplus=True), inputs, [dy, dstate])
    data = {"in_" + k: v.numpy().astype(np.float32) for k, v in inputs.items()}
    data.update(dy=dy.numpy(), dstate=dstate.numpy(), y=outs[0].numpy(), new_state=outs[1].numpy())
    data.update({"grad_" + k: v.numpy() for k, v in grads.items()})
    np.savez_compressed(os.path.join(HERE, "decode_small.npz"), **data)


if __name__ == "__main__":
    mamba1()
    ssd()
    decode()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
