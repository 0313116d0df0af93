"""The committed golden fixtures are what the (pinned) oracle computes."""

import os

import numpy as np
import torch

import oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(HERE, name))


def _inputs(data):
    return {k[3:]: torch.from_numpy(data[k]).double() for k in data.files if k.startswith("in_")}


def test_mamba1_fixture():
    data = _load("mamba1_c1.npz")
    out = oracle.selective_scan(**_inputs(data), delta_softplus=True)
    assert np.allclose(out.numpy(), data["out"], rtol=0, atol=1e-12)


def test_ssd_fixture():
    data = _load("ssd_small.npz")
    y, s = oracle.mamba2_chunk_scan_recurrence(**_inputs(data), dt_softplus=True)
    assert np.allclose(y.numpy(), data["y"], rtol=0, atol=1e-12)
    assert np.allclose(s.numpy(), data["final_state"], rtol=0, atol=1e-12)


def test_decode_fixture():
    data = _load("decode_small.npz")
    y, s = oracle.mamba2_state_update(**_inputs(data), dt_softplus=True)
    assert np.allclose(y.numpy(), data["y"], rtol=0, atol=1e-12)
    assert np.allclose(s.numpy(), data["new_state"], rtol=0, atol=1e-12)
