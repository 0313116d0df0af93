#!/usr/bin/env python
"""Benchmark of the SSM scan hot path on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints one JSON line.

Headline (``value``): the Mamba-1 selective scan forward+backward at the 2.8B-layer
shape (batch 4, d_inner 5120, seqlen 4096, d_state 16, ngroups 1; u/z/B/C bf16,
delta fp32, fp32 scan state), as whole-job algorithmic GB/s: the bytes of every
input read once and every output written once per pass (fwd 839.9 MB + bwd
1512.1 MB per step), divided by the measured time per step.  A step is one
forward and one backward over the same synthetic batch, inputs resident in HBM.

``roofline`` describes the dominant kernel of the timed region: its algorithmic
bytes per launch over its average launch time, both measured live with HIP events
recorded by libmko on the kernel's own stream.  ``cpu_baseline`` times the float64
oracle's restatement (run in float32 with autograd) on a bounded sample on this
host.  ``also`` carries the other workloads of the path (Mamba-1 130M layer,
Mamba-2 decode, Mamba-2 SSD chunk scan when present) with their own rooflines.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "metal-kernelops_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
METRIC = "selective-scan fwd+bwd GB/s (% HBM peak); Mamba-2 SSD tokens/s (% MFMA peak)"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def mamba1_bytes(batch, dim, length, dstate, groups, act=2, delta=4):
    """Algorithmic bytes (fwd, bwd) of one selective-scan step, per the survey's count."""
    e = batch * dim * length
    bc = batch * groups * dstate * length
    fwd = e * (act + delta + act + act) + 2 * bc * act          # u, delta, z in; out; B, C in
    bwd = e * (act + delta + act + act + act + delta + act) + 4 * bc * act  # + dout in; du, ddelta, dz; dB, dC
    return fwd, bwd


def timed(step, steps, warmup):
    """ms per step over `steps` after `warmup`, then per-kernel HIP-event times.

    The headline loop runs with the library's kernel timing off; a second loop of
    the same length runs with it on, for the per-kernel figures.
    """
    from metal_kernelops import _native as nat
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ms = start.elapsed_time(stop) / steps
    nat.kernel_timing_reset()
    nat.kernel_timing(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    nat.kernel_timing(False)
    return ms, wall, nat.kernel_times()


def dominant(kernels):
    name = max(kernels, key=lambda k: kernels[k][0])
    total, count = kernels[name]
    return name, total / max(count, 1), count


def roofline(bytes_per_launch, avg_ms, traffic=None):
    achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic}


def load_traffic(name):
    """HBM bytes per launch from a committed PMC summary (profiles/traffic.json), if any."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(name)


# --------------------------------------------------------------------- Mamba-1


def mamba1_case(batch, dim, length, steps, warmup, seed=0):
    from cases import mamba1_layer
    from metal_kernelops import selective_scan
    inputs, dout = mamba1_layer(batch, dim, length, seed=seed)
    dev = torch.device("cuda")
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in inputs.items()}
    dout = dout.to(dev)
    order = list(leaves.values())

    def step():
        out = selective_scan(**leaves, delta_softplus=True)
        torch.autograd.grad(out, order, dout)

    ms, wall, kernels = timed(step, steps, warmup)
    fwd_b, bwd_b = mamba1_bytes(batch, dim, length, 16, 1)
    name, avg, count = dominant(kernels)
    per_kernel = {"selscan_bwd_main": bwd_b, "selscan_fwd_replay": fwd_b}
    roof = roofline(per_kernel.get(name, fwd_b + bwd_b), avg, load_traffic(f"{name}@{batch}x{dim}x{length}"))
    roof["kernel"] = name
    roof["algorithmic_bytes"] = per_kernel.get(name, fwd_b + bwd_b)
    del leaves, dout
    torch.cuda.empty_cache()
    return {
        "ms_per_step": ms, "wall_ms_per_step": wall, "gbs": (fwd_b + bwd_b) / (ms * 1e-3) / 1e9,
        "bytes_per_step": fwd_b + bwd_b, "roofline": roof,
        "kernels_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in sorted(kernels.items())},
    }


def mamba1_cpu_baseline(batch=1, dim=256, length=2048):
    """The oracle's per-timestep recurrence in float32 with autograd on the host cores."""
    import oracle
    from cases import mamba1_layer
    torch.set_num_threads(os.cpu_count() or 1)
    inputs, dout = mamba1_layer(batch, dim, length, seed=0, act=torch.float32)
    leaves = {k: v.float().requires_grad_(True) for k, v in inputs.items()}

    def run():
        out = oracle.selective_scan(**leaves, delta_softplus=True, dtype=torch.float32)
        torch.autograd.grad(out, list(leaves.values()), dout.float())

    run()  # warm-up
    best = None
    for _ in range(2):
        t0 = time.perf_counter()
        run()
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    fwd_b, bwd_b = mamba1_bytes(batch, dim, length, 16, 1)
    return {"value": round((fwd_b + bwd_b) / best / 1e9, 6), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"Mamba-1 fwd+bwd, batch {batch} x dim {dim} x seqlen {length}, d_state 16, "
                      f"float32 per-step recurrence with autograd (oracle/ssm.py), best of 2 after "
                      f"1 warm-up: {best:.2f} s per step"}


# --------------------------------------------------------------------- decode


def decode_case(steps=1024, warmup=16):
    from cases import decode_problem
    from metal_kernelops.cv import mamba2_state_update
    dev = torch.device("cuda")
    p = decode_problem(256, 80, 64, 128, 1, seed=0)
    state = p["state"].to(dev)
    ring = []
    for i in range(8):  # per-step x, dt, B, C, z from a seeded ring of 8
        g = torch.Generator().manual_seed(100 + i)
        ring.append({"x": torch.randn(256, 80, 64, generator=g).bfloat16().to(dev),
                     "dt": torch.randn(256, 80, generator=g).to(dev),
                     "B": torch.randn(256, 1, 128, generator=g).bfloat16().to(dev),
                     "C": torch.randn(256, 1, 128, generator=g).bfloat16().to(dev),
                     "z": torch.randn(256, 80, 64, generator=g).bfloat16().to(dev)})
    A, D, bias = p["A"].to(dev), p["D"].to(dev), p["dt_bias"].to(dev)
    it = [0]

    def step():
        r = ring[it[0] % 8]
        it[0] += 1
        mamba2_state_update(state, r["x"], r["dt"], A, r["B"], r["C"], D=D, z=r["z"], dt_bias=bias,
                            dt_softplus=True, out_state=state)

    with torch.no_grad():
        ms, wall, kernels = timed(step, steps, warmup)
    rmw = 2 * state.numel() * 4
    other = 256 * 80 * 64 * 2 * 3 + 256 * 128 * 2 * 2 + 256 * 80 * 4
    name, avg, count = dominant(kernels)
    roof = roofline(rmw + other, avg, load_traffic(f"{name}@256x80x64x128"))
    roof["kernel"] = name
    roof["algorithmic_bytes"] = rmw + other
    del state, ring
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "wall_ms_per_step": wall, "steps": steps,
            "state_rmw_gbs": rmw / (ms * 1e-3) / 1e9, "roofline": roof,
            "kernels_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in sorted(kernels.items())}}


def decode_cpu_baseline(steps=4):
    import oracle
    from cases import decode_problem
    torch.set_num_threads(os.cpu_count() or 1)
    p = decode_problem(256, 80, 64, 128, 1, seed=0)
    p = {k: v.float() for k, v in p.items()}
    state = p.pop("state")
    oracle.mamba2_state_update(state, **p, dt_softplus=True, dtype=torch.float32)
    t0 = time.perf_counter()
    for _ in range(steps):
        _, state = oracle.mamba2_state_update(state, **p, dt_softplus=True, dtype=torch.float32)
    per = (time.perf_counter() - t0) / steps
    return {"value": round(2 * state.numel() * 4 / per / 1e9, 4), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"decode step at the config-5 shape in float32 (oracle/ssm.py), {steps} steps, "
                      f"{per * 1e3:.1f} ms per step"}


# --------------------------------------------------------------------- main


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--only", choices=["mamba1", "decode", "all"], default="all")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    torch.backends.cuda.matmul.allow_tf32 = False

    log("mamba1 config 3 (4x5120x4096) fwd+bwd")
    head = mamba1_case(4, 5120, 4096, args.steps, args.warmup)
    log(f"  {head['ms_per_step']:.3f} ms/step, {head['gbs']:.1f} GB/s; kernels {head['kernels_ms']}")
    also = {}
    if args.only == "all":
        log("mamba1 config 2 (8x1536x2048) fwd+bwd")
        c2 = mamba1_case(8, 1536, 2048, args.steps, args.warmup)
        also["mamba1_130m_layer_fwd_bwd"] = {
            "value": round(c2["gbs"], 1), "unit": "GB/s", "ms_per_step": round(c2["ms_per_step"], 4),
            "config": {"batch": 8, "dim": 1536, "seqlen": 2048, "dstate": 16, "ngroups": 1},
            "roofline": c2["roofline"], "kernels_ms": c2["kernels_ms"]}
        log(f"  {c2['ms_per_step']:.3f} ms/step, {c2['gbs']:.1f} GB/s")
        log("mamba2 decode config 5 (256x80x64x128), 1024 in-place steps")
        dec = decode_case()
        also["mamba2_decode_state_rmw"] = {
            "value": round(dec["state_rmw_gbs"], 1), "unit": "GB/s",
            "ms_per_step": round(dec["ms_per_step"], 5), "steps": dec["steps"],
            "config": {"batch": 256, "nheads": 80, "headdim": 64, "dstate": 128, "ngroups": 1,
                       "state_dtype": "f32", "io_dtype": "bf16"},
            "roofline": dec["roofline"], "kernels_ms": dec["kernels_ms"]}
        log(f"  {dec['ms_per_step'] * 1e3:.1f} us/step, {dec['state_rmw_gbs']:.1f} GB/s state RMW")
    cpu = None
    if not args.skip_cpu:
        log("cpu baseline (mamba1 sample)")
        cpu = mamba1_cpu_baseline()
        log(f"  {cpu['sample']}")
        if "mamba2_decode_state_rmw" in also:
            also["mamba2_decode_state_rmw"]["cpu_baseline"] = decode_cpu_baseline()
    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "mamba1_selective_scan_fwd_bwd_2.8b_layer", "batch": 4, "dim": 5120,
                   "seqlen": 4096, "dstate": 16, "ngroups": 1, "io_dtype": "bf16",
                   "delta_dtype": "f32", "state_dtype": "f32",
                   "hbm_frac_whole_step": round(head["gbs"] / HBM_PEAK_GBS, 4)},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "kernels_ms": head["kernels_ms"],
        "also": also,
        "torch": torch.__version__,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
