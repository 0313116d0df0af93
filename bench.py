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
Mamba-2 decode, Mamba-2 SSD chunk scan, the four-path 2D scan, the causal conv1d
ahead of the scan, the gated RMSNorm after it, and the integration verifier's blocks with a
Mamba-2 2.7B layer) with their own rooflines where a kernel dominates.
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
# Vector ALU issue: 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz, one wave64 instruction per SIMD per
# 4 cycles (transcendentals take longer, so this is an upper bound for them)
VALU_PEAK_TLANE_OPS = 256 * 4 * 16 * 2.4e9 / 1e12
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


def valu_roofline(name, avg_ms):
    """The dominant kernel against the vector-ALU issue rate: its wave VALU instructions per
    launch (SQ_INSTS_VALU from a committed PMC summary, profiles/valu.json) x 64 lanes over
    its measured launch time."""
    path = os.path.join(ROOT, "profiles", "valu.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        insts = json.load(f).get(name)
    if insts is None:
        return None
    achieved = insts * 64 / (avg_ms * 1e-3) / 1e12
    return {"bound": "valu", "achieved": round(achieved, 2), "peak": round(VALU_PEAK_TLANE_OPS, 2),
            "unit": "T lane-ops/s", "frac": round(achieved / VALU_PEAK_TLANE_OPS, 4),
            "valu_insts_per_launch": insts}


def copy_floor(gib=1.0, runs=20):
    """The part's read-and-write streaming rate in this run: libmko's streaming copy
    (mko_stream_copy) of ``gib`` GiB, with the nontemporal hint (as the decode kernels
    access their state) and without it, ``runs`` timed copies each after 3 warm-ups."""
    from metal_kernelops import _native as nat
    n = int(gib * (1 << 30)) // 4
    src = torch.empty(n, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    out = {"kernel": "mko_stream_copy", "bytes_read": n * 4, "bytes_written": n * 4, "runs": runs}
    for key, nt in (("nontemporal", True), ("plain", False)):
        for _ in range(3):
            nat.stream_copy(src, dst, nt)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(runs):
            nat.stream_copy(src, dst, nt)
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / runs
        gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
        out[key] = {"us": round(ms * 1e3, 1), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if not torch.equal(src, dst):
        raise RuntimeError("mko_stream_copy: the copy differs from its source")
    del src, dst
    torch.cuda.empty_cache()
    out["gbs"] = max(out["nontemporal"]["gbs"], out["plain"]["gbs"])
    return out


def of_copy(gbs, floor):
    """A streaming rate as a fraction of the run's copy floor."""
    return None if floor is None else round(gbs / floor["gbs"], 4)


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
    # each direction's algorithmic bytes belong to its main kernel
    per_kernel = {"selscan_bwd_lane": bwd_b, "selscan_bwd_main": bwd_b, "selscan_fwd_lane": fwd_b,
                  "selscan_fwd_replay": fwd_b}
    tag = f"{name}@{batch}x{dim}x{length}"
    roof = roofline(per_kernel.get(name, fwd_b + bwd_b), avg, load_traffic(tag))
    roof["kernel"] = name
    roof["algorithmic_bytes"] = per_kernel.get(name, fwd_b + bwd_b)
    valu = valu_roofline(tag, avg)
    del leaves, dout
    torch.cuda.empty_cache()
    return {
        "ms_per_step": ms, "wall_ms_per_step": wall, "gbs": (fwd_b + bwd_b) / (ms * 1e-3) / 1e9,
        "bytes_per_step": fwd_b + bwd_b, "roofline": roof, "roofline_valu": valu,
        "kernels_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in sorted(kernels.items())},
    }


def host_cpu():
    """The host's CPU model (lscpu's "Model name"), the cores it reports and the threads torch uses."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}


def mamba1_cpu_baseline(batch, dim, length):
    """The oracle's per-timestep recurrence in float32 on the host cores, forward only, at
    the full layer shape.

    The forward+backward with autograd is out of reach on the host: at config 2 it ran past
    15 minutes on 8 cores, and at config 3 autograd would hold about 16 GB of per-step
    tensors.  So the baseline is the forward at the full shape, one timed run after a
    warm-up over a 256-step prefix, against the forward's algorithmic bytes."""
    import oracle
    from cases import mamba1_layer
    torch.set_num_threads(os.cpu_count() or 1)
    inputs, _ = mamba1_layer(batch, dim, length, seed=0, act=torch.float32)
    inputs = {k: v.float() for k, v in inputs.items()}
    prefix = {k: (v[..., :256].contiguous() if k in ("u", "dt", "z", "B", "C") else v) for k, v in inputs.items()}
    with torch.no_grad():
        oracle.selective_scan(**prefix, delta_softplus=True, dtype=torch.float32)
        t0 = time.perf_counter()
        oracle.selective_scan(**inputs, delta_softplus=True, dtype=torch.float32)
        sec = time.perf_counter() - t0
    fwd_b, _ = mamba1_bytes(batch, dim, length, 16, 1)
    return {"value": round(fwd_b / sec / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", **host_cpu(),
            "sample": f"Mamba-1 forward only at the full {batch} x {dim} x {length} shape (d_state 16), "
                      f"float32 per-step recurrence of oracle/ssm.py on the host, one run after a 256-step "
                      f"warm-up: {sec:.2f} s for {fwd_b / 1e6:.1f} MB of forward algorithmic bytes "
                      f"(forward+backward with autograd does not fit a bench run on the host)"}


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

    # The backward at the same geometry: one step's gradients for every input through
    # autograd (state, x, dt, A, B, C, D, z, dt_bias), timed as forward+backward steps and by
    # the backward kernel's own launches.  It reads the state and the adjoint of the new
    # state and writes the adjoint of the state (fp32), besides the per-token vectors.
    r = ring[0]
    leaves = [state.detach().clone(), r["x"], r["dt"], A, r["B"], r["C"], D, r["z"], bias]
    leaves = [t.detach().clone().requires_grad_(True) for t in leaves]
    g = torch.Generator().manual_seed(7)
    dy = torch.randn(256, 80, 64, generator=g).to(dev)
    dnew = torch.randn(256, 80, 64, 128, generator=g).to(dev)
    st, x, dt, Ap, Bp, Cp, Dp, zp, bp = leaves

    def bstep():
        y, ns = mamba2_state_update(st, x, dt, Ap, Bp, Cp, D=Dp, z=zp, dt_bias=bp, dt_softplus=True)
        torch.autograd.grad((y, ns), leaves, (dy.to(y.dtype), dnew))

    ms_fb, _, kb = timed(bstep, 20, 3)
    bwd_name = "state_update_bwd"
    bwd_ms = kb[bwd_name][0] / max(kb[bwd_name][1], 1)
    bwd_bytes = 3 * state.numel() * 4 + 256 * 80 * 64 * 2 * 5 + 256 * 128 * 2 * 4 + 256 * 80 * 4 * 2
    broof = roofline(bwd_bytes, bwd_ms, load_traffic(f"{bwd_name}@256x80x64x128"))
    broof["kernel"] = bwd_name
    broof["algorithmic_bytes"] = bwd_bytes
    bwd = {"ms_per_fwd_bwd_step": round(ms_fb, 4), "bwd_kernel_ms": round(bwd_ms, 4),
           "bwd_gbs": round(bwd_bytes / (bwd_ms * 1e-3) / 1e9, 1), "bwd_algorithmic_bytes": bwd_bytes,
           "bwd_hbm_frac": round(bwd_bytes / (bwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "roofline": broof,
           "kernels_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in sorted(kb.items())}}
    del state, ring, leaves, dy, dnew
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "wall_ms_per_step": wall, "steps": steps,
            "state_rmw_gbs": rmw / (ms * 1e-3) / 1e9, "roofline": roof, "backward": bwd,
            "kernels_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in sorted(kernels.items())}}


def decode_cpu_baseline(steps=16):
    """The oracle's decode step in float32 on the host cores at the config-5 shape, timed
    over ``steps`` in-place steps after one warm-up step."""
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
            "cores": torch.get_num_threads(), "kind": "port", **host_cpu(),
            "sample": f"decode step at the config-5 shape in float32 (oracle/ssm.py), {steps} steps after "
                      f"1 warm-up, {per * 1e3:.1f} ms per step"}


# --------------------------------------------------------------------- Mamba-2 SSD


def ssd_flops(batch, length, nheads, headdim, ngroups, dstate, q):
    """Algorithmic FLOPs per kernel, causal count: each contraction once, lower triangles only.

    Per token and head: P(Q+1) for the masked scores . X product, 2NP for the chunk
    state and 2NP for C . state; per token and group N(Q+1) for C . B^T.  The backward
    does two gradient contractions per forward one.  ssd_gate is element-wise here: the
    forward saves the chunk output for it when a gradient will be taken.
    """
    tok = batch * length
    P, N, H, G = headdim, dstate, nheads, ngroups
    tri_x = tok * H * P * (q + 1)
    state = tok * H * 2 * N * P
    cb = tok * G * N * (q + 1)
    return {
        "ssd_cb": cb, "ssd_chunk_state": state, "ssd_chunk_scan": tri_x + state,
        "ssd_chunk_state_bwd": state, "ssd_du": tri_x + state, "ssd_dcb": tri_x,
        "ssd_dbc_state": 2 * state, "ssd_dbc_final": 2 * cb,
    }


def ssd_bytes(batch, length, nheads, headdim, ngroups, dstate, act=2):
    """Algorithmic bytes (fwd, bwd): each input read once, each output written once."""
    e = batch * length * nheads * headdim
    bc = batch * length * ngroups * dstate
    dtb = batch * length * nheads * 4
    st = batch * nheads * headdim * dstate * act
    fwd = 3 * e * act + dtb + 2 * bc * act + st                  # x, z in, y out; dt; B, C; final
    bwd = 5 * e * act + 2 * dtb + 4 * bc * act + st              # x, z, dy in; dx, dz out; dt, ddt; B, C, dB, dC; d_final
    return fwd, bwd


def ssd_case(steps, warmup, batch=4, length=4096, nheads=64, headdim=64, ngroups=1, dstate=128, chunk=256):
    from cases import ssd_problem
    from metal_kernelops.cv import mamba2_chunk_scan
    dev = torch.device("cuda")
    p = ssd_problem(batch, length, nheads, headdim, ngroups, dstate, seed=0, act=torch.bfloat16, init=False)
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in p.items() if v is not None}
    g = torch.Generator().manual_seed(1)
    dy = torch.randn(batch, length, nheads, headdim, generator=g).bfloat16().to(dev)
    dfinal = torch.randn(batch, nheads, headdim, dstate, generator=g).bfloat16().to(dev)
    order = list(leaves.values())
    names = ("x", "dt", "A", "B", "C")

    def step():
        y, s = mamba2_chunk_scan(*(leaves[k] for k in names), chunk, D=leaves["D"], z=leaves["z"],
                                 dt_bias=leaves["dt_bias"], dt_softplus=True)
        torch.autograd.grad((y, s), order, (dy, dfinal))

    ms, wall, kernels = timed(step, steps, warmup)
    flops = ssd_flops(batch, length, nheads, headdim, ngroups, dstate, chunk)
    total = sum(flops.values())
    if "ssd_gate_state" in kernels:  # the fused gate carries the local state adjoint's contraction
        flops["ssd_gate_state"] = flops.pop("ssd_chunk_state_bwd")
    fwd_b, bwd_b = ssd_bytes(batch, length, nheads, headdim, ngroups, dstate)
    per = {k: v[0] / max(v[1], 1) for k, v in kernels.items()}
    mfma = {}
    for k, f in flops.items():
        if k in per:
            tf = f / (per[k] * 1e-3) / 1e12
            mfma[k] = {"ms": round(per[k], 4), "gflop": round(f / 1e9, 2), "tflops": round(tf, 1),
                       "frac": round(tf / BF16_PEAK_TFLOPS, 4)}
    name = max((k for k in per if k in flops), key=lambda k: per[k])
    achieved = flops[name] / (per[name] * 1e-3) / 1e12
    traffic = load_traffic(f"{name}@{batch}x{length}x{nheads}x{headdim}x{dstate}")
    roof = {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": traffic,
            "kernel": name, "algorithmic_gflop": round(flops[name] / 1e9, 2)}
    # the same kernel against HBM: its measured bytes per launch (PMC counters) over its time
    roof_hbm = None
    if traffic:
        gbs = traffic / (per[name] * 1e-3) / 1e9
        roof_hbm = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": name}
    del leaves, dy, dfinal
    torch.cuda.empty_cache()
    tflops = total / (ms * 1e-3) / 1e12
    return {"ms_per_step": ms, "wall_ms_per_step": wall, "tokens_per_s": batch * length / (ms * 1e-3),
            "gflop_per_step": total / 1e9, "tflops": tflops, "mfma_frac": tflops / BF16_PEAK_TFLOPS,
            "gbs": (fwd_b + bwd_b) / (ms * 1e-3) / 1e9, "bytes_per_step": fwd_b + bwd_b,
            "roofline": roof, "roofline_hbm": roof_hbm, "kernels": mfma,
            "kernels_ms": {k: round(v, 4) for k, v in sorted(per.items())}}


def ssd_cpu_baseline(batch=4, length=4096):
    """The reference's CPU composition (oracle restatement) at the c4 shape."""
    import oracle
    from cases import ssd_problem
    torch.set_num_threads(os.cpu_count() or 1)
    p = ssd_problem(batch, length, 64, 64, 1, 128, seed=0, act=torch.bfloat16, init=False)
    leaves = {k: v.requires_grad_(True) for k, v in p.items() if v is not None}
    dy = torch.randn(batch, length, 64, 64, generator=torch.Generator().manual_seed(1)).bfloat16()

    def run():
        y, _ = oracle.mamba2_chunk_scan_composition(
            leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], chunk_size=256, D=leaves["D"],
            z=leaves["z"], dt_bias=leaves["dt_bias"], dt_softplus=True)
        torch.autograd.grad(y, list(leaves.values()), dy)

    run()
    best = None
    for _ in range(2):
        t0 = time.perf_counter()
        run()
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    return {"value": round(batch * length / best, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port", **host_cpu(),
            "sample": f"SSD fwd+bwd, batch {batch} x seqlen {length} at the c4 head shape (H64 P64 N128, chunk 256), "
                      f"bf16 chunked composition with autograd (oracle/ssm.py), best of 2 after 1 warm-up: "
                      f"{best:.2f} s"}


# --------------------------------------------------------------------- ss2d

SS2D_SHAPE = (1, 96, 1, 16, 56, 56)  # batch, channels, groups, states, height, width (b1_d96_56x56)


def ss2d_bytes(batch, channels, groups, states, height, width):
    """Algorithmic bytes (fwd, bwd) of one four-path scan step, float32 throughout."""
    e = batch * channels * height * width
    bc = batch * groups * states * height * width
    return 4 * (3 * e + 2 * bc), 4 * (5 * e + 4 * bc)  # u, dt, out / u, dt, dy, du, ddt; B, C (+ dB, dC)


def ss2d_inputs(shape, seed=101):
    batch, channels, groups, states, height, width = shape
    g = torch.Generator().manual_seed(seed)
    dims = (batch, channels, height, width)
    return {"u": torch.randn(dims, generator=g), "dt": torch.rand(dims, generator=g) * 0.2 + 0.05,
            "A": -(torch.rand((channels, states), generator=g) + 0.1),
            "B": torch.randn((batch, groups, states, height, width), generator=g),
            "C": torch.randn((batch, groups, states, height, width), generator=g)}, torch.randn(dims, generator=g)


def ss2d_case(steps, warmup, shape=SS2D_SHAPE):
    from metal_kernelops.cv import ss2d_scan
    inputs, dy = ss2d_inputs(shape)
    dev = torch.device("cuda")
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in inputs.items()}
    dy = dy.to(dev)
    order = list(leaves.values())

    def step():
        out = ss2d_scan(**leaves)
        torch.autograd.grad(out, order, dy)

    ms, wall, kernels = timed(step, steps, warmup)
    fwd_b, bwd_b = ss2d_bytes(*shape)
    name, avg, count = dominant(kernels)
    per_kernel = {"selscan_bwd_main": bwd_b, "selscan_fwd_replay": fwd_b}
    roof = roofline(per_kernel.get(name, fwd_b + bwd_b), avg)
    roof["kernel"] = name
    roof["algorithmic_bytes"] = per_kernel.get(name, fwd_b + bwd_b)
    del leaves, dy
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "wall_ms_per_step": wall, "gbs": (fwd_b + bwd_b) / (ms * 1e-3) / 1e9,
            "bytes_per_step": fwd_b + bwd_b, "roofline": roof,
            "kernels_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in sorted(kernels.items())}}


def ss2d_cpu_baseline(shape=(1, 96, 1, 16, 28, 28)):
    """The oracle's four-path restatement in float32 with autograd on the host cores.

    A bounded sample: the GPU workload's channels and states on a 28 x 28 map (a
    quarter of its steps), so one run stays near 6 s.
    """
    import oracle
    torch.set_num_threads(os.cpu_count() or 1)
    inputs, dy = ss2d_inputs(shape)
    leaves = {k: v.requires_grad_(True) for k, v in inputs.items()}

    def run():
        out = oracle.ss2d_scan(**leaves, dtype=torch.float32)
        torch.autograd.grad(out, list(leaves.values()), dy)

    run()
    t0 = time.perf_counter()
    run()
    best = time.perf_counter() - t0
    fwd_b, bwd_b = ss2d_bytes(*shape)
    return {"value": round((fwd_b + bwd_b) / best / 1e9, 6), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"ss2d fwd+bwd at {shape} (batch, channels, groups, states, H, W), float32 per-step "
                      f"recurrence over the four paths with autograd (oracle/ssm.py), one run after 1 warm-up: "
                      f"{best:.2f} s"}


# --------------------------------------------------------------------- causal conv1d

CONV_SHAPE = (4, 5120, 4096, 4)  # batch, channels, length, width: the conv ahead of the c3 scan


def conv1d_bytes(batch, channels, length, width, esz=2):
    """Algorithmic bytes (fwd, bwd): x in, out; x, dout in, dx out (weights negligible)."""
    e = batch * channels * length
    return 2 * e * esz, 3 * e * esz


def conv1d_case(steps, warmup, shape=CONV_SHAPE):
    from metal_kernelops.cv import causal_conv1d_fn, causal_conv1d_update
    batch, channels, length, width = shape
    g = torch.Generator().manual_seed(0)
    dev = torch.device("cuda")
    x = torch.randn(batch, channels, length, generator=g).bfloat16().to(dev).requires_grad_(True)
    w = (0.5 * torch.randn(channels, 1, width, generator=g)).bfloat16().to(dev).requires_grad_(True)
    b = torch.randn(channels, generator=g).bfloat16().to(dev).requires_grad_(True)
    dout = torch.randn(batch, channels, length, generator=g).bfloat16().to(dev)

    def step():
        out = causal_conv1d_fn(x, w, b, "silu")
        torch.autograd.grad(out, (x, w, b), dout)

    ms, wall, kernels = timed(step, steps, warmup)
    fwd_b, bwd_b = conv1d_bytes(*shape)
    name, avg, count = dominant(kernels)
    per_kernel = {"conv1d_bwd": bwd_b, "conv1d_fwd": fwd_b}
    roof = roofline(per_kernel.get(name, fwd_b + bwd_b), avg,
                    load_traffic(f"{name}@{batch}x{channels}x{length}x{width}"))
    roof["kernel"] = name
    roof["algorithmic_bytes"] = per_kernel.get(name, fwd_b + bwd_b)
    # decode: one token against a 3-column state, 64 x 2048 (the reference's update-64x2048x1)
    xs = torch.randn(64, 2048, generator=g).to(dev)
    state = torch.randn(64, 2048, 3, generator=g).to(dev)
    wd, bd = (0.5 * torch.randn(2048, 4, generator=g)).to(dev), torch.randn(2048, generator=g).to(dev)
    with torch.no_grad():
        dms, _, _ = timed(lambda: causal_conv1d_update(xs, state, wd, bd, "silu"), 200, 20)
    del x, w, b, dout
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "wall_ms_per_step": wall, "gbs": (fwd_b + bwd_b) / (ms * 1e-3) / 1e9,
            "bytes_per_step": fwd_b + bwd_b, "roofline": roof, "update_us": dms * 1e3,
            "kernels_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in sorted(kernels.items())}}


def conv1d_cpu_baseline(shape=(1, 1024, 4096, 4)):
    """The oracle's window product in float32 with autograd, on a bounded sample."""
    import oracle
    torch.set_num_threads(os.cpu_count() or 1)
    batch, channels, length, width = shape
    g = torch.Generator().manual_seed(0)
    x = torch.randn(batch, channels, length, generator=g).requires_grad_(True)
    w = (0.5 * torch.randn(channels, 1, width, generator=g)).requires_grad_(True)
    b = torch.randn(channels, generator=g).requires_grad_(True)
    dout = torch.randn(batch, channels, length, generator=g)

    def run():
        out, _ = oracle.causal_conv1d(x, w, b, "silu", dtype=torch.float32)
        torch.autograd.grad(out, (x, w, b), dout)

    run()
    best = None
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    fwd_b, bwd_b = conv1d_bytes(*shape, esz=4)
    return {"value": round((fwd_b + bwd_b) / best / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"causal conv1d fwd+bwd at {shape} (batch, channels, length, width), float32 window "
                      f"product with autograd (oracle/conv1d.py), best of 3 after 1 warm-up: {best * 1e3:.1f} ms"}


NORM_SHAPE = (8192, 2560)  # rows, features: the reference's first gated-norm bench shape, one group per row


def norm_bytes(rows, features, esz=2):
    """Algorithmic bytes (fwd, bwd) with z and no parameter gradients: x, z in, out;
    x, z, dout in, dx, dz out (weight, bias and the per-row rstd are negligible)."""
    e = rows * features
    return 3 * e * esz, 5 * e * esz


def norm_case(steps, warmup, shape=NORM_SHAPE):
    from metal_kernelops.cv import rmsnorm_gated
    rows, features = shape
    g = torch.Generator().manual_seed(0)
    dev = torch.device("cuda")
    x = torch.randn(rows, features, generator=g).bfloat16().to(dev).requires_grad_(True)
    z = torch.randn(rows, features, generator=g).bfloat16().to(dev).requires_grad_(True)
    w = torch.randn(features, generator=g).bfloat16().to(dev)
    b = torch.randn(features, generator=g).bfloat16().to(dev)
    dout = torch.randn(rows, features, generator=g).bfloat16().to(dev)

    def step():
        out = rmsnorm_gated(x, w, b, z)
        torch.autograd.grad(out, (x, z), dout)

    ms, wall, kernels = timed(step, steps, warmup)
    fwd_b, bwd_b = norm_bytes(*shape)
    name, avg, count = dominant(kernels)
    per_kernel = {"gated_norm_bwd": bwd_b, "gated_norm_fwd": fwd_b}
    roof = roofline(per_kernel.get(name, fwd_b + bwd_b), avg, load_traffic(f"{name}@{rows}x{features}"))
    roof["kernel"] = name
    roof["algorithmic_bytes"] = per_kernel.get(name, fwd_b + bwd_b)
    with torch.no_grad():
        fms, _, fk = timed(lambda: rmsnorm_gated(x, w, b, z), steps, warmup)
    del x, z, w, b, dout
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "wall_ms_per_step": wall, "gbs": (fwd_b + bwd_b) / (ms * 1e-3) / 1e9,
            "bytes_per_step": fwd_b + bwd_b, "roofline": roof, "fwd_us": fms * 1e3,
            "fwd_gbs": fwd_b / (fms * 1e-3) / 1e9,
            "kernels_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in sorted(kernels.items())}}


def norm_cpu_baseline(shape=(2048, 2560)):
    """The oracle's forward in float32 with autograd (dx, dz), on a bounded sample."""
    import oracle
    torch.set_num_threads(os.cpu_count() or 1)
    rows, features = shape
    g = torch.Generator().manual_seed(0)
    x = torch.randn(rows, features, generator=g).requires_grad_(True)
    z = torch.randn(rows, features, generator=g).requires_grad_(True)
    w, b = torch.randn(features, generator=g), torch.randn(features, generator=g)
    dout = torch.randn(rows, features, generator=g)

    def run():
        out, _ = oracle.rmsnorm_gated(x, w, b, z, dtype=torch.float32)
        torch.autograd.grad(out, (x, z), dout)

    run()
    best = None
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    fwd_b, bwd_b = norm_bytes(*shape, esz=4)
    return {"value": round((fwd_b + bwd_b) / best / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"gated RMSNorm fwd+bwd (dx, dz) at {shape} (rows, features), gate after the norm, "
                      f"float32 composition with autograd (oracle/norm.py), best of 3 after 1 warm-up: "
                      f"{best * 1e3:.1f} ms"}


class Mamba2Layer(torch.nn.Module):
    """The reference verifier's Mamba-2 block (``benchmarks/verify_cv_integration.py:38-78``):
    in_proj, causal conv1d with SiLU, chunked SSD scan with skip, step bias and softplus, gated
    RMSNorm (gate before the norm), out_proj -- on the package's kernels."""

    def __init__(self, d_model, heads, head_dim, d_state, conv=4, chunk=256):
        super().__init__()
        self.heads, self.head_dim, self.d_state, self.chunk = heads, head_dim, d_state, chunk
        inner = heads * head_dim
        self.inner = inner
        self.in_proj = torch.nn.Linear(d_model, 2 * inner + 2 * d_state + heads)
        self.conv_weight = torch.nn.Parameter(torch.randn(inner + 2 * d_state, 1, conv) * .3)
        self.conv_bias = torch.nn.Parameter(torch.randn(inner + 2 * d_state) * .1)
        self.a_log = torch.nn.Parameter(torch.randn(heads) * .2)
        self.d_skip = torch.nn.Parameter(torch.ones(heads))
        self.dt_bias = torch.nn.Parameter(torch.randn(heads) * .2)
        self.norm_weight = torch.nn.Parameter(torch.ones(inner))
        self.out_proj = torch.nn.Linear(inner, d_model)

    def forward(self, x):
        from metal_kernelops.cv import causal_conv1d_fn, mamba2_chunk_scan, rmsnorm_gated
        inner, n = self.inner, self.d_state
        zxbcdt = self.in_proj(x)
        z, xbc, dt = zxbcdt[..., :inner], zxbcdt[..., inner:2 * inner + 2 * n], zxbcdt[..., 2 * inner + 2 * n:]
        xbc = causal_conv1d_fn(xbc.transpose(1, 2), self.conv_weight.reshape(inner + 2 * n, -1), self.conv_bias,
                               activation="silu").transpose(1, 2)
        x_ssm = xbc[..., :inner].reshape(x.shape[0], x.shape[1], self.heads, self.head_dim)
        y, _ = mamba2_chunk_scan(x_ssm, dt, -torch.exp(self.a_log), xbc[..., inner:inner + n].unsqueeze(2),
                                 xbc[..., inner + n:].unsqueeze(2), chunk_size=self.chunk, D=self.d_skip,
                                 dt_bias=self.dt_bias, dt_softplus=True)
        y = rmsnorm_gated(y.reshape(x.shape[0], x.shape[1], inner), self.norm_weight, z=z, norm_before_gate=False)
        return self.out_proj(y)


class PathLayer(torch.nn.Module):
    """The verifier's VMamba-style block (``benchmarks/verify_cv_integration.py:81-100``)."""

    def __init__(self, channels=6, groups=2, states=4):
        super().__init__()
        self.groups, self.states = groups, states
        self.u = torch.nn.Conv2d(channels, channels, 3, padding=1)
        self.dt = torch.nn.Conv2d(channels, channels, 1)
        self.b = torch.nn.Conv2d(channels, groups * states, 1)
        self.c = torch.nn.Conv2d(channels, groups * states, 1)
        self.a = torch.nn.Parameter(-torch.rand(channels, states))

    def forward(self, x):
        from metal_kernelops.cv import ss2d_scan
        shape = (x.shape[0], self.groups, self.states, x.shape[2], x.shape[3])
        return ss2d_scan(self.u(x), torch.nn.functional.softplus(self.dt(x)), self.a,
                         self.b(x).reshape(shape), self.c(x).reshape(shape), merge="sum")


BLOCK_LAYER = dict(d_model=2560, heads=80, head_dim=64, d_state=128)  # Mamba-2 2.7B layer
BLOCK_TOKENS = (2, 4096)


def block_case(steps, warmup):
    """The verifier's two blocks at its shapes (fwd + bwd + zero_grad per step, as its timing
    loop, ``verify_cv_integration.py:141-155``), and a Mamba-2 2.7B layer in bf16."""
    torch.manual_seed(17)
    dev = torch.device("cuda")
    out = {}
    with torch.backends.cudnn.flags(enabled=False):  # torch's own convolutions, no MIOpen tuning
        for name, layer, shape in (("mamba2_block", Mamba2Layer(24, 2, 6, 5, chunk=8), (2, 19, 24)),
                                   ("path_block", PathLayer(), (2, 6, 9, 11))):
            layer = layer.to(dev)
            x = torch.randn(*shape, device=dev)

            def step():
                layer(x).square().mean().backward()
                layer.zero_grad(set_to_none=True)

            ms, _, _ = timed(step, steps, warmup)
            out[name] = {"ms_per_step": round(ms, 4), "shape": list(shape)}
    layer = Mamba2Layer(**BLOCK_LAYER).to(dev).bfloat16()
    for p in (layer.a_log, layer.d_skip, layer.dt_bias):
        p.data = p.data.float()
    batch, length = BLOCK_TOKENS
    x = torch.randn(batch, length, BLOCK_LAYER["d_model"], device=dev, dtype=torch.bfloat16)
    gy = torch.randn_like(x)

    def layer_step():
        layer(x).backward(gy)
        layer.zero_grad(set_to_none=True)

    ms, _, kernels = timed(layer_step, max(steps // 2, 3), warmup)
    tokens = batch * length
    out["mamba2_2.7b_layer"] = {
        "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 4),
        "config": dict(BLOCK_LAYER, batch=batch, seqlen=length, conv=4, dtype="bf16", ngroups=1),
        "kernels_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in sorted(kernels.items())},
        "mko_kernels_ms_per_step": round(sum(v[0] for v in kernels.values()) / max(steps // 2, 3), 4)}
    del layer, x, gy
    torch.cuda.empty_cache()
    return out


# --------------------------------------------------------------------- main


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--only", choices=["mamba1", "ssd", "decode", "ss2d", "conv1d", "norm", "block", "copy", "all"],
                    default="all",
                    help="one workload (mamba1 = the config-3 headline and config 2) or all of them; copy = "
                         "a plain 1 GiB device copy, the calibration point of the PMC byte counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    torch.backends.cuda.matmul.allow_tf32 = False

    if args.only == "copy":
        # Under rocprofv3 --pmc, FETCH_SIZE / WRITE_SIZE per dispatch of these copies calibrate
        # the byte counters against a known 1 GiB read and 1 GiB write (23 dispatches each of
        # the plain and the nontemporal form); the timed copies give the part's streaming rate.
        print(json.dumps(copy_floor()), flush=True)
        return
    log("copy floor: libmko streaming copy of 1 GiB")  # every run measures the floor it is compared with
    floor = copy_floor()
    log(f"  nontemporal {floor['nontemporal']['gbs']:.0f} GB/s, plain {floor['plain']['gbs']:.0f} GB/s")
    also = {}
    want = (lambda w: args.only in (w, "all"))
    if want("ssd"):
        log("mamba2 SSD config 4 (4x4096, H64 P64 N128, chunk 256) fwd+bwd")
        ssd = ssd_case(args.steps, args.warmup)
        also["mamba2_ssd_chunk_scan_fwd_bwd"] = {
            "value": round(ssd["tokens_per_s"], 1), "unit": "tokens/s",
            "ms_per_step": round(ssd["ms_per_step"], 4),
            "gflop_per_step": round(ssd["gflop_per_step"], 2), "tflops": round(ssd["tflops"], 1),
            "mfma_frac_whole_step": round(ssd["mfma_frac"], 4),
            "hbm_gbs_whole_step": round(ssd["gbs"], 1),
            "hbm_frac_whole_step": round(ssd["gbs"] / HBM_PEAK_GBS, 4),
            "config": {"batch": 4, "seqlen": 4096, "nheads": 64, "headdim": 64, "dstate": 128, "ngroups": 1,
                       "chunk_size": 256, "io_dtype": "bf16", "dt_dtype": "f32"},
            "roofline": ssd["roofline"], "roofline_hbm": ssd["roofline_hbm"], "kernels": ssd["kernels"],
            "kernels_ms": ssd["kernels_ms"]}
        log(f"  {ssd['ms_per_step']:.3f} ms/step, {ssd['tokens_per_s'] / 1e6:.2f} M tokens/s, "
            f"{ssd['tflops']:.1f} TFLOP/s ({100 * ssd['mfma_frac']:.1f}% MFMA), {ssd['gbs']:.0f} GB/s; "
            f"kernels {ssd['kernels_ms']}")
    head = None
    if want("mamba1"):
        log("mamba1 config 3 (4x5120x4096) fwd+bwd")
        head = mamba1_case(4, 5120, 4096, args.steps, args.warmup)
        log(f"  {head['ms_per_step']:.3f} ms/step, {head['gbs']:.1f} GB/s; kernels {head['kernels_ms']}")
        log("mamba1 config 2 (8x1536x2048) fwd+bwd")
        c2 = mamba1_case(8, 1536, 2048, args.steps, args.warmup)
        also["mamba1_130m_layer_fwd_bwd"] = {
            "value": round(c2["gbs"], 1), "unit": "GB/s", "ms_per_step": round(c2["ms_per_step"], 4),
            "config": {"batch": 8, "dim": 1536, "seqlen": 2048, "dstate": 16, "ngroups": 1},
            "hbm_frac_whole_step": round(c2["gbs"] / HBM_PEAK_GBS, 4),
            "roofline": c2["roofline"], "roofline_valu": c2["roofline_valu"], "kernels_ms": c2["kernels_ms"]}
        log(f"  {c2['ms_per_step']:.3f} ms/step, {c2['gbs']:.1f} GB/s")
    if want("decode"):
        log("mamba2 decode config 5 (256x80x64x128), 1024 in-place steps")
        dec = decode_case()
        also["mamba2_decode_state_rmw"] = {
            "value": round(dec["state_rmw_gbs"], 1), "unit": "GB/s",
            "ms_per_step": round(dec["ms_per_step"], 5), "steps": dec["steps"],
            "config": {"batch": 256, "nheads": 80, "headdim": 64, "dstate": 128, "ngroups": 1,
                       "state_dtype": "f32", "io_dtype": "bf16"},
            "roofline": dec["roofline"], "kernels_ms": dec["kernels_ms"], "backward": dec["backward"],
            "of_copy_floor": of_copy(dec["roofline"]["achieved"], floor),
            "backward_of_copy_floor": of_copy(dec["backward"]["roofline"]["achieved"], floor)}
        log(f"  {dec['ms_per_step'] * 1e3:.1f} us/step, {dec['state_rmw_gbs']:.1f} GB/s state RMW; backward "
            f"{dec['backward']['bwd_kernel_ms'] * 1e3:.1f} us, {dec['backward']['bwd_gbs']:.1f} GB/s")
    if want("ss2d"):
        log(f"ss2d four-path scan {SS2D_SHAPE} (batch, channels, groups, states, H, W) fwd+bwd, float32")
        s2 = ss2d_case(args.steps, args.warmup)
        also["ss2d_four_path_scan_fwd_bwd"] = {
            "value": round(s2["gbs"], 1), "unit": "GB/s", "ms_per_step": round(s2["ms_per_step"], 4),
            "config": dict(zip(("batch", "channels", "groups", "states", "height", "width"), SS2D_SHAPE),
                           dtype="f32"),
            "roofline": s2["roofline"], "kernels_ms": s2["kernels_ms"]}
        log(f"  {s2['ms_per_step']:.3f} ms/step, {s2['gbs']:.1f} GB/s; kernels {s2['kernels_ms']}")
    if want("conv1d"):
        log(f"causal conv1d {CONV_SHAPE} (batch, channels, length, width) fwd+bwd, bf16, silu")
        cv = conv1d_case(args.steps, args.warmup)
        also["causal_conv1d_fwd_bwd"] = {
            "value": round(cv["gbs"], 1), "unit": "GB/s", "ms_per_step": round(cv["ms_per_step"], 4),
            "config": dict(zip(("batch", "channels", "length", "width"), CONV_SHAPE), dtype="bf16",
                           activation="silu"),
            "roofline": cv["roofline"], "kernels_ms": cv["kernels_ms"],
            "decode_update_us": round(cv["update_us"], 2),
            "decode_update_config": {"batch": 64, "channels": 2048, "q": 1, "width": 4, "state_columns": 3,
                                     "dtype": "f32"}}
        log(f"  {cv['ms_per_step']:.3f} ms/step, {cv['gbs']:.1f} GB/s; decode update {cv['update_us']:.1f} us; "
            f"kernels {cv['kernels_ms']}")
    if want("norm"):
        log(f"gated RMSNorm {NORM_SHAPE} (rows, features) fwd+bwd, bf16, z and bias, gate after the norm")
        nm = norm_case(args.steps, args.warmup)
        also["gated_rmsnorm_fwd_bwd"] = {
            "value": round(nm["gbs"], 1), "unit": "GB/s", "ms_per_step": round(nm["ms_per_step"], 4),
            "fwd_us": round(nm["fwd_us"], 2), "fwd_gbs": round(nm["fwd_gbs"], 1),
            "config": {"rows": NORM_SHAPE[0], "features": NORM_SHAPE[1], "group_size": NORM_SHAPE[1],
                       "dtype": "bf16", "z": True, "bias": True, "norm_before_gate": True,
                       "grads": "x, z"},
            "roofline": nm["roofline"], "kernels_ms": nm["kernels_ms"]}
        log(f"  {nm['ms_per_step'] * 1e3:.1f} us/step, {nm['gbs']:.1f} GB/s; forward {nm['fwd_us']:.1f} us; "
            f"kernels {nm['kernels_ms']}")
    if want("block"):
        log("Mamba-2 block and path-scan block at the integration verifier's shapes; Mamba-2 2.7B layer bf16")
        bl = block_case(args.steps, args.warmup)
        also["integration_blocks_fwd_bwd"] = bl
        log(f"  verifier blocks {bl['mamba2_block']['ms_per_step']:.3f} / {bl['path_block']['ms_per_step']:.3f} ms; "
            f"2.7B layer {bl['mamba2_2.7b_layer']['ms_per_step']:.3f} ms/step, "
            f"{bl['mamba2_2.7b_layer']['value'] / 1e6:.2f} M tokens/s; kernels {bl['mamba2_2.7b_layer']['kernels_ms']}")
    if head is None:  # a single non-headline workload: print its own record
        also["copy_floor"] = floor
        print(json.dumps(also), flush=True)
        return
    cpu = None
    if not args.skip_cpu:
        log("cpu baseline (mamba1 config 3, forward)")
        cpu = mamba1_cpu_baseline(4, 5120, 4096)
        log(f"  {cpu['sample']}")
        if "mamba1_130m_layer_fwd_bwd" in also:
            log("cpu baseline (mamba1 config 2, forward)")
            also["mamba1_130m_layer_fwd_bwd"]["cpu_baseline"] = mamba1_cpu_baseline(8, 1536, 2048)
        if "mamba2_decode_state_rmw" in also:
            also["mamba2_decode_state_rmw"]["cpu_baseline"] = decode_cpu_baseline()
        if "mamba2_ssd_chunk_scan_fwd_bwd" in also:
            also["mamba2_ssd_chunk_scan_fwd_bwd"]["cpu_baseline"] = ssd_cpu_baseline()
        if "ss2d_four_path_scan_fwd_bwd" in also:
            also["ss2d_four_path_scan_fwd_bwd"]["cpu_baseline"] = ss2d_cpu_baseline()
        if "causal_conv1d_fwd_bwd" in also:
            also["causal_conv1d_fwd_bwd"]["cpu_baseline"] = conv1d_cpu_baseline()
        if "gated_rmsnorm_fwd_bwd" in also:
            also["gated_rmsnorm_fwd_bwd"]["cpu_baseline"] = norm_cpu_baseline()
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
        "roofline_valu": head["roofline_valu"],
        "copy_floor": floor,
        "cpu_baseline": cpu,
        "kernels_ms": head["kernels_ms"],
        "also": also,
        "torch": torch.__version__,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
