"""Benchmark of the HIP backend on its headline workload.

One step = one training pass of the batch-32 harmonic + FIR-noise synth with
multi-scale spectral loss (benchmark config 3): control MLP forward (MFMA
GEMMs), synth forward, 6-scale spectral loss, backward to all 0.59M MLP
parameters, and the Adam update, with every input resident in HBM.

Prints ONE JSON line (rank 0):
  value         audio samples/s over the timed steps (B*T per step)
  roofline      the dominant kernel (largest roofline time = algorithmic
                cost; ties broken by measured time) against its own roof,
                timed with HIP events on the stream it launches on
  longest_kernel / kernels   the longest op by measured time and the top
                ops, each against its own bound (hbm, mfma or fp32 valu):
                `ms` is the op run alone (HIP events over repeated solo
                runs), `in_step_ms` its event interval inside the step,
                which for a side-stream op also covers waiting for CU slots
                beside the stream-0 work it overlaps
  step_roofline sum of per-op roofline times / measured step time
  phase_chain   the phase chain alone and in the step against its latency
                floor (T dependent add+fract steps at their measured cycles)
  cpu_baseline  the CPU oracle forward (fp32, -O3 -ffast-math) on a bounded
                sample of the same workload, timed on this host

With ``--workload biquad`` the same line is printed for benchmark config 4
(256-lane x 2^18 tensor biquad bank, forward + loss + BPTT + Adam) and with
``--workload stft`` for config 2 (8 x 2^20 STFT round trip with per-bin
gains, forward + loss + gain gradient + Adam) and with ``--workload
membrane`` for config 5 (512^2 membrane, 4800 steps, forward + loss + adjoint
+ Adam) and with ``--workload oscbank`` for config 1 (16-oscillator bank,
65536 frames, forward only) and with ``--workload svf`` / ``svf-sat`` for
the 256-lane x 2^18 ZDF SVF bank (linear / learnable saturation, forward +
loss + BPTT + Adam) instead; the default workload is the headline config 3.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--workload harmonic|biquad|stft|membrane|oscbank|svf|svf-sat]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dgen-audio_amd"))

METRIC = "fwd+bwd audio samples/sec, batch-32 harmonic synth + MSS loss; % HBM peak"
BIQUAD_METRIC = "fwd+bwd lane-samples/sec, 256-lane x 2^18 tensor biquad bank with BPTT"
STFT_METRIC = "fwd+bwd input samples/sec, 8 x 2^20 hop-gated STFT round trip with 513 learnable gains"
MEMBRANE_METRIC = "fwd+bwd cell-steps/sec, 512^2 membrane x 4800 steps with BPTT to (c2, d)"
SVF_METRIC = "fwd+bwd lane-samples/sec, 256-lane x 2^18 ZDF SVF bank with BPTT"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def host_cpu() -> str:
    """The host's CPU model (first /proc/cpuinfo entry) and thread count."""
    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{model}, nproc {os.cpu_count()}"


def median_time(fn, repeats: int) -> float:
    """Median wall time of `repeats` calls of fn() after one warm-up call."""
    fn()
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def cpu_baseline(cfg, lanes: int, repeats: int) -> dict:
    """Time the oracle's emission-faithful fp32 forward (built with the
    reference C backend's -O3 -ffast-math -ffp-contract=fast policy) on
    `lanes` lanes of the same workload: same T, F, K, NF, MLP and FFT sizes.
    Single thread, like the reference C backend.  Median of `repeats` runs
    after one warm-up run."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import oracle as O
    from dgen_hip import HarmonicConfig

    f0, uv, X = cfg.data()
    sub = HarmonicConfig(**{**cfg.__dict__, "B": lanes})
    Xs = np.ascontiguousarray(X.reshape(cfg.B, cfg.F, cfg.din)[:lanes].reshape(-1, cfg.din))
    f0s = np.ascontiguousarray(f0[:, :lanes])
    uvs = np.ascontiguousarray(uv[:, :lanes])
    P = cfg.weights()
    tgt = np.zeros((lanes, cfg.T), np.float32)
    med = median_time(lambda: O.harmonic_step(sub, Xs, P, f0s, uvs, tgt, grad=False, prec="f32",
                                              libname="liboracle_bench.so"), repeats)
    return {
        "value": lanes * cfg.T / med,
        "unit": "audio samples/s",
        "cores": 1,
        "kind": "port",
        "host_cpu": host_cpu(),
        "sample": (f"forward only (the reference C backend has no backward): {lanes} of {cfg.B} lanes x "
                   f"T={cfg.T}, MLP {cfg.layers}x{cfg.hidden} + synth + {len(cfg.fft_sizes)}-scale spectral "
                   f"loss; median of {repeats} after 1 warm-up; host {host_cpu()}"),
    }


def time_session(rt, program, args):
    """Warm up, time args.steps back-to-back runs, then profile every op and
    time the dominant one (largest roofline time) with HIP events."""
    from dgen_hip.roofline import step_roof_ms, table
    if args.graphs:
        rt.set_graphs(True)
    # The timed region is the device work of the steps: with the program's
    # output cells declared, the sync that ends it would also copy them (the
    # rendered audio, 8 MB to 268 MB) to the host, which no step needs.
    rt.setOutputs(None)
    log(f"bench: warmup {args.warmup} (runs replayed as a HIP graph: {args.graphs})")
    for _ in range(args.warmup):
        rt.run_async()
    rt.sync()
    log(f"bench: timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        rt.run_async()
    rt.sync()
    wall = time.perf_counter() - t0
    log("bench: per-op profile")
    rows = table(program, rt.profileKernels())
    # among ops of equal roofline time, prefer stream-0 ops: a side-stream
    # op's event interval also covers the stream-0 work it overlaps
    from dgen_hip.runtime import OP_SIDE
    dom = max(rows, key=lambda r: (round(r.roof_ms, 6), not (program.ops[r.index].flags & OP_SIDE), r.meas_ms))
    # the longest ops (by their in-step interval), each also run alone
    for r in rows:
        r.in_step_ms = r.meas_ms
        r.side = bool(program.ops[r.index].flags & OP_SIDE)
    dom.meas_ms = rt.time_op(dom.index, args.op_iters)
    top = sorted(rows, key=lambda r: -r.in_step_ms)[:14]
    for r in top:
        r.meas_ms = rt.time_op_alone(r.index, args.op_iters)
    for r in sorted(top, key=lambda r: -r.meas_ms):
        log(f"  {r.label:18s} {r.bound:5s} {'side' if r.side else 'main'} alone {r.meas_ms * 1e3:8.1f} us  "
            f"in step {r.in_step_ms * 1e3:8.1f} us  roof {r.roof_ms * 1e3:8.1f} us  frac {r.frac:6.3f}")
    return wall, rows, dom, step_roof_ms(program)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")


def measured_traffic(workload: str, label: str):
    """HBM bytes per run of op `label`, from the rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes recorded by ``python -m dgen_hip.traffic`` (counters
    scaled by a plain copy of known size), or None if not measured."""
    try:
        with open(TRAFFIC_FILE) as fh:
            return json.load(fh)[workload][label]["bytes_per_run"]
    except (OSError, KeyError, ValueError):
        return None


def traffic_run(sess, workload: str, runs: int, labels: str | None = None) -> int:
    """Driver for the counter passes: one full run (so every cell holds
    its values), then for each op with the largest roofline time (or each
    op in the comma-separated `labels`) a plain 1 GiB device-to-device copy
    (the HIP runtime's copy kernel: the counter calibration, and a
    separator) and the op alone `runs` times.  Prints the op labels as one
    JSON line."""
    import ctypes

    from dgen_hip.roofline import roof_seconds
    from dgen_hip.runtime import OP_STATIC
    prog = sess.program
    per_run = [(i, roof_seconds(op)) for i, op in enumerate(prog.ops) if not op.flags & OP_STATIC]
    top = max(r for _, r in per_run)
    idx = [i for i, r in per_run if r >= top * (1.0 - 1e-9)]
    if labels:
        idx = [prog.find(lab) for lab in labels.split(",")]
    sess.rt.runNoCopy()
    hip = ctypes.CDLL("libamdhip64.so")  # the runtime libdgen_hip.so is linked against, already loaded
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMemcpyDtoD.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    n = 1 << 30
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(src), n) or hip.hipMalloc(ctypes.byref(dst), n):
        raise RuntimeError("traffic run: hipMalloc of the calibration buffers failed")
    try:
        for i in idx:
            if hip.hipMemcpyDtoD(dst, src, n) or hip.hipDeviceSynchronize():
                raise RuntimeError("traffic run: calibration copy failed")
            for _ in range(runs):
                sess.rt.run_op(i)
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)
    print(json.dumps({"traffic_ops": [prog.ops[i].label for i in idx], "runs": runs, "workload": workload}),
          flush=True)
    return 0


# cycles of one dependent add+fract step of a lone wave, measured on gfx950
# (dgen-audio_amd/csrc/probe_chain.cpp, mode 0)
CHAIN_STEP_CYCLES = 9.2


def roofline_fields(rows, dom, roof_ms, ms_per_step, workload: str = "harmonic"):
    longest = max(rows, key=lambda r: r.meas_ms)
    ach, peak, unit = dom.achieved()
    return {
        "roofline": {"kernel": dom.label, "bound": dom.bound, "achieved": ach, "peak": peak, "unit": unit,
                     "frac": ach / peak, "traffic": measured_traffic(workload, dom.label), "ms": dom.meas_ms},
        "longest_kernel": {"kernel": longest.label, "bound": longest.bound, "ms": longest.meas_ms,
                           "frac": longest.frac},
        "kernels": [{"kernel": r.label, "bound": r.bound, "stream": "side" if getattr(r, "side", False) else "main",
                     "ms": round(r.meas_ms, 4), "in_step_ms": round(getattr(r, "in_step_ms", r.meas_ms), 4),
                     "roof_ms": round(r.roof_ms, 4), "frac": round(r.frac, 4)}
                    for r in sorted(rows, key=lambda r: -r.meas_ms)[:10]],
        "step_roofline": {"roof_ms": roof_ms, "measured_ms": ms_per_step, "frac": roof_ms / ms_per_step,
                          "kernel_sum_ms": sum(getattr(r, "in_step_ms", r.meas_ms) for r in rows)},
    }


def biquad_cpu_baseline(cfg, repeats: int) -> dict:
    """The oracle's fp32 biquad step (forward, loss and BPTT backward; built
    with the reference C backend's -O3 -ffast-math policy) over the whole
    config-4 workload, single thread.  Median of `repeats` after a warm-up."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    x, m, p = cfg.inputs(), cfg.modulation(), cfg.params()
    tgt = O.biquad_fwd(x, None, cfg.target_params()[:cfg.B], cfg.target_params()[cfg.B:])
    fn = O._fn("dgen_oracle_biquad_step", "f32", "liboracle_bench.so")
    import ctypes
    import numpy as np
    g = np.zeros(2 * cfg.B, np.float32)
    med = median_time(lambda: fn(x, m.ctypes.data_as(ctypes.c_void_p), np.ascontiguousarray(p[:cfg.B]),
                                 np.ascontiguousarray(p[cfg.B:]), tgt, cfg.B, cfg.T, None,
                                 g.ctypes.data_as(ctypes.c_void_p)), repeats)
    return {
        "value": cfg.B * cfg.T / med,
        "unit": "lane-samples/s",
        "cores": 1,
        "kind": "port",
        "host_cpu": host_cpu(),
        "sample": (f"whole workload ({cfg.B} lanes x {cfg.T} frames): sequential fp32 forward, loss and BPTT "
                   f"backward (no Adam); median of {repeats} after 1 warm-up; host {host_cpu()}"),
    }


def run_biquad(args) -> dict:
    from dgen_hip import BiquadConfig
    from dgen_hip.programs import BQ_CHUNK, BiquadSession
    cfg = BiquadConfig()
    chunk = args.chunk or BQ_CHUNK
    log(f"bench: biquad session B={cfg.B} T={cfg.T} chunk={chunk}")
    sess = BiquadSession(cfg, device=0, optimizer=True, chunk=chunk)
    if args.traffic_runs:
        try:
            traffic_run(sess, "biquad", args.traffic_runs)
        finally:
            sess.close()
        return None
    try:
        wall, rows, dom, roof_ms = time_session(sess.rt, sess.program, args)
        loss = sess.loss()
    finally:
        sess.close()
    ms_per_step = wall * 1e3 / args.steps
    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline (biquad)")
        cpu = biquad_cpu_baseline(cfg, args.cpu_repeats)
    out = {
        "metric": BIQUAD_METRIC, "value": cfg.B * cfg.T * args.steps / wall, "unit": "lane-samples/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (U[-1,1] SplitMix64 input per lane, 2 Hz geometric cutoff sweep)",
        "config": {"workload": "config 4: tensor biquad bank, RBJ low-pass with per-sample coefficients, MSE vs "
                               "fixed bank, BPTT to base cutoff and Q, Adam", "B": cfg.B, "T": cfg.T, "sr": cfg.sr,
                   "chunk": chunk, "parallelism": "single GPU"},
    }
    out.update(roofline_fields(rows, dom, roof_ms, ms_per_step, "biquad"))
    out["loss"] = loss
    out["cpu_baseline"] = cpu
    return out


def svf_cpu_baseline(cfg, lanes: int, repeats: int) -> dict:
    """The oracle's fp32 SVF step (forward, loss and BPTT backward; built with
    the reference C backend's -O3 -ffast-math policy, single thread) on
    `lanes` of the bank's lanes over all frames.  Median of `repeats` after a
    warm-up."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ctypes

    import numpy as np
    import oracle as O
    x = np.ascontiguousarray(cfg.inputs()[:, :lanes])
    m, env = cfg.modulation(), cfg.envelope()
    p = cfg.params().reshape(cfg.P, cfg.B)[:, :lanes]
    tp = cfg.target_params().reshape(2, cfg.B)[:, :lanes]
    tgt = O.svf_fwd(x, tp[0], tp[1], None, m, env, cfg.sr)
    fn = O._fn("dgen_oracle_svf_step", "f32", "liboracle_bench.so")
    base, res = np.ascontiguousarray(p[0]), np.ascontiguousarray(p[1])
    ks = np.ascontiguousarray(p[2]) if cfg.saturating else None
    g = np.zeros(3 * lanes, np.float32)
    vp = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    med = median_time(lambda: fn(x, vp(m), vp(env), base, res, vp(ks), tgt, lanes, cfg.T, cfg.sr, None, vp(g), None),
                      repeats)
    return {
        "value": lanes * cfg.T / med,
        "unit": "lane-samples/s",
        "cores": 1,
        "kind": "port",
        "host_cpu": host_cpu(),
        "sample": (f"{lanes} of {cfg.B} lanes x {cfg.T} frames: sequential fp32 forward, loss and BPTT backward "
                   f"(no Adam); median of {repeats} after 1 warm-up; host {host_cpu()}"),
    }


def run_svf(args, saturating: bool) -> dict:
    from dgen_hip import SvfConfig
    from dgen_hip.programs import SVF_CHUNK, SvfSession
    cfg = SvfConfig(saturating=saturating)
    name = "svf-sat" if saturating else "svf"
    chunk = args.chunk or SVF_CHUNK
    log(f"bench: SVF session B={cfg.B} T={cfg.T} saturating={saturating} chunk={chunk}")
    sess = SvfSession(cfg, device=0, optimizer=True, chunk=chunk)
    if args.traffic_runs:
        try:
            traffic_run(sess, name, args.traffic_runs)
        finally:
            sess.close()
        return None
    try:
        wall, rows, dom, roof_ms = time_session(sess.rt, sess.program, args)
        loss = sess.loss()
    finally:
        sess.close()
    ms_per_step = wall * 1e3 / args.steps
    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline (svf)")
        cpu = svf_cpu_baseline(cfg, 32, args.cpu_repeats)
    out = {
        "metric": SVF_METRIC, "value": cfg.B * cfg.T * args.steps / wall, "unit": "lane-samples/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (U[-1,1] SplitMix64 input per lane, 2 Hz geometric cutoff sweep + 900 Hz envelope)",
        "config": {"workload": "ZDF SVF bank (SVFBPTTScratchTests.swift:21-34 per lane), MSE vs a fixed linear bank, "
                               "BPTT to base cutoff, res" + (" and kSat" if saturating else "") + ", Adam",
                   "B": cfg.B, "T": cfg.T, "sr": cfg.sr, "saturating": saturating, "chunk": chunk,
                   "parallelism": "single GPU"},
    }
    out.update(roofline_fields(rows, dom, roof_ms, ms_per_step, name))
    out["loss"] = loss
    out["cpu_baseline"] = cpu
    return out


def stft_cpu_baseline(cfg, signals: int, repeats: int) -> dict:
    """The oracle's fp32 STFT step (forward, loss and gain gradient; built
    with the reference C backend's -O3 -ffast-math policy) on `signals` of the
    config-2 signals at full length, single thread."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ctypes

    import numpy as np

    import oracle as O
    from dgen_hip import StftConfig
    sub = StftConfig(**{**cfg.__dict__, "S": signals})
    x = sub.inputs()
    fn = O._fn("dgen_oracle_stft_step", "f32", "liboracle_bench.so")
    dg = np.zeros(cfg.bins, np.float32)
    win, gains = cfg.window(), cfg.gains()
    med = median_time(lambda: fn(x, signals, cfg.T, cfg.N, cfg.H, win, gains, None,
                                 dg.ctypes.data_as(ctypes.c_void_p)), repeats)
    return {
        "value": signals * cfg.T / med,
        "unit": "input samples/s",
        "cores": 1,
        "kind": "port",
        "host_cpu": host_cpu(),
        "sample": (f"{signals} of {cfg.S} signals x {cfg.T} samples: radix-2 tensorFFT forward, gains, IFFT, "
                   f"overlap-add, loss and gain gradient (no Adam); median of {repeats} after 1 warm-up; host "
                   f"{host_cpu()}"),
    }


def run_stft(args) -> dict:
    from dgen_hip import StftConfig
    from dgen_hip.programs import StftSession
    cfg = StftConfig()
    log(f"bench: stft session S={cfg.S} T={cfg.T} N={cfg.N} H={cfg.H}")
    sess = StftSession(cfg, device=0, optimizer=True)
    if args.traffic_runs:
        try:
            traffic_run(sess, "stft", args.traffic_runs)
        finally:
            sess.close()
        return None
    try:
        wall, rows, dom, roof_ms = time_session(sess.rt, sess.program, args)
        loss = sess.loss()
    finally:
        sess.close()
    ms_per_step = wall * 1e3 / args.steps
    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline (stft)")
        cpu = stft_cpu_baseline(cfg, cfg.S, args.cpu_repeats)
    out = {
        "metric": STFT_METRIC, "value": cfg.S * cfg.T * args.steps / wall, "unit": "input samples/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (N(0, 0.25) SplitMix64 noise per signal)",
        "config": {"workload": "config 2: buffer N=1024 hop 256, periodic Hann, FFT, per-bin gains, IFFT, "
                               "overlapAdd, MSE vs input, gain gradient, Adam", "S": cfg.S, "T": cfg.T, "N": cfg.N,
                   "H": cfg.H, "parallelism": "single GPU"},
    }
    out.update(roofline_fields(rows, dom, roof_ms, ms_per_step, "stft"))
    out["loss"] = loss
    out["cpu_baseline"] = cpu
    return out


def membrane_cpu_baseline(cfg, frames: int, repeats: int) -> dict:
    """The oracle's fp32 membrane step (forward, loss and adjoint with
    checkpoint recomputation; -O3 -ffast-math build) on the full grid for
    the first `frames` frames, single thread."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ctypes

    import numpy as np

    import oracle as O
    u0 = cfg.bump()
    tgt = np.zeros(frames, np.float32)
    fn = O._fn("dgen_oracle_membrane_step", "f32", "liboracle_bench.so")
    g = np.zeros(2, np.float32)
    py, px = cfg.pickup
    med = median_time(lambda: fn(u0, cfg.R, cfg.C, frames, cfg.c2, cfg.d, py, px, tgt, None,
                                 g.ctypes.data_as(ctypes.c_void_p)), repeats)
    return {
        "value": cfg.R * cfg.C * frames / med,
        "unit": "cell-steps/s",
        "cores": 1,
        "kind": "port",
        "host_cpu": host_cpu(),
        "sample": (f"{cfg.R}x{cfg.C} grid, first {frames} of {cfg.T} frames: sequential fp32 forward, loss and "
                   f"adjoint with checkpoint recomputation (no Adam); median of {repeats} after 1 warm-up; host "
                   f"{host_cpu()}"),
    }


def run_membrane(args) -> dict:
    from dgen_hip import MembraneConfig
    from dgen_hip.programs import MembraneSession
    cfg = MembraneConfig()
    log(f"bench: membrane session {cfg.R}x{cfg.C} T={cfg.T} steps/launch={args.mem_steps}")
    sess = MembraneSession(cfg, device=0, optimizer=True, steps=args.mem_steps)
    if args.traffic_runs:
        try:
            traffic_run(sess, "membrane", args.traffic_runs)
        finally:
            sess.close()
        return None
    try:
        wall, rows, dom, roof_ms = time_session(sess.rt, sess.program, args)
        loss = sess.loss()
    finally:
        sess.close()
    ms_per_step = wall * 1e3 / args.steps
    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline (membrane)")
        cpu = membrane_cpu_baseline(cfg, cfg.T // 10, args.cpu_repeats)
    out = {
        "metric": MEMBRANE_METRIC, "value": cfg.R * cfg.C * cfg.T * args.steps / wall, "unit": "cell-steps/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (Gaussian bump at a SplitMix64 position)",
        "config": {"workload": "config 5: damped 2D wave equation, 3x3 Laplacian, pickup MSE vs (0.25, 0.002) "
                               "target, adjoint to (c2, d), Adam", "R": cfg.R, "C": cfg.C, "T": cfg.T,
                   "steps_per_launch": args.mem_steps, "parallelism": "single GPU"},
    }
    out.update(roofline_fields(rows, dom, roof_ms, ms_per_step, "membrane"))
    out["loss"] = loss
    out["cpu_baseline"] = cpu
    return out


OSCBANK_METRIC = "output samples/sec, 16-oscillator deterministic phasor bank -> sum -> one-pole, 65536 frames"


def oscbank_cpu_baseline(cfg, repeats: int) -> dict:
    """The oracle's fp32 oscillator bank (-O3 -ffast-math build) over the
    whole config-1 workload, single thread, like the reference C backend."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    freqs, amps = cfg.inputs()
    med = median_time(lambda: O.oscbank(freqs, amps, cfg.sr, cfg.pole, cfg.frames, libname="liboracle_bench.so"),
                      repeats)
    return {
        "value": cfg.frames / med,
        "unit": "output samples/s",
        "cores": 1,
        "kind": "port",
        "host_cpu": host_cpu(),
        "sample": (f"whole workload ({cfg.n_osc} oscillators x {cfg.frames} frames): frame-sequential fp32 "
                   f"phasors, sin, sum and one-pole; median of {repeats} after 1 warm-up; host {host_cpu()}"),
    }


def run_oscbank(args) -> dict:
    from dgen_hip import OscBankConfig
    from dgen_hip.programs import oscbank_program
    from dgen_hip.runtime import HIPLazyRuntime
    cfg = OscBankConfig()
    log(f"bench: oscillator bank n_osc={cfg.n_osc} frames={cfg.frames}")
    prog = oscbank_program(cfg)
    freqs, amps = cfg.inputs()
    with HIPLazyRuntime(prog, 0) as rt:
        rt.write("freqs", freqs)
        rt.write("amps", amps)
        wall, rows, dom, roof_ms = time_session(rt, prog, args)
    ms_per_step = wall * 1e3 / args.steps
    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline (oscillator bank)")
        cpu = oscbank_cpu_baseline(cfg, args.cpu_repeats)
    out = {
        "metric": OSCBANK_METRIC, "value": cfg.frames * args.steps / wall, "unit": "output samples/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (amplitudes U[0,1] from SplitMix64, normalised to sum 1)",
        "config": {"workload": "config 1: 16 deterministic phasors at k*220 Hz, sin, amplitude sum, history "
                               "one-pole 0.9, forward only", "n_osc": cfg.n_osc, "frames": cfg.frames, "sr": cfg.sr,
                   "parallelism": "single GPU"},
    }
    out.update(roofline_fields(rows, dom, roof_ms, ms_per_step, "oscbank"))
    out["cpu_baseline"] = cpu
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-lanes", type=int, default=4)
    ap.add_argument("--cpu-repeats", type=int, default=5)
    ap.add_argument("--op-iters", type=int, default=10, help="runs averaged for the dominant kernel's time")
    ap.add_argument("--traffic-runs", type=int, default=0,
                    help="instead of timing: run the dominant op alone this many times (for rocprofv3 --pmc)")
    ap.add_argument("--traffic-ops", default=None,
                    help="with --traffic-runs: the comma-separated op labels to run instead of the dominant op")
    ap.add_argument("--no-graphs", dest="graphs", action="store_false",
                    help="enqueue every kernel from the host instead of replaying each step as a HIP graph")
    ap.add_argument("--workload", choices=("harmonic", "biquad", "stft", "membrane", "oscbank", "svf", "svf-sat"),
                    default="harmonic")
    ap.add_argument("--mem-steps", type=int, default=16, help="membrane frames per time-blocked launch")
    ap.add_argument("--chunk", type=int, default=None,
                    help="biquad / SVF scan chunk length (frames; default: the program's, 512 biquad, 256 SVF)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this backend runs on one GPU; the multi-GPU "
              f"design (lane sharding + one gradient all-reduce) is not built.", file=sys.stderr)
        return 2
    run = {"biquad": run_biquad, "stft": run_stft, "membrane": run_membrane, "harmonic": run_harmonic,
           "oscbank": run_oscbank, "svf": lambda a: run_svf(a, False),
           "svf-sat": lambda a: run_svf(a, True)}[args.workload]
    res = run(args)
    if res is not None:
        print(json.dumps(res), flush=True)
    return 0


def run_harmonic(args) -> dict:
    from dgen_hip import HarmonicConfig
    from dgen_hip.programs import HarmonicSession

    cfg = HarmonicConfig()  # B=32, T=64000 @ 16 kHz, K=60, NF=65, MLP 3x512, FFT 2048..64
    log(f"bench: building session B={cfg.B} T={cfg.T} K={cfg.K} hidden={cfg.hidden}")
    sess = HarmonicSession(cfg, device=0, optimizer=True)
    if args.traffic_runs:
        try:
            traffic_run(sess, "harmonic", args.traffic_runs, args.traffic_ops)
        finally:
            sess.close()
        return None
    try:
        wall, rows, dom, roof_ms = time_session(sess.rt, sess.program, args)
        loss = sess.loss()
    finally:
        sess.close()
    ms_per_step = wall * 1e3 / args.steps
    cpu = None
    if not args.no_cpu:
        log(f"bench: cpu baseline ({args.cpu_lanes} lanes)")
        cpu = cpu_baseline(cfg, args.cpu_lanes, args.cpu_repeats)
    out = {
        "metric": METRIC,
        "value": cfg.B * cfg.T * args.steps / wall,
        "unit": "audio samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64 controls, random-init MLP weights)",
        "config": {"workload": "config 3: batch-32 harmonic+FIR-noise synth, 3x512 MLP decoder, 6-scale MSS "
                               "loss, fwd+bwd+Adam", "B": cfg.B, "T": cfg.T, "sr": cfg.sr, "harmonics": cfg.K,
                   "noise_taps": cfg.NF, "fft_sizes": list(cfg.fft_sizes), "mlp": [cfg.din] + [cfg.hidden] * cfg.layers
                   + [cfg.NC], "parallelism": "single GPU"},
    }
    out.update(roofline_fields(rows, dom, roof_ms, ms_per_step, "harmonic"))
    # the phase chain is a latency bound, not a VALU-throughput one: its
    # floor is T dependent add+fract steps at the cycles one takes
    # (dgen-audio_amd/csrc/probe_chain.cpp) at the part's 2.4 GHz
    chain = [r for r in rows if r.label == "phasor_carry"]
    if chain:
        floor_ms = cfg.T * CHAIN_STEP_CYCLES / 2.4e9 * 1e3
        out["phase_chain"] = {"ms": chain[0].meas_ms, "in_step_ms": getattr(chain[0], "in_step_ms", chain[0].meas_ms),
                              "latency_floor_ms": floor_ms, "frac_of_floor": floor_ms / chain[0].meas_ms,
                              "step_cycles_measured_floor": CHAIN_STEP_CYCLES}
    out["loss"] = loss
    out["cpu_baseline"] = cpu
    return out


if __name__ == "__main__":
    sys.exit(main())
