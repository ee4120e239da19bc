"""Benchmark of the HIP backend on its headline workload.

One step = one training pass of the batch-32 harmonic + FIR-noise synth with
multi-scale spectral loss: control MLP forward (MFMA
GEMMs), synth forward, 6-scale spectral loss, backward to all 0.59M MLP
parameters, and the Adam update, with every input resident in HBM.

Prints ONE JSON line (rank 0):
  value         audio samples/s over the timed steps (B*T per step)
  roofline      the dominant kernel (largest roofline time = algorithmic
                cost; ties broken by measured time) against its own roof,
                timed with HIP events on the stream it launches on
  longest_kernel / kernels   the longest op by measured time and the top
                ops, each against its own bound (hbm, mfma or fp32 valu)
  step_roofline sum of per-op roofline times / measured step time
  cpu_baseline  the CPU oracle forward (fp32, -O3 -ffast-math) on a bounded
                sample of the same workload, timed on this host

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
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


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


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
    times = []
    for i in range(repeats + 1):
        t0 = time.perf_counter()
        O.harmonic_step(sub, Xs, P, f0s, uvs, tgt, grad=False, prec="f32", libname="liboracle_bench.so")
        dt = time.perf_counter() - t0
        if i:
            times.append(dt)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": lanes * cfg.T / med,
        "unit": "audio samples/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"forward only (the reference C backend has no backward): {lanes} of {cfg.B} lanes x "
                   f"T={cfg.T}, MLP {cfg.layers}x{cfg.hidden} + synth + {len(cfg.fft_sizes)}-scale spectral "
                   f"loss; median of {repeats} after 1 warm-up; host {platform.processor() or platform.machine()}, "
                   f"nproc {os.cpu_count()}"),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-lanes", type=int, default=4)
    ap.add_argument("--cpu-repeats", type=int, default=3)
    ap.add_argument("--op-iters", type=int, default=10, help="runs averaged for the dominant kernel's time")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this backend runs on one GPU; the multi-GPU "
              f"design (lane sharding + one gradient all-reduce) is not built.", file=sys.stderr)
        return 2

    from dgen_hip import HarmonicConfig
    from dgen_hip.programs import HarmonicSession
    from dgen_hip.roofline import step_roof_ms, table

    cfg = HarmonicConfig()  # B=32, T=64000 @ 16 kHz, K=60, NF=65, MLP 3x512, FFT 2048..64
    log(f"bench: building session B={cfg.B} T={cfg.T} K={cfg.K} hidden={cfg.hidden}")
    sess = HarmonicSession(cfg, device=0, optimizer=True)
    rt = sess.rt
    try:
        log(f"bench: warmup {args.warmup}")
        for _ in range(args.warmup):
            rt.run_async()
        rt.sync()
        log(f"bench: timing {args.steps} steps")
        t0 = time.perf_counter()
        for _ in range(args.steps):
            rt.run_async()
        rt.sync()
        wall = time.perf_counter() - t0
        ms_per_step = wall * 1e3 / args.steps
        value = cfg.B * cfg.T * args.steps / wall

        log("bench: per-op profile")
        prof = rt.profileKernels()
        rows = table(sess.program, prof)
        dom = max(rows, key=lambda r: (round(r.roof_ms, 6), r.meas_ms))
        longest = max(rows, key=lambda r: r.meas_ms)
        dom_ms = rt.time_op(dom.index, args.op_iters)
        dom.meas_ms = dom_ms
        ach, peak, unit = dom.achieved()
        roof_ms = step_roof_ms(sess.program)
        meas_sum = sum(r.meas_ms for r in rows)
        loss = sess.loss()
    finally:
        sess.close()

    for r in sorted(rows, key=lambda r: -r.meas_ms):
        log(f"  {r.label:18s} {r.bound:5s} meas {r.meas_ms * 1e3:9.1f} us  roof {r.roof_ms * 1e3:8.1f} us  "
            f"frac {r.frac:6.3f}")

    cpu = None
    if not args.no_cpu:
        log(f"bench: cpu baseline ({args.cpu_lanes} lanes)")
        cpu = cpu_baseline(cfg, args.cpu_lanes, args.cpu_repeats)

    out = {
        "metric": METRIC,
        "value": value,
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
        "roofline": {"kernel": dom.label, "bound": dom.bound, "achieved": ach, "peak": peak, "unit": unit,
                     "frac": ach / peak, "traffic": None, "ms": dom_ms},
        "longest_kernel": {"kernel": longest.label, "bound": longest.bound, "ms": longest.meas_ms,
                           "frac": longest.frac},
        "kernels": [{"kernel": r.label, "bound": r.bound, "ms": round(r.meas_ms, 4), "roof_ms": round(r.roof_ms, 4),
                     "frac": round(r.frac, 4)} for r in sorted(rows, key=lambda r: -r.meas_ms)[:10]],
        "step_roofline": {"roof_ms": roof_ms, "measured_ms": ms_per_step, "frac": roof_ms / ms_per_step,
                          "kernel_sum_ms": meas_sum},
        "loss": loss,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
