"""In-kernel timing of the config-3 phase chain (DGEN_HIP_K_PHASOR_CARRY's
timed build): where the chain wave's cycles go.

    python -m dgen_hip.chain_timer [--md summary.md]

The chain steps phase = fract(phase + inc) for 64000 frames per lane,
Emit+State.swift:322-369: two dependent VALU instructions a frame.  The
timed build stamps the shader clock (s_memtime) and the 100 MHz real-time
counter (s_memrealtime) in each workgroup and sums the cycles the chain
wave and the first producer wave waited at the interval barriers.  From
that, per workgroup: the chain's cycles per frame with and without the
barrier waits, the producers' slack, and the clock the CUs ran at.  It is
taken once with the op alone (DGEN_HIP_K_PHASOR_CARRY launched by itself)
and once inside the training step (the MLP forward beside it)."""
from __future__ import annotations

import argparse
import json

import numpy as np

from .programs import HarmonicSession
from .workloads import HarmonicConfig

WORDS = 8


def records(rt) -> np.ndarray:
    """[G*B][8] uint64 timer records from the chain_timer cell."""
    return rt.read("chain_timer").view(np.uint64).reshape(-1, WORDS)


def summarize(rec: np.ndarray, T: int) -> dict:
    cyc = (rec[:, 3] - rec[:, 2]).astype(np.float64)
    real_ns = (rec[:, 5] - rec[:, 4]).astype(np.float64) * 10.0
    wait, pwait = rec[:, 0].astype(np.float64), rec[:, 1].astype(np.float64)
    step = cyc - wait
    return {
        "workgroups": int(rec.shape[0]),
        "us": float(real_ns.max() / 1e3),
        "clock_ghz": float(np.median(cyc / real_ns)),
        "cycles_per_frame": float(np.median(cyc) / T),
        "stepping_cycles_per_frame": float(np.median(step) / T),
        "chain_wait_frac": float(np.median(wait / cyc)),
        "producer_wait_frac": float(np.median(pwait / cyc)),
        "cycles_per_dependent_op": float(np.median(step) / T / 2.0),
    }


def measure(cfg: HarmonicConfig | None = None, steps: int = 20) -> dict:
    cfg = cfg or HarmonicConfig()
    s = HarmonicSession(cfg, chain_timer=True)
    try:
        i = s.program.find("phasor_carry")
        alone_us = s.rt.time_op_alone(i, 10) * 1e3
        alone = summarize(records(s.rt), cfg.T)
        s.rt.set_graphs(True)
        for _ in range(steps):
            s.rt.run_async()
        s.rt.sync()
        in_step = summarize(records(s.rt), cfg.T)
        in_step_us = s.rt.time_op(i, 10) * 1e3
    finally:
        s.close()
    return {"config": {"B": cfg.B, "T": cfg.T, "K": cfg.K}, "alone": alone, "alone_event_us": alone_us,
            "in_step": in_step, "in_step_event_us": in_step_us}


def markdown(r: dict) -> str:
    rows = [("alone", r["alone"], r["alone_event_us"]), ("in the step", r["in_step"], r["in_step_event_us"])]
    out = ["| Run | µs (events) | µs (in-kernel) | clock GHz | cycles / frame | stepping cycles / frame | "
           "cycles / dependent op | chain barrier wait | producer barrier wait |",
           "|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for name, x, ev in rows:
        out.append(f"| {name} | {ev:.1f} | {x['us']:.1f} | {x['clock_ghz']:.2f} | {x['cycles_per_frame']:.2f} | "
                   f"{x['stepping_cycles_per_frame']:.2f} | {x['cycles_per_dependent_op']:.2f} | "
                   f"{100 * x['chain_wait_frac']:.1f}% | {100 * x['producer_wait_frac']:.1f}% |")
    return "\n".join(out) + "\n"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--md")
    ap.add_argument("--steps", type=int, default=20)
    args = ap.parse_args()
    r = measure(steps=args.steps)
    print(json.dumps(r), flush=True)
    text = markdown(r)
    print(text)
    if args.md:
        with open(args.md, "w") as fh:
            fh.write(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
