"""Writes tests/golden/harmonic_small.npz: a small config-3 training step
evaluated by the CPU oracle (a restatement of the reference's semantics;
the reference itself cannot be built here, so these are oracle-generated
vectors, not reference-generated ones).

  inputs   X [B*F][2], f0 [F][B], uv [F][B], params (SplitMix64 init),
           target [B][T] (the same synth from the target-seed weights)
  outputs  y [B][T] (fp32 forward), loss (sum over frames), loss_frames [T],
           grad [params] (fp64 backward), f0_frames [B][T], checkpoints

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "dgen-audio_amd"), os.path.join(ROOT, "oracle")]

import oracle as O  # noqa: E402
from dgen_hip import HarmonicConfig  # noqa: E402

CFG = dict(B=2, T=1024, hidden=16, fft_sizes=(256, 128, 64))


def main():
    cfg = HarmonicConfig(**CFG)
    f0, uv, X = cfg.data()
    P = cfg.weights()
    zeros = np.zeros((cfg.B, cfg.T), np.float32)
    target = O.harmonic_step(cfg, X, cfg.weights(seed=cfg.target_seed), f0, uv, zeros, grad=False, want_y=True,
                             prec="f32")[2]
    loss, _, y = O.harmonic_step(cfg, X, P, f0, uv, target, grad=False, want_y=True, prec="f32")
    _, lf = O.mss_fwd(y, target, cfg.B, cfg.T, cfg.fft_sizes, cfg.hop_div, cfg.w_lin, cfg.w_log, cfg.T, frames=True)
    _, grad, _ = O.harmonic_step(cfg, X, P.astype(np.float64), f0, uv, target, grad=True, prec="f64")
    f0f = O.lerp_frames(f0, cfg.B, cfg.F, cfg.T)
    ck = O.phase_checkpoints(f0f, cfg.B, cfg.K, cfg.T, cfg.sr)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "harmonic_small.npz")
    np.savez_compressed(out, X=X, f0=f0, uv=uv, params=P, target=target, y=y, loss=np.float64(loss),
                        loss_frames=lf, grad=grad, f0_frames=f0f, checkpoints=ck,
                        config=np.array([cfg.B, cfg.T, cfg.hidden] + list(cfg.fft_sizes), np.int64))
    print(out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
