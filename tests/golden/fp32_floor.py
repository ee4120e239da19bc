"""The fp32 floor of the config-3 gradient at the full per-lane shape (B=4,
T=64000, hidden 512, six FFT sizes), measured on the CPU oracle.

The fp32 evaluation of the reference semantics (the oracle's fp32 build) is
compared with central finite differences of its fp64 build, at the default
parameters and at NDRAWS last-ulp moves of them (every parameter moved one
ulp up or down at random, numpy default_rng(4321)), which move the
forward's fp32 rounding the way a different fp32 implementation does.  For
each draw: the along-gradient error, the errors of the 8 largest
components, the whole gradient's relative L2 distance from the fp64
gradient, and the spectral dL/dy stage at the fp32 prediction against fp64
at the same prediction.  The per-draw values and their medians and maxima go
to fp32_floor.json, which tests/test_gpu_harmonic_full.py reads for its
bars.

Run from the repository root: python tests/golden/fp32_floor.py [NDRAWS]
(about 40 s per draw on 8 cores)."""
import dataclasses
import json
import os
import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "dgen-audio_amd"), os.path.join(ROOT, "oracle"), ROOT]
import oracle as O  # noqa: E402
from dgen_hip import HarmonicConfig  # noqa: E402

SEED = 4321


def param_draw(P0, rng):
    up = rng.random(P0.shape) < 0.5
    return np.where(up, np.nextafter(P0, np.float32(np.inf)), np.nextafter(P0, np.float32(-np.inf))).astype(np.float32)


def main(ndraws: int) -> None:
    cfg = HarmonicConfig(B=4)
    one = dataclasses.replace(cfg, B=1)
    f0, uv, X = cfg.data()
    Xl = X.reshape(cfg.B, cfg.F, cfg.din)
    pool = ThreadPoolExecutor(min(8, os.cpu_count() or 1))
    P0 = cfg.weights()
    # the target: the oracle's fp32 render of the target seed's weights
    zeros = np.zeros((1, cfg.T), np.float32)
    Pt = cfg.weights(seed=cfg.target_seed)
    tgt = np.concatenate(list(pool.map(lambda b: O.harmonic_step(
        one, np.ascontiguousarray(Xl[b]), Pt, np.ascontiguousarray(f0[:, b:b + 1]),
        np.ascontiguousarray(uv[:, b:b + 1]), zeros, grad=False, want_y=True, prec="f32")[2], range(cfg.B))))

    def step(P, grad, prec, want_y=False):
        def f(b):
            return O.harmonic_step(one, np.ascontiguousarray(Xl[b]), P, np.ascontiguousarray(f0[:, b:b + 1]),
                                   np.ascontiguousarray(uv[:, b:b + 1]), np.ascontiguousarray(tgt[b:b + 1]),
                                   grad=grad, want_y=want_y, prec=prec)
        r = list(pool.map(f, range(cfg.B)))
        return (sum(x[0] for x in r) / cfg.B, sum(x[1].astype(np.float64) for x in r) / cfg.B if grad else None,
                np.concatenate([x[2] for x in r]) if want_y else None)

    def mssb(y, prec):
        return np.concatenate(list(pool.map(lambda b: O.mss_bwd(
            y[b:b + 1], tgt[b:b + 1], 1, cfg.T, cfg.fft_sizes, cfg.hop_div, cfg.w_lin, cfg.w_log, cfg.T,
            prec=prec) / cfg.B, range(cfg.B))))

    def rel(a, b):
        return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))

    rng = np.random.default_rng(SEED)
    draws = []
    for d in range(ndraws + 1):
        P32 = P0 if d == 0 else param_draw(P0, rng)
        P64 = P32.astype(np.float64)
        _, g64, _ = step(P64, True, "f64")
        _, g32, y32 = step(P32, True, "f32", want_y=True)
        u = g64 / np.linalg.norm(g64)
        fd = (step(P64 + 1e-6 * u, False, "f64")[0] - step(P64 - 1e-6 * u, False, "f64")[0]) / 2e-6
        comps = []
        for i in np.argsort(-np.abs(g64))[:8]:
            e = np.zeros_like(P64)
            e[i] = 1.0
            c = (step(P64 + 1e-7 * e, False, "f64")[0] - step(P64 - 1e-7 * e, False, "f64")[0]) / 2e-7
            comps.append(dict(param=int(i), rel_err=abs(g32[i] - c) / abs(c)))
        r = dict(draw=d, along=abs(g32 @ u - fd) / abs(fd), along_fp64=abs(g64 @ u - fd) / abs(fd),
                 whole=rel(g32, g64), dy_stage=rel(mssb(y32, "f32"), mssb(y32, "f64")), components=comps)
        draws.append(r)
        print(json.dumps({k: v for k, v in r.items() if k != "components"}), flush=True)

    def stats(vals):
        v = np.asarray(vals)
        return dict(median=float(np.median(v)), max=float(v.max()), min=float(v.min()))

    out = dict(
        config=dict(B=cfg.B, T=cfg.T, hidden=cfg.hidden, fft_sizes=list(cfg.fft_sizes), seed=SEED, draws=ndraws + 1),
        along=stats([r["along"] for r in draws]), whole=stats([r["whole"] for r in draws]),
        dy_stage=stats([r["dy_stage"] for r in draws]),
        components=stats([c["rel_err"] for r in draws for c in r["components"]]),
        draws=draws)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fp32_floor.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {path}")


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 11)
