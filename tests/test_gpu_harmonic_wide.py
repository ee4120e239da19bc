"""Config 3 beyond one harmonic group: the HarmonicE2E model takes any
numHarmonics and noiseFilterSize (Examples/HarmonicE2E/Model.swift:36-40,
Config.swift:24-25), and the synth kernels run harmonics 64 to a group,
up to four groups (K <= 256) and K + 2 + NF <= 512 control columns.

Each stage of the HIP step against the CPU oracle fed the HIP path's own
upstream values, as tests/test_gpu_harmonic.py does for the default shape:
the phase checkpoints bit-exact, the controls and the synth forward within
1e-5, the audio within 1e-4 end to end, the synth and MLP backward within
1e-4 (relative L2); and at the bench's size (B=32, T=64000) with 100
harmonics and 100 noise taps.  Needs a GPU."""
import dataclasses
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle as O
from dgen_hip import HarmonicConfig
from dgen_hip.programs import HarmonicSession

pytestmark = pytest.mark.gpu

WORKERS = max(1, min(16, os.cpu_count() or 1))


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def run_step(cfg, tgt=None):
    s = HarmonicSession(cfg, optimizer=False, target=tgt)
    try:
        s.step()
        out = {k: s.rt.read(k) for k in ("ctrl", "y", "dy", "dctrl", "grads", "checkpoints", "f0_frames")}
        out["loss"] = s.loss()
        out["target"] = s.target
    finally:
        s.close()
    return out


# (K, NF): two groups with one spare lane short of a full group, the
# reference's defaults (one group, 97 columns), exactly one full group and
# 128 columns (no spare lane), a mostly masked wide bank with the fewest
# taps, and both maxima
SHAPES = [(65, 63), (32, 63), (64, 62), (200, 7), (100, 100), (256, 254)]


@pytest.mark.parametrize("K,NF", SHAPES, ids=[f"K{k}-NF{n}" for k, n in SHAPES])
def test_harmonic_groups_stage_parity(gpu, K, NF):
    cfg = HarmonicConfig(B=3, T=6400, K=K, NF=NF)
    print(f"K={K} NF={NF} NC={cfg.NC} ldc={cfg.ldc} B={cfg.B} T={cfg.T}", flush=True)
    f0, uv, X = cfg.data()
    tgt = O.harmonic_step(cfg, X, cfg.weights(seed=cfg.target_seed), f0, uv, np.zeros((cfg.B, cfg.T), np.float32),
                          grad=False, want_y=True, prec="f32")[2]
    out = run_step(cfg, tgt)
    f0f = out["f0_frames"].reshape(cfg.B, cfg.T)
    ck = O.phase_checkpoints(f0f, cfg.B, cfg.K, cfg.T, cfg.sr)
    np.testing.assert_array_equal(out["checkpoints"].reshape(ck.shape), ck)
    ctrl = out["ctrl"].reshape(cfg.M, cfg.ldc)[:, :cfg.NC]
    ref_c = O.mlp_fwd(X, cfg.weights(), cfg.M, cfg.din, cfg.hidden, cfg.layers, cfg.K, cfg.NF)
    e_c = np.abs(ctrl - ref_c).max()
    y = out["y"].reshape(cfg.B, cfg.T)
    e_s = np.abs(y - O.synth_fwd(ctrl, f0, uv, cfg.B, cfg.F, cfg.T, cfg.K, cfg.NF, cfg.sr)).max()
    _, _, ref_y = O.harmonic_step(cfg, X, cfg.weights(), f0, uv, tgt, grad=False, want_y=True, prec="f32")
    e_y = np.abs(y - ref_y).max()
    dy = out["dy"].reshape(cfg.B, cfg.T)
    dctrl = out["dctrl"].reshape(cfg.M, cfg.ldc)[:, :cfg.NC]
    e_dc = rel(dctrl, O.synth_bwd(ctrl, f0, uv, dy, cfg.B, cfg.F, cfg.T, cfg.K, cfg.NF, cfg.sr, prec="f64"))
    e_g = rel(out["grads"], O.mlp_bwd(X, cfg.weights(), dctrl, cfg.M, cfg.din, cfg.hidden, cfg.layers, cfg.K,
                                      cfg.NF, prec="f64"))
    # the padding columns of the stored rows stay zero
    pad = out["dctrl"].reshape(cfg.M, cfg.ldc)[:, cfg.NC:]
    print(f"controls {e_c:.2e}, synth forward {e_s:.2e}, y end to end {e_y:.2e}, synth backward {e_dc:.2e}, "
          f"MLP backward {e_g:.2e}", flush=True)
    assert e_c < 1e-5 and e_s < 1e-5 and e_y < 1e-4
    assert e_dc < 1e-4 and e_g < 1e-4
    assert not pad.any()


def test_hundred_harmonics_and_taps_at_full_size(gpu):
    """B=32, T=64000, K=100, NF=100 (two harmonic groups, 202 columns)."""
    cfg = HarmonicConfig(K=100, NF=100)
    print(f"full size K={cfg.K} NF={cfg.NF}: B={cfg.B} T={cfg.T} hidden={cfg.hidden}", flush=True)
    f0, uv, X = cfg.data()
    out = run_step(cfg)
    one = dataclasses.replace(cfg, B=1)
    Xb = X.reshape(cfg.B, cfg.F, cfg.din)
    f0f = out["f0_frames"].reshape(cfg.B, cfg.T)
    ck = O.phase_checkpoints(f0f, cfg.B, cfg.K, cfg.T, cfg.sr)
    np.testing.assert_array_equal(out["checkpoints"].reshape(ck.shape), ck)

    def lane(b, P, tgt, prec):
        return O.harmonic_step(one, np.ascontiguousarray(Xb[b]), P, np.ascontiguousarray(f0[:, b:b + 1]),
                               np.ascontiguousarray(uv[:, b:b + 1]), np.ascontiguousarray(tgt[b:b + 1]), grad=False,
                               want_y=True, prec=prec)

    zeros = np.zeros((cfg.B, cfg.T), np.float32)
    with ThreadPoolExecutor(WORKERS) as pool:
        tgt_ref = np.concatenate([r[2] for r in pool.map(
            lambda b: lane(b, cfg.weights(seed=cfg.target_seed), zeros, "f32"), range(cfg.B))])
        res32 = list(pool.map(lambda b: lane(b, cfg.weights(), out["target"], "f32"), range(cfg.B)))
        l64 = sum(r[0] for r in pool.map(lambda b: lane(b, cfg.weights().astype(np.float64), out["target"], "f64"),
                                          range(cfg.B))) / cfg.B
    y = out["y"].reshape(cfg.B, cfg.T)
    e_y = np.abs(y - np.concatenate([r[2] for r in res32])).max()
    e_t = np.abs(out["target"] - tgt_ref).max()
    e_l = abs(out["loss"] - l64) / abs(l64)
    ctrl = out["ctrl"].reshape(cfg.M, cfg.ldc)[:, :cfg.NC]
    dctrl = out["dctrl"].reshape(cfg.M, cfg.ldc)[:, :cfg.NC]
    dy = out["dy"].reshape(cfg.B, cfg.T)
    e_dc = rel(dctrl, O.synth_bwd(ctrl, f0, uv, dy, cfg.B, cfg.F, cfg.T, cfg.K, cfg.NF, cfg.sr, prec="f64"))
    e_g = rel(out["grads"], O.mlp_bwd(X, cfg.weights(), dctrl, cfg.M, cfg.din, cfg.hidden, cfg.layers, cfg.K,
                                      cfg.NF, prec="f64"))
    print(f"max|y - oracle| {e_y:.2e}, target {e_t:.2e}, loss rel to fp64 {e_l:.2e}, synth backward {e_dc:.2e}, "
          f"MLP backward {e_g:.2e}", flush=True)
    assert e_y < 1e-4 and e_t < 1e-4
    assert e_l < 1e-5
    assert e_dc < 1e-4 and e_g < 1e-4
