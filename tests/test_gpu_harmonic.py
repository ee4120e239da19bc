"""Config 3 parity: the HIP training step against the CPU oracle.

Each stage is compared with the oracle fed the HIP path's own upstream
values (so a mismatch names its stage), then end to end.  Tolerances:
forward audio 1e-4 max-abs (north star), losses 1e-5 relative, gradients of
the well-conditioned stages 1e-3 relative (L2)."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import HarmonicConfig
from dgen_hip.programs import HarmonicSession

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def small(gpu):
    cfg = HarmonicConfig(B=3, T=6400, hidden=512, fft_sizes=(2048, 1024, 512, 256, 128, 64))
    f0, uv, X = cfg.data()
    tgt = O.harmonic_step(cfg, X, cfg.weights(seed=cfg.target_seed), f0, uv, np.zeros((cfg.B, cfg.T), np.float32),
                          grad=False, want_y=True, prec="f32")[2]
    s = HarmonicSession(cfg, optimizer=False, target=tgt)
    s.step()
    out = {k: s.rt.read(k) for k in ("ctrl", "y", "loss_frames", "dy", "dctrl", "grads", "playhead", "noise")}
    s.close()
    return cfg, X, f0, uv, tgt, out


def test_static_tables(small):
    cfg, X, f0, uv, tgt, out = small
    np.testing.assert_array_equal(out["playhead"], O.playhead(cfg.F, cfg.T))
    np.testing.assert_array_equal(out["noise"], O.noise_stream(cfg.T))


def test_controls_match_oracle_mlp(small):
    cfg, X, f0, uv, tgt, out = small
    ctrl = out["ctrl"].reshape(cfg.M, 128)[:, :cfg.NC]
    ref = O.mlp_fwd(X, cfg.weights(), cfg.M, cfg.din, cfg.hidden, cfg.layers, cfg.K, cfg.NF)
    assert np.abs(ctrl - ref).max() < 1e-5


def test_synth_forward_matches_oracle(small):
    cfg, X, f0, uv, tgt, out = small
    ctrl = out["ctrl"].reshape(cfg.M, 128)[:, :cfg.NC]
    y = out["y"].reshape(cfg.B, cfg.T)
    ref = O.synth_fwd(ctrl, f0, uv, cfg.B, cfg.F, cfg.T, cfg.K, cfg.NF, cfg.sr)
    assert np.abs(y - ref).max() < 2e-6


def test_forward_end_to_end_within_1e4(small):
    cfg, X, f0, uv, tgt, out = small
    _, _, ref_y = O.harmonic_step(cfg, X, cfg.weights(), f0, uv, tgt, grad=False, want_y=True, prec="f32")
    assert np.abs(out["y"].reshape(cfg.B, cfg.T) - ref_y).max() < 1e-4


def test_loss_frames_match_oracle(small):
    cfg, X, f0, uv, tgt, out = small
    y = out["y"].reshape(cfg.B, cfg.T)
    tot, lf = O.mss_fwd(y, tgt, cfg.B, cfg.T, cfg.fft_sizes, cfg.hop_div, cfg.w_lin, cfg.w_log, cfg.T, frames=True)
    assert abs(out["loss_frames"].astype(np.float64).sum() - tot) / tot < 1e-5
    assert np.abs(out["loss_frames"] - lf).max() <= 1e-5 * np.abs(lf).max()


def test_synth_backward_matches_oracle(small):
    cfg, X, f0, uv, tgt, out = small
    ctrl = out["ctrl"].reshape(cfg.M, 128)[:, :cfg.NC]
    dy = out["dy"].reshape(cfg.B, cfg.T)
    ref = O.synth_bwd(ctrl, f0, uv, dy, cfg.B, cfg.F, cfg.T, cfg.K, cfg.NF, cfg.sr)
    got = out["dctrl"].reshape(cfg.M, 128)[:, :cfg.NC]
    assert rel(got, ref) < 1e-4


def test_mlp_backward_matches_oracle(small):
    cfg, X, f0, uv, tgt, out = small
    dctrl = out["dctrl"].reshape(cfg.M, 128)[:, :cfg.NC]
    ref = O.mlp_bwd(X, cfg.weights(), dctrl, cfg.M, cfg.din, cfg.hidden, cfg.layers, cfg.K, cfg.NF)
    assert rel(out["grads"], ref) < 1e-4
