"""The oracle still reproduces the committed golden step (tests/golden/,
written by tests/golden/make_golden.py).  CPU only."""
import os

import numpy as np
import pytest

import oracle as O
from dgen_hip import HarmonicConfig

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "harmonic_small.npz")


@pytest.fixture(scope="module")
def golden():
    g = np.load(GOLDEN, allow_pickle=False)
    c = g["config"]
    cfg = HarmonicConfig(B=int(c[0]), T=int(c[1]), hidden=int(c[2]), fft_sizes=tuple(int(v) for v in c[3:]))
    return cfg, g


def test_inputs_regenerate(golden):
    cfg, g = golden
    f0, uv, X = cfg.data()
    np.testing.assert_array_equal(X, g["X"])
    np.testing.assert_array_equal(f0, g["f0"])
    np.testing.assert_array_equal(cfg.weights(), g["params"])


def test_forward_and_loss(golden):
    cfg, g = golden
    loss, _, y = O.harmonic_step(cfg, g["X"], g["params"], g["f0"], g["uv"], g["target"], grad=False, want_y=True,
                                 prec="f32")
    np.testing.assert_allclose(y, g["y"], atol=1e-6)
    assert abs(loss - float(g["loss"])) <= 1e-6 * abs(float(g["loss"]))


def test_gradient(golden):
    cfg, g = golden
    _, grad, _ = O.harmonic_step(cfg, g["X"], g["params"].astype(np.float64), g["f0"], g["uv"], g["target"], grad=True,
                                 prec="f64")
    np.testing.assert_allclose(grad, g["grad"], rtol=1e-9, atol=1e-14)


def test_frame_tables(golden):
    cfg, g = golden
    f0f = O.lerp_frames(g["f0"], cfg.B, cfg.F, cfg.T)
    np.testing.assert_array_equal(f0f, g["f0_frames"])
    np.testing.assert_array_equal(O.phase_checkpoints(f0f, cfg.B, cfg.K, cfg.T, cfg.sr), g["checkpoints"])
