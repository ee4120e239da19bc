"""Pins of the config-4 biquad oracle (oracle/dgen_oracle.c, bq_*) against
the RBJ cookbook low-pass as scipy.signal evaluates it, closed-form filter
properties, lane independence and central finite differences.  CPU only."""
import math

import numpy as np
import pytest
import scipy.signal as ss

import oracle as O
from dgen_hip import BiquadConfig

W0_PER_HZ = float(np.float32(0.00014247585730565955))


def rbj_lowpass(fc, Q):
    """RBJ Audio-EQ-Cookbook LPF, normalised by a0, in fp64."""
    w = abs(fc) * W0_PER_HZ
    c, s = math.cos(w), math.sin(w)
    al = s / (2.0 * abs(Q))
    b = np.array([(1 - c) / 2, 1 - c, (1 - c) / 2]) / (1 + al)
    a = np.array([1.0, -2 * c / (1 + al), (1 - al) / (1 + al)])
    return b, a


def noise(T, B, seed):
    return np.random.default_rng(seed).uniform(-1, 1, (T, B)).astype(np.float32)


def test_w0_constant_is_two_pi_over_44100():
    # Sources/DGen/HigherOps.swift:446-447 hardcodes 44.1 kHz
    assert np.float32(0.00014247585730565955) == np.float32(2 * math.pi / 44100)


def test_constant_cutoff_matches_scipy_lfilter():
    T, base, Q = 4096, [200.0, 1000.0, 5000.0, 12000.0], [0.707, 2.0, 0.5, 0.9]
    x = noise(T, 4, 1)
    y = O.biquad_fwd(x, None, base, Q, prec="f64")
    for k in range(4):
        b, a = rbj_lowpass(base[k], Q[k])
        ref = ss.lfilter(b, a, x[:, k].astype(np.float64))
        err = np.abs(y[:, k] - ref).max()
        assert err <= 1e-6 * max(1.0, np.abs(ref).max()), (k, err)


def test_negative_cutoff_and_q_use_magnitudes():
    x = noise(512, 2, 2)
    y_pos = O.biquad_fwd(x, None, [700.0, 700.0], [0.8, 0.8], prec="f64")
    y_neg = O.biquad_fwd(x, None, [-700.0, 700.0], [0.8, -0.8], prec="f64")
    np.testing.assert_array_equal(y_pos, y_neg)


def test_dc_gain_is_one_and_gain_at_cutoff_is_q():
    # bilinear-transformed 1/(s^2 + s/Q + 1): |H(0)| = 1, |H(e^{j w0})| = Q
    T, fc, Q = 40000, 1000.0, 1.7
    step = np.ones((T, 1), np.float32)
    y = O.biquad_fwd(step, None, [fc], [Q], prec="f64")
    assert abs(y[-1, 0] - 1.0) < 1e-6
    w0 = fc * W0_PER_HZ
    n = np.arange(T)
    sine = np.sin(w0 * n).astype(np.float32)[:, None]
    y = O.biquad_fwd(sine, None, [fc], [Q], prec="f64")[:, 0].astype(np.float64)
    tail = slice(T // 2, T)
    A = np.stack([np.sin(w0 * n[tail]), np.cos(w0 * n[tail])], 1)
    coef, *_ = np.linalg.lstsq(A, y[tail], rcond=None)
    assert abs(np.hypot(*coef) - Q) < 1e-4 * Q


def test_per_sample_coefficients_switch_like_lfiltic_continuation():
    # a cutoff step at frame h: frames >= h use the new coefficients with the
    # old input/output history (Direct Form I), which scipy expresses as
    # lfilter(..., zi=lfiltic(b2, a2, y_hist, x_hist))
    T, h = 6000, 2500
    base, Q = [300.0, 800.0], [0.707, 1.3]
    m = np.ones(T, np.float32)
    m[h:] = 2.5
    x = noise(T, 2, 3)
    y = O.biquad_fwd(x, m, base, Q, prec="f64")
    for k in range(2):
        xs = x[:, k].astype(np.float64)
        b1, a1 = rbj_lowpass(base[k], Q[k])
        b2, a2 = rbj_lowpass(base[k] * 2.5, Q[k])
        first = ss.lfilter(b1, a1, xs[:h])
        zi = ss.lfiltic(b2, a2, [first[-1], first[-2]], [xs[h - 1], xs[h - 2]])
        second, _ = ss.lfilter(b2, a2, xs[h:], zi=zi)
        ref = np.concatenate([first, second])
        assert np.abs(y[:, k] - ref).max() <= 1e-6 * np.abs(ref).max(), k


def test_lanes_are_independent():
    # batched == per-lane serial (Tests/DGenLazyTests/TensorBiquadGradientTests.swift:109-140)
    cfg = BiquadConfig(B=4, T=3000)
    x, m = cfg.inputs(), cfg.modulation()
    base = [200.0, 350.0, 90.0, 1200.0]
    Q = [0.707, 0.5, 2.0, 1.1]
    y = O.biquad_fwd(x, m, base, Q)
    for k in range(4):
        yk = O.biquad_fwd(np.ascontiguousarray(x[:, k:k + 1]), m, [base[k]], [Q[k]])
        np.testing.assert_array_equal(y[:, k], yk[:, 0])


def test_fp32_build_within_parity_bar_of_fp64():
    cfg = BiquadConfig(B=8, T=1 << 15)
    x, m, p = cfg.inputs(), cfg.modulation(), cfg.params()
    y32 = O.biquad_fwd(x, m, p[:8], p[8:], prec="f32")
    y64 = O.biquad_fwd(x, m, p[:8], p[8:], prec="f64")
    assert np.abs(y32 - y64).max() < 1e-4


def test_modulation_sweeps_the_configured_range():
    cfg = BiquadConfig(B=1, T=44100)
    m = cfg.modulation().astype(np.float64)
    assert abs(m[0] - math.sqrt(20.0)) < 1e-5          # sin(0) -> geometric midpoint
    assert abs(m.max() - 20.0) < 1e-3 and abs(m.min() - 1.0) < 1e-4
    assert abs(m[11025] - m[0]) < 1e-3                  # 2 Hz: period 22050 samples
    assert np.argmax(m[:22050]) == pytest.approx(22050 / 4, abs=2)


def test_gradient_matches_central_differences():
    cfg = BiquadConfig(B=3, T=3000)
    x, m = cfg.inputs(), cfg.modulation()
    base = np.array([200.0, 420.0, 90.0])
    Q = np.array([0.707, 1.4, 0.6])
    tgt = O.biquad_fwd(x, None, [1000.0] * 3, [0.707] * 3, prec="f64")
    _, g, _ = O.biquad_step(x, m, base, Q, tgt, prec="f64")
    for j in range(6):
        p = np.concatenate([base, Q])
        eps = 1e-6 * abs(p[j])
        pp, pm = p.copy(), p.copy()
        pp[j] += eps
        pm[j] -= eps
        lp = O.biquad_step(x, m, pp[:3], pp[3:], tgt, grad=False, prec="f64")[0]
        lm = O.biquad_step(x, m, pm[:3], pm[3:], tgt, grad=False, prec="f64")[0]
        fd = (lp - lm) / (2 * eps)
        assert abs(g[j] - fd) <= 1e-6 * abs(fd) + 1e-9, (j, g[j], fd)


def test_step_loss_is_sum_of_squared_error():
    cfg = BiquadConfig(B=2, T=500)
    x, m = cfg.inputs(), cfg.modulation()
    tgt = noise(500, 2, 9)
    loss, _, y = O.biquad_step(x, m, [300.0, 500.0], [0.7, 0.9], tgt, grad=False, want_y=True, prec="f64")
    assert loss == pytest.approx(float(((y.astype(np.float64) - tgt) ** 2).sum()), rel=1e-6)
