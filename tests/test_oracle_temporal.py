"""Pins of the oracle's temporal gradient (dgen_oracle_temporal_scan,
dgen_oracle_swept_phasor_step): the reset-aware exclusive suffix scan of
Emit+TemporalGradient.swift:56-81 against its closed form, and the swept
phasor bank's gradient against central finite differences of the fp64
build, with and without resets, including the reference's own
TemporalGradientTests.swift:24-60 setup.  CPU only."""
import numpy as np

import oracle as O

SR = 44100.0


def closed_form_scan(g, reset):
    """out[n] = 0 at a reset frame, else the sum of g over (n, r] with r the
    next reset frame after n (or the last frame)."""
    T, E = g.shape
    out = np.zeros((T, E))
    rs = np.zeros(T, bool) if reset is None else reset > 0
    for n in range(T):
        if rs[n]:
            continue
        r = n + 1
        while r < T and not rs[r]:
            r += 1
        out[n] = g[n + 1:min(r + 1, T)].astype(np.float64).sum(axis=0)
    return out


def test_scan_without_resets_is_the_exclusive_suffix_sum():
    rng = np.random.default_rng(0)
    g = rng.standard_normal((3000, 5)).astype(np.float32)
    got = O.temporal_scan(g)
    ref = np.concatenate([np.cumsum(g[::-1].astype(np.float64), axis=0)[::-1][1:], np.zeros((1, 5))])
    assert np.abs(got - ref).max() < 1e-4 * np.abs(ref).max()


def test_scan_resets_cut_the_suffix_sums():
    rng = np.random.default_rng(1)
    g = rng.standard_normal((400, 3)).astype(np.float32)
    for reset in (np.zeros(400, np.float32), (np.arange(400) % 37 == 5).astype(np.float32),
                  (np.arange(400) >= 200).astype(np.float32), np.ones(400, np.float32)):
        got = O.temporal_scan(g, reset)
        assert np.abs(got - closed_form_scan(g, reset)).max() < 1e-4
    assert not O.temporal_scan(g, np.ones(400, np.float32)).any()


def fd(slope, i, eps, T, reset_from, smooth=False):
    p, m = slope.copy(), slope.copy()
    p[i] += eps
    m[i] -= eps
    lp = O.swept_phasor_step(p, T, SR, 80.0, 0.08, reset_from, smooth, grad=False)[0]
    lm = O.swept_phasor_step(m, T, SR, 80.0, 0.08, reset_from, smooth, grad=False)[0]
    return (lp - lm) / (2 * eps)


def test_reference_swept_phasor_setup():
    # TemporalGradientTests.swift:24-60: 128 frames, slope 1200, epsilon 1,
    # agreement within 2% there; exact in the fp64 build
    slope = np.array([1200.0])
    _, g, _ = O.swept_phasor_step(slope, 128, SR, 80.0, 0.08)
    d = fd(slope, 0, 1.0, 128, -1)
    assert abs(g[0] - d) <= 1e-6 * abs(d)


def test_swept_phasor_bank_gradient_matches_finite_differences_across_resets():
    slope = np.array([900.0, 1200.0, 3000.0, 25000.0])
    for T, reset_from in ((2000, -1), (2000, 1000), (500, 0)):
        _, g, _ = O.swept_phasor_step(slope, T, SR, 80.0, 0.08, reset_from)
        for i in range(len(slope)):
            d = fd(slope, i, 1e-3, T, reset_from)
            assert abs(g[i] - d) <= 1e-6 * max(abs(d), 1e-12), (T, reset_from, i, g[i], d)
        if reset_from == 0:
            assert not g.any()  # every increment discarded


def test_fp32_build_is_the_reference_semantics():
    slope = np.array([1200.0, 5000.0], np.float32)
    l32, g32, p32 = O.swept_phasor_step(slope, 4000, SR, 80.0, 0.08, 2500, want_phase=True, prec="f32")
    l64, g64, p64 = O.swept_phasor_step(slope, 4000, SR, 80.0, 0.08, 2500, want_phase=True, prec="f64")
    assert np.abs(p32 - p64).max() < 1e-4
    assert np.abs(g32 - g64).max() < 1e-3 * np.abs(g64).max()
    assert np.all(p32[2500:] == 0.0) or np.all(p32[2501:] == 0.0)


def test_smooth_loss_over_a_long_run_matches_finite_differences():
    # sin(2 pi phase) keeps the loss continuous across the phase's wraps, so
    # central differences stay meaningful over 2^16 frames (~100 wraps).  The
    # gradient is a sum of terms ~1e5 that cancel to 2..500, and the fp64
    # phase recursion's rounding differs between the two perturbed runs: the
    # differences scatter ~3e-4 around the analytic value at eps = 1e-7 slope
    slope = np.array([600.0, 5000.0, 24000.0])
    T = 1 << 16
    for reset_from in (-1, 40000):
        _, g, _ = O.swept_phasor_step(slope, T, SR, 80.0, 0.08, reset_from, True)
        for i in range(len(slope)):
            d = fd(slope, i, 1e-7 * slope[i], T, reset_from, True)
            assert abs(g[i] - d) <= 1e-3 * abs(d), (reset_from, i, g[i], d)
