"""Pins of the oracle's ZDF SVF bank (dgen_oracle_svf_fwd / _step), the
two-cell Cytomic/TPT low-pass of Tests/DGenLazyTests/SVFBPTTScratchTests.swift:
21-34.  Forward: the TPT low-pass magnitude |H| on a steady sinusoid, scipy's
lfilter of the prewarped bilinear transfer function, odd symmetry, the exact
2x scaling invariant of the saturation (x -> 2x, kSat -> kSat/2 doubles every
value bit for bit), and the small-signal limit.  Backward: central finite
differences of the fp64 build, with modulation, an envelope, saturation and
an active clip, plus the reference's own two SVF gradient setups
(SVFBPTTScratchTests.swift:56-108).  CPU only."""
import numpy as np
import scipy.signal as ss

import oracle as O

SR = 44100.0
PI32 = float(np.float32(np.pi))


def tpt_ba(fc, res, sr=SR):
    """H(z) of the linear SVF low-pass: H(s) = 1/(s^2 + s/res + 1) with
    s = (1/g)(1 - z^-1)/(1 + z^-1), g = tan(pi fc / sr)."""
    g = np.tan(np.float64(np.float32(PI32 * np.float32(fc)) / np.float32(sr)))
    k = 1.0 / res
    b = g * g * np.array([1.0, 2.0, 1.0])
    a = np.array([1 + k * g + g * g, 2 * (g * g - 1), 1 - k * g + g * g])
    return b / a[0], a / a[0], g


def test_steady_sinusoid_has_the_tpt_lowpass_magnitude():
    T = 12000
    n = np.arange(T)
    for fc, res in ((300.0, 0.707), (1000.0, 1.2), (5000.0, 3.0)):
        for f in (50.0, fc * 0.5, fc, fc * 2.0, 9000.0):
            w = 2 * np.pi * f / SR
            x = np.sin(w * n).astype(np.float32)
            y = O.svf_fwd(x[:, None], [fc], [res], prec="f64")[:, 0].astype(np.float64)
            # least-squares amplitude over the settled second half
            seg = slice(T // 2, T)
            A = np.stack([np.sin(w * n[seg]), np.cos(w * n[seg])], 1)
            coef, *_ = np.linalg.lstsq(A, y[seg], rcond=None)
            mag = np.hypot(*coef)
            _, _, g = tpt_ba(fc, res)
            ww = np.tan(w / 2) / g
            ref = 1.0 / np.sqrt((1 - ww * ww) ** 2 + (ww / res) ** 2)
            # x is a float32 sinusoid (quantisation ~3e-8 of full scale)
            assert abs(mag - ref) <= 1e-6 * max(ref, 1e-3), (fc, res, f, mag, ref)


def test_linear_bank_is_the_bilinear_transfer_function():
    rng = np.random.default_rng(3)
    T = 5000
    x = rng.uniform(-1, 1, (T, 3)).astype(np.float32)
    fcs, ress = [200.0, 2500.0, 12000.0], [0.5, 0.707, 4.0]
    y = O.svf_fwd(x, fcs, ress, prec="f64")
    for k in range(3):
        b, a, _ = tpt_ba(fcs[k], ress[k])
        ref = ss.lfilter(b, a, x[:, k].astype(np.float64))
        assert np.abs(y[:, k] - ref).max() < 1e-6
    y32 = O.svf_fwd(x, fcs, ress)
    assert np.abs(y32 - y).max() < 1e-4


def bank(T=3000, B=4, seed=5):
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (T, B)).astype(np.float32)
    m = np.exp2(rng.uniform(0, 3, T)).astype(np.float32)
    return x, m


def test_saturation_is_odd_and_scales_exactly():
    x, m = bank()
    base = np.array([150.0, 400.0, 1500.0, 6000.0], np.float32)
    res = np.array([0.6, 1.2, 2.0, 5.0], np.float32)
    ks = np.array([0.3, 1.2, 4.0, 0.05], np.float32)
    y = O.svf_fwd(x, base, res, ks, m)
    np.testing.assert_array_equal(O.svf_fwd(-x, base, res, ks, m), -y)
    np.testing.assert_array_equal(O.svf_fwd(2 * x, base, res, ks / 2, m), 2 * y)
    # kSat = 0 is the linear filter, and the constant-0 graph
    np.testing.assert_array_equal(O.svf_fwd(x, base, res, np.zeros(4, np.float32), m), O.svf_fwd(x, base, res, None, m))
    # small signals barely reach the saturation: the deviation from the
    # linear filter, relative to its output, falls in proportion to the level
    dev = []
    for level in (1e-3, 1e-4):
        lin = O.svf_fwd(level * x, base, res, None, m, prec="f64").astype(np.float64)
        sat = O.svf_fwd(level * x, base, res, ks, m, prec="f64").astype(np.float64)
        dev.append(np.abs(sat - lin).max() / np.abs(lin).max())
    assert dev[1] < 2e-3 and 0.05 < dev[1] / dev[0] < 0.2, dev
    # and large ones are compressed
    assert np.abs(O.svf_fwd(8 * x, base, res, ks, m)).max() < 8 * np.abs(O.svf_fwd(x, base, res, None, m)).max()


def test_state_carries_between_blocks():
    x, m = bank()
    base, res, ks = [300.0, 800.0, 2000.0, 7000.0], [0.707] * 4, [0.0, 0.5, 1.0, 2.0]
    one = O.svf_fwd(x, base, res, ks, m)
    st = np.zeros((2, 4), np.float32)
    a = O.svf_fwd(x[:1234], base, res, ks, m[:1234], state=st)
    b = O.svf_fwd(x[1234:], base, res, ks, m[1234:], state=st)
    np.testing.assert_array_equal(np.concatenate([a, b]), one)


def fd_grad(x, base, res, ks, tgt, m, env, which, k, eps):
    p = [np.array(base, np.float64), np.array(res, np.float64), None if ks is None else np.array(ks, np.float64)]
    out = []
    for sgn in (1, -1):
        q = [None if a is None else a.copy() for a in p]
        q[which][k] += sgn * eps
        out.append(O.svf_step(x, q[0], q[1], tgt, q[2], m, env, grad=False)[0])
    return (out[0] - out[1]) / (2 * eps)


def test_bptt_gradient_matches_finite_differences():
    x, m = bank(T=2500)
    env = (300.0 * np.exp(-np.arange(2500) / 400.0)).astype(np.float32)
    base = np.array([150.0, 400.0, 1500.0, 9000.0])
    res = np.array([0.6, 1.2, 2.0, 5.0])
    ks = np.array([0.3, 1.2, 0.0, 0.05])
    tgt = O.svf_fwd(x, [500.0] * 4, [1.0] * 4, None, None, prec="f64")
    for mm, ee in ((None, None), (m, None), (m, env)):
        _, g, _, _ = O.svf_step(x, base, res, tgt, ks, mm, ee)
        g = g.reshape(3, 4)
        for which in range(3):
            for k in range(4):
                p = (base, res, ks)[which][k]
                d = fd_grad(x, base, res, ks, tgt, mm, ee, which, k, 1e-5 * max(1.0, abs(p)))
                assert abs(g[which, k] - d) <= 1e-5 * max(abs(d), 1e-6), (which, k, g[which, k], d)
    # sign(0) = 0: no gradient reaches kSat at 0
    assert g[2, 2] == 0.0


def test_clipped_frames_pass_no_cutoff_gradient():
    # base * m crosses 20 kHz on part of the frames: those frames contribute
    # nothing (the clip's max/min masks), the rest match finite differences
    x, m = bank(T=2000)
    base = np.array([9000.0, 9000.0])
    res = np.array([0.8, 0.8])
    tgt = np.zeros((2000, 2), np.float32)
    x2 = x[:, :2]
    _, g, _, _ = O.svf_step(x2, base, res, tgt, None, m)
    d = fd_grad(x2, base, res, None, tgt, m, None, 0, 0, 1e-3)
    assert (m * 9000.0 > 20000.0).any() and (m * 9000.0 < 20000.0).any()
    assert abs(g[0] - d) <= 1e-5 * abs(d)
    # all frames clipped: zero gradient, finite differences agree
    _, g, _, _ = O.svf_step(x2, np.array([30000.0, 30000.0]), res, tgt, None, m)
    assert g[0] == 0.0 and g[1] == 0.0


def test_xbar_is_the_input_gradient():
    x, _ = bank(T=600, B=2)
    base, res, ks = np.array([700.0, 3000.0]), np.array([1.0, 2.0]), np.array([0.8, 0.0])
    tgt = np.zeros((600, 2), np.float32)
    _, _, _, xb = O.svf_step(x, base, res, tgt, ks, want_xbar=True)
    for n, k in ((0, 0), (123, 1), (599, 0), (300, 0)):
        eps = 1e-3
        # the oracle takes float32 x: the step is what float32 represents
        xp = x.copy()
        xm = x.copy()
        xp[n, k] += np.float32(eps)
        xm[n, k] -= np.float32(eps)
        h = (float(xp[n, k]) - float(xm[n, k])) / 2
        d = (O.svf_step(xp, base, res, tgt, ks, grad=False)[0] - O.svf_step(xm, base, res, tgt, ks, grad=False)[0]) / (2 * h)
        assert abs(xb[n, k] - d) <= 1e-4 * max(abs(d), 1e-3), (n, k, xb[n, k], d)
    # the input gradient alone (no parameter gradient requested)
    _, g, _, xb2 = O.svf_step(x, base, res, tgt, ks, grad=False, want_xbar=True)
    assert g is None
    np.testing.assert_array_equal(xb2, xb)


def reference_scene(T=512):
    """SVFBPTTScratchTests.swift:56-74: a 55 Hz saw (phasor * 2 - 1), the
    cutoff fBase + 900 exp(-t / 0.15) with t = accum(1/44100), kDamp = 1/1.2."""
    saw = (O.phasor(np.full(T, 55.0, np.float32), SR) * np.float32(2) - np.float32(1)).astype(np.float32)
    t = (np.arange(T, dtype=np.float64) / SR).astype(np.float32)
    env = (np.float32(900.0) * np.exp(-t / np.float32(0.15))).astype(np.float32)
    return saw[:, None], env


def test_reference_time_varying_cutoff_setup():
    # testTimeVaryingCutoffGradientMatchesFD (:84-101): fBase 300 -> target 400, eps 0.5, 5% there
    x, env = reference_scene()
    tgt = O.svf_fwd(x, [400.0], [1.2], None, None, env, prec="f64")
    _, g, _, _ = O.svf_step(x, [300.0], [1.2], tgt, None, None, env)
    d = fd_grad(x, [300.0], [1.2], None, tgt, None, env, 0, 0, 0.5)
    assert abs(g[0] - d) <= 1e-4 * abs(d)
    assert g[0] < 0  # the student's cutoff is below the target's


def test_reference_filter_saturation_setup():
    # testFiltSatGradientMatchesFD (:103-120): kSat 1.0 against a kSat 0 target, eps 1e-2
    x, env = reference_scene()
    tgt = O.svf_fwd(x, [400.0], [1.2], None, None, env, prec="f64")
    _, g, _, _ = O.svf_step(x, [300.0], [1.2], tgt, [1.0], None, env)
    d = fd_grad(x, [300.0], [1.2], [1.0], tgt, None, env, 2, 0, 1e-2)
    assert abs(g[2] - d) <= 1e-3 * abs(d)
