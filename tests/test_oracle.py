"""Pins of the CPU oracle (oracle/dgen_oracle.c) against the reference's own
known answers, independent libraries (numpy.fft), closed forms and central
finite differences.  CPU only."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import HarmonicConfig


# ---------------------------------------------------------------- known answers
def test_stateful_phasor_known_answers():
    # Tests/DGenLazyTests/CBackendTests.swift:46-59: 100 Hz at sr 1000
    out = O.phasor(np.full(12, 100.0), 1000.0)
    for n, v in ((0, 0.0), (1, 0.1), (5, 0.5), (9, 0.9)):
        assert abs(out[n] - v) < 1e-4
    # pre-increment output: the first frame is the initial state
    assert out[0] == 0.0


def test_stateful_phasor_matches_exact_phase_sum():
    # fp32 accumulation stays within a few ulp-steps of the exact phase
    rng = np.random.default_rng(0)
    f = rng.uniform(20.0, 2000.0, 5000).astype(np.float32)
    out = O.phasor(f, 16000.0).astype(np.float64)
    inc = f.astype(np.float64) / 16000.0
    exact = np.concatenate([[0.0], np.cumsum(inc)[:-1]]) % 1.0
    d = np.abs(out - exact)
    d = np.minimum(d, 1.0 - d)  # circular distance
    assert d.max() < 5e-4


def test_sine_known_answers():
    # CBackendTests.swift:61-76: 1 Hz at sr 4 -> 0, 1, 0, -1
    out = O.oscbank(np.array([1.0]), np.array([1.0]), 4.0, 0.0, 4)
    np.testing.assert_allclose(out, [0.0, 1.0, 0.0, -1.0], atol=1e-4)


def test_onepole_is_convolution_with_geometric_kernel():
    # y[n] = x[n] + p y[n-1]  <=>  y = x * (p^k)_k ; x = sin of a 3-osc bank
    freqs = np.array([110.0, 220.0, 330.0], np.float32)
    amps = np.array([0.5, 0.3, 0.2], np.float32)
    sr, p, T = 44100.0, 0.9, 4096
    y = O.oscbank(freqs, amps, sr, p, T).astype(np.float64)
    n = np.arange(T)
    x = sum(a * np.sin(2 * np.pi * ((f / sr * n) % 1.0)) for f, a in zip(freqs.astype(np.float64), amps))
    ref = np.convolve(x, p ** np.arange(T))[:T]
    assert np.abs(y - ref).max() < 1e-4


def test_oscbank_config1_inputs():
    # benchmark config 1: 16 phasors at k * 220 Hz, amps normalised to sum 1
    freqs = (np.arange(1, 17) * 220.0).astype(np.float32)
    rng = np.random.default_rng(1)
    amps = rng.uniform(0, 1, 16).astype(np.float32)
    amps /= amps.sum()
    y = O.oscbank(freqs, amps, 44100.0, 0.9, 2048)
    assert np.isfinite(y).all() and np.abs(y).max() < 10.0


def test_noise_bit_exact():
    # xorshift32 on a zeroed state (0 -> 1), u = s / 2^32 (CRenderer.swift:685-693)
    T = 2000
    s, ref = 0, []
    for _ in range(T):
        if s == 0:
            s = 1
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        ref.append(np.float32(np.float32(s) / np.float32(4294967296.0)))
    np.testing.assert_array_equal(O.noise_stream(T), np.array(ref, np.float32))


def test_playhead_properties():
    F, T = 100, 6400
    p = O.playhead(F, T).astype(np.float64)
    step = np.float32(F - 1) / np.float32(T - 1)
    assert p[0] == 0.0 and p[1] == np.float32(step)
    assert p.min() >= 0.0 and p.max() <= F - 1 - 1e-4 + 1e-6
    ideal = np.arange(T) * (F - 1) / (T - 1)
    body = slice(0, T - 64)
    assert np.abs(p[body] - ideal[body]).max() < 0.05
    assert np.all(np.diff(p[body]) > 0)


def test_lerp_frames_of_a_ramp_is_the_playhead():
    # sampleRow of src[f][b] = f + 100 b gives the playhead (plus 100 b), except
    # where the upper row wraps to row 0 (Emit+RowSelection.swift:170-197)
    B, F, T = 3, 40, 2560
    src = (np.arange(F)[:, None] + 100.0 * np.arange(B)[None, :]).astype(np.float32)
    out = O.lerp_frames(src, B, F, T).astype(np.float64)
    p = O.playhead(F, T).astype(np.float64)
    lo = np.floor(p)
    wrap = lo + 1 >= F
    for b in range(B):
        ref = np.where(wrap, (1 - (p - lo)) * (lo + 100 * b) + (p - lo) * (100 * b), p + 100 * b)
        assert np.abs(out[b] - ref).max() < 1e-3


def test_one_control_row_is_read_by_every_frame():
    # F = 1: the playhead stays at row 0 (step 0, and the accumulator's wrap
    # span is 1, as the schedule's accumulator table is set up), so every
    # frame reads the single row exactly
    B, T = 3, 100
    src = np.array([[430.25, -1.5, 0.0]], np.float32)
    assert not O.playhead(1, T).any()
    np.testing.assert_array_equal(O.lerp_frames(src, B, 1, T), np.repeat(src[0][:, None], T, 1))


def test_phase_checkpoints_follow_the_phasor():
    B, K, T, sr = 2, 5, 700, 16000.0
    rng = np.random.default_rng(2)
    f0f = rng.uniform(60, 1000, (B, T)).astype(np.float32)
    ck = O.phase_checkpoints(f0f, B, K, T, sr)
    for b in range(B):
        for k in range(K):
            seq = O.phasor((np.float32(k + 1) * f0f[b]).astype(np.float32), sr)
            np.testing.assert_array_equal(ck[:, b, k], seq[::64])


# ---------------------------------------------------------------- spectral loss
def np_mss(x, tgt, sizes, w_lin, w_log, max_frames, mode=0, w_mse=0.0):
    """Multi-scale spectral loss per frame with numpy.fft: windows end at the
    hop frame (zero before 0), symmetric Hann (all ones with
    MSS_RECT_WINDOW), bins 0..N/2; the magnitude term and the term on
    log(magnitude + 1e-8) (with MSS_SMOOTH_LOG on 0.5 log(|X|^2 + 1e-16)),
    each L1 or (MSS_L2_*) L2; batch mean, / maxFrames; plus the time-domain
    term w_mse * sum_b (x - tgt)^2 / B per frame."""
    x = np.asarray(x, np.float64)
    tgt = np.asarray(tgt, np.float64)
    B, T = x.shape
    lf = w_mse * ((x - tgt) ** 2).sum(0) / B
    for N in sizes:
        H = N // 4
        hann = np.ones(N) if mode & O.MSS_RECT_WINDOW else 0.5 * (1 - np.cos(2 * np.pi * np.arange(N) / (N - 1)))
        frames = np.arange(0, T, H)
        idx = frames[:, None] - (N - 1) + np.arange(N)[None, :]
        valid = idx >= 0
        idc = np.clip(idx, 0, T - 1)
        lin = np.zeros(len(frames))
        lg = np.zeros(len(frames))
        for b in range(B):
            X = np.fft.rfft(np.where(valid, x[b][idc], 0.0) * hann, axis=1)
            Y = np.fft.rfft(np.where(valid, tgt[b][idc], 0.0) * hann, axis=1)
            dlin = np.abs(X) - np.abs(Y)
            if mode & O.MSS_SMOOTH_LOG:
                dlog = 0.5 * (np.log(np.abs(X) ** 2 + 1e-16) - np.log(np.abs(Y) ** 2 + 1e-16))
            else:
                dlog = np.log(np.abs(X) + 1e-8) - np.log(np.abs(Y) + 1e-8)
            lin += (dlin ** 2 if mode & O.MSS_L2_LIN else np.abs(dlin)).sum(1)
            lg += (dlog ** 2 if mode & O.MSS_L2_LOG else np.abs(dlog)).sum(1)
        lf[frames] += (lin / B / max_frames) * (w_lin / len(sizes)) + (lg / B / max_frames) * (w_log / len(sizes))
    return lf


MODES = [0, O.MSS_L2_LIN | O.MSS_L2_LOG, O.MSS_SMOOTH_LOG, O.MSS_L2_LOG | O.MSS_SMOOTH_LOG | O.MSS_RECT_WINDOW,
         O.MSS_RECT_WINDOW]


@pytest.fixture(scope="module")
def signals():
    rng = np.random.default_rng(7)
    B, T = 2, 2048
    x = (0.3 * rng.standard_normal((B, T))).astype(np.float32)
    t = (0.3 * rng.standard_normal((B, T))).astype(np.float32)
    return B, T, x, t


@pytest.mark.parametrize("mode", MODES)
def test_spectral_loss_matches_numpy_fft(signals, mode):
    B, T, x, t = signals
    sizes = (512, 256, 128, 64)
    w_mse = 0.25 if mode else 0.0
    tot, lf = O.mss_fwd(x, t, B, T, sizes, 4, 1.0, 0.5, T, prec="f64", frames=True, mode=mode, w_mse=w_mse)
    ref = np_mss(x, t, sizes, 1.0, 0.5, T, mode=mode, w_mse=w_mse)
    assert abs(tot - ref.sum()) / ref.sum() < 1e-6
    np.testing.assert_allclose(lf, ref, rtol=1e-5, atol=1e-12)


@pytest.mark.parametrize("mode", [O.MSS_SMOOTH_LOG, O.MSS_SMOOTH_LOG | O.MSS_L2_LOG, 0])
def test_spectral_log_terms_near_the_epsilon(mode):
    """Signals of amplitude ~1e-9 put |X| near the 1e-8 epsilon, where the
    smooth log magnitude 0.5 log(|X|^2 + eps^2) and log(|X| + eps) differ by
    up to log(sqrt 2): the oracle follows the mode's formula there."""
    rng = np.random.default_rng(17)
    B, T = 2, 1024
    x = (1e-9 * rng.standard_normal((B, T))).astype(np.float32)
    t = (3e-9 * rng.standard_normal((B, T))).astype(np.float32)
    sizes = (256, 64)
    tot, lf = O.mss_fwd(x, t, B, T, sizes, 4, 0.0, 1.0, T, prec="f64", frames=True, mode=mode)
    ref = np_mss(x, t, sizes, 0.0, 1.0, T, mode=mode)
    other = np_mss(x, t, sizes, 0.0, 1.0, T, mode=mode ^ O.MSS_SMOOTH_LOG)
    assert abs(tot - ref.sum()) / ref.sum() < 1e-6
    assert abs(other.sum() - ref.sum()) / ref.sum() > 1e-3  # the two forms differ here (1000x the bar)


@pytest.mark.parametrize("mode", MODES)
def test_spectral_loss_of_identical_signals_is_zero(signals, mode):
    # TensorFFTTests.swift:1057-1098: same signal -> zero loss per bin
    B, T, x, _ = signals
    sizes = (256, 64)
    assert O.mss_fwd(x, x, B, T, sizes, 4, 1.0, 0.5, T, mode=mode, w_mse=0.5) == 0.0
    assert np.all(O.mss_bwd(x, x, B, T, sizes, 4, 1.0, 0.5, T, mode=mode, w_mse=0.5) == 0.0)


@pytest.mark.parametrize("mode", MODES)
def test_spectral_gradient_matches_finite_differences(signals, mode):
    B, T, x, t = signals
    sizes = (256, 128, 64)
    w_mse = 0.25 if mode else 0.0
    g = O.mss_bwd(x, t, B, T, sizes, 4, 1.0, 0.5, T, prec="f64", mode=mode, w_mse=w_mse).astype(np.float64)
    rng = np.random.default_rng(3)
    x64 = x.astype(np.float64)
    # directional derivatives with a step far below the distance to the
    # loss's kinks (|m1 - m2| and log-term sign changes)
    for _ in range(3):
        v = rng.standard_normal((B, T))
        eps = 1e-7
        lp = O.mss_fwd_x64(x64 + eps * v, t, B, T, sizes, 4, 1.0, 0.5, T, mode=mode, w_mse=w_mse)
        lm = O.mss_fwd_x64(x64 - eps * v, t, B, T, sizes, 4, 1.0, 0.5, T, mode=mode, w_mse=w_mse)
        fd = (lp - lm) / (2 * eps)
        an = float((g * v).sum())
        assert abs(fd - an) / abs(an) < 1e-5, (fd, an)


def test_mse_term_closed_form(signals):
    """Trainer.swift:547-551: w * sum_b (x - t)^2 / B per frame; gradient
    2 w (x - t) / B."""
    B, T, x, t = signals
    tot, lf = O.mss_fwd(x, t, B, T, (64,), 4, 0.0, 0.0, T, prec="f64", frames=True, w_mse=0.75)
    d = x.astype(np.float64) - t
    np.testing.assert_allclose(lf, 0.75 * (d * d).sum(0) / B, rtol=1e-6)
    g = O.mss_bwd(x, t, B, T, (64,), 4, 0.0, 0.0, T, prec="f64", w_mse=0.75)
    np.testing.assert_allclose(g, 0.75 * 2 * d / B, rtol=1e-6)


# ---------------------------------------------------------------- control network + whole step
def small_cfg():
    return HarmonicConfig(B=2, T=1024, hidden=16, fft_sizes=(256, 128, 64))


def np_mlp(cfg, X, P):
    """Independent numpy forward of the decoder (Model.swift:96-120)."""
    P = np.asarray(P, np.float64)
    h = np.asarray(X, np.float64)
    off, fan = 0, cfg.din
    for _ in range(cfg.layers):
        W = P[off:off + fan * cfg.hidden].reshape(fan, cfg.hidden)
        b = P[off + fan * cfg.hidden:off + fan * cfg.hidden + cfg.hidden]
        h = np.tanh(h @ W + b)
        off += fan * cfg.hidden + cfg.hidden
        fan = cfg.hidden
    Wh = P[off:off + cfg.hidden * cfg.NC].reshape(cfg.hidden, cfg.NC)
    bh = P[off + cfg.hidden * cfg.NC:]
    z = h @ Wh + bh
    sp = np.logaddexp(0.0, z)
    K, NF = cfg.K, cfg.NF
    amps = sp[:, :K] / (sp[:, :K].sum(1, keepdims=True) + 1e-6)
    taps = np.tanh(z[:, K + 2:])
    taps = taps / (np.abs(taps).sum(1, keepdims=True) + 1e-4)
    return np.concatenate([amps, sp[:, K:K + 2], taps], axis=1)


def test_mlp_matches_numpy():
    cfg = small_cfg()
    f0, uv, X = cfg.data()
    P = cfg.weights()
    got = O.mlp_fwd(X, P, cfg.M, cfg.din, cfg.hidden, cfg.layers, cfg.K, cfg.NF, prec="f64")
    np.testing.assert_allclose(got, np_mlp(cfg, X, P), rtol=1e-5, atol=1e-7)


def test_parameter_count_matches_layout():
    cfg = HarmonicConfig()
    assert O.mlp_param_count(cfg.din, cfg.hidden, cfg.layers, cfg.NC) == cfg.param_count() == len(cfg.weights())
    # 2->512->512->512 trunk and 512 -> (60 + 2 + 65) heads
    assert cfg.param_count() == (2 * 512 + 512) + 2 * (512 * 512 + 512) + 512 * 127 + 127


def test_whole_step_gradient_matches_finite_differences():
    """d sum_frames(loss) / d params of the fp64 oracle against central
    differences of its own forward along random directions."""
    cfg = small_cfg()
    f0, uv, X = cfg.data()
    tgt = O.harmonic_step(cfg, X, cfg.weights(seed=cfg.target_seed), f0, uv, np.zeros((cfg.B, cfg.T), np.float32),
                          grad=False, want_y=True, prec="f32")[2]
    P = cfg.weights().astype(np.float64)
    _, g, _ = O.harmonic_step(cfg, X, P, f0, uv, tgt, grad=True, prec="f64")
    rng = np.random.default_rng(11)
    for _ in range(3):
        v = rng.standard_normal(len(P))
        v /= np.linalg.norm(v)
        eps = 1e-6
        lp = O.harmonic_step(cfg, X, P + eps * v, f0, uv, tgt, grad=False, prec="f64")[0]
        lm = O.harmonic_step(cfg, X, P - eps * v, f0, uv, tgt, grad=False, prec="f64")[0]
        fd = (lp - lm) / (2 * eps)
        an = float(g @ v)
        assert abs(fd - an) / abs(an) < 1e-4, (fd, an)


def test_single_parameter_gradients_match_finite_differences():
    cfg = small_cfg()
    f0, uv, X = cfg.data()
    tgt = O.harmonic_step(cfg, X, cfg.weights(seed=cfg.target_seed), f0, uv, np.zeros((cfg.B, cfg.T), np.float32),
                          grad=False, want_y=True, prec="f32")[2]
    P = cfg.weights().astype(np.float64)
    _, g, _ = O.harmonic_step(cfg, X, P, f0, uv, tgt, grad=True, prec="f64")
    for i in np.argsort(-np.abs(g))[:6]:  # the largest components: harmonic and tap heads, biases
        e = np.zeros_like(P)
        e[i] = 1e-7
        fd = (O.harmonic_step(cfg, X, P + e, f0, uv, tgt, grad=False, prec="f64")[0]
              - O.harmonic_step(cfg, X, P - e, f0, uv, tgt, grad=False, prec="f64")[0]) / 2e-7
        assert abs(fd - g[i]) <= 1e-3 * abs(g[i]) + 1e-9, (i, fd, g[i])


def test_adam_closed_form():
    # Optimizers.swift:164-204 with bias corrections at step t
    rng = np.random.default_rng(4)
    n = 1000
    p, g = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    m, v = (0.1 * rng.standard_normal(n)).astype(np.float32), rng.uniform(0, 0.1, n).astype(np.float32)
    lr, b1, b2, eps, t = 1e-3, 0.9, 0.999, 1e-8, 3
    p2, m2, v2 = O.adam(p, g, m, v, lr, b1, b2, eps, t, prec="f64")
    # the hyper-parameters cross the C boundary as fp32 (Float in the reference)
    lr, b1, b2, eps = (float(np.float32(c)) for c in (lr, b1, b2, eps))
    mr = b1 * m.astype(np.float64) + (1 - b1) * g
    vr = b2 * v.astype(np.float64) + (1 - b2) * g.astype(np.float64) ** 2
    pr = p - lr * (mr / (1 - b1 ** t)) / (np.sqrt(vr / (1 - b2 ** t)) + eps)
    np.testing.assert_allclose(m2, mr, rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(v2, vr, rtol=1e-6, atol=1e-10)
    np.testing.assert_allclose(p2, pr, rtol=1e-5, atol=1e-7)
