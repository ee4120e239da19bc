"""Pins of the config-2 STFT oracle (oracle/dgen_oracle.c, tf_* and
dgen_oracle_stft_step): the reference's tensorFFT known answers
(Tests/DGenLazyTests/TensorFFTTests.swift), numpy.fft, the overlap-add and
STFT-identity closed forms, and central finite differences.  CPU only."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import StftConfig


# ---------------------------------------------------------------- tensorFFT
def test_fft_impulse_dc_cosine_parseval_roundtrip():
    # TensorFFTTests.swift:23-121, 229-245 (N = 8)
    N = 8
    re, im = O.tensor_fft([1, 0, 0, 0, 0, 0, 0, 0])
    np.testing.assert_allclose(re, 1.0, atol=1e-12)
    np.testing.assert_allclose(im, 0.0, atol=1e-12)
    re, im = O.tensor_fft(np.ones(N))
    assert abs(re[0] - N) < 1e-12 and np.abs(re[1:]).max() < 1e-6 and np.abs(im).max() < 1e-6
    c = np.cos(2 * np.pi * np.arange(N) / N)
    re, im = O.tensor_fft(c)
    assert abs(re[1] - N / 2) < 1e-6 and abs(re[N - 1] - N / 2) < 1e-6 and abs(re[0]) < 1e-6
    assert np.abs(im).max() < 1e-6
    d = np.array([3, 1, 4, 1, 5, 9, 2, 6], float)
    re, im = O.tensor_fft(d)
    # the twiddles are fp32 values (computed in Float), so the transform is
    # unitary only to fp32 level even in the fp64 build
    assert abs((re ** 2 + im ** 2).sum() / N - (d ** 2).sum()) < 1e-6 * (d ** 2).sum()
    rr, _ = O.tensor_fft(re, im, inverse=True)
    np.testing.assert_allclose(rr, d, atol=1e-6)
    rr32, _ = O.tensor_fft(*O.tensor_fft(d, prec="f32"), inverse=True, prec="f32")
    np.testing.assert_allclose(rr32, d, atol=1e-5)


@pytest.mark.parametrize("N", [2, 64, 1024])
def test_fft_matches_numpy(N):
    rng = np.random.default_rng(N)
    a = rng.standard_normal(N) + 1j * rng.standard_normal(N)
    re, im = O.tensor_fft(a.real, a.imag)
    ref = np.fft.fft(a)
    # twiddles are fp32 values (computed in Float), so agreement is to fp32 level
    assert np.abs(re + 1j * im - ref).max() < 1e-6 * np.abs(ref).max() * np.log2(N)
    re, im = O.tensor_fft(a.real, a.imag, inverse=True)
    ref = np.fft.ifft(a)
    assert np.abs(re + 1j * im - ref).max() < 1e-6 * np.abs(ref).max() * np.log2(N)


# ---------------------------------------------------------------- overlap-add / identity
def test_overlap_add_of_constant_rectangular_windows():
    # TensorFFTTests.swift:531-561: constant 1, rectangular window -> N/H
    N, H, T = 64, 16, 512
    loss, _, y = O.stft_step(np.ones((1, T)), N, H, np.ones(N), np.ones(N // 2 + 1), grad=False, want_y=True)
    np.testing.assert_allclose(y[0, N:], N / H, atol=1e-9)


def test_stft_identity_is_twice_the_input_delayed_by_n_minus_1():
    # periodic Hann at 75% overlap sums to 2; latency N-1 (STFTIdentityTests.swift:152-187)
    cfg = StftConfig(S=2, T=6000, N=256, H=64)
    x = cfg.inputs()
    _, _, y = O.stft_step(x, cfg.N, cfg.H, cfg.window(), cfg.gains(), grad=False, want_y=True)
    np.testing.assert_allclose(y[:, :cfg.N - 1], 0.0, atol=1e-6)  # fp32-valued twiddles leak ~1e-7
    np.testing.assert_allclose(y[:, cfg.N - 1:], 2.0 * x[:, :cfg.T - cfg.N + 1], atol=1e-6)


def test_gained_round_trip_matches_numpy_pipeline():
    N, H, T = 128, 32, 1000
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, T)).astype(np.float32)
    g = rng.uniform(0.2, 1.8, N // 2 + 1)
    win = StftConfig(N=N).window()
    _, _, y = O.stft_step(x, N, H, win, g, grad=False, want_y=True)
    gfull = np.zeros(N)
    gfull[0], gfull[N // 2] = g[0], g[N // 2]
    gfull[1:N // 2] = 2 * g[1:N // 2]
    ref = np.zeros((2, T))
    for s in range(2):
        xp = np.concatenate([np.zeros(N - 1), x[s].astype(np.float64)])
        for h in range(0, T, H):
            z = np.fft.ifft(np.fft.fft(win * xp[h:h + N]) * gfull).real
            n = min(N, T - h)
            ref[s, h:h + n] += z[:n]
    assert np.abs(y - ref).max() < 1e-5 * np.abs(ref).max()


def test_loss_is_mean_over_frames_summed_over_signals():
    cfg = StftConfig(S=3, T=700, N=64, H=16)
    x = cfg.inputs()
    loss, _, y = O.stft_step(x, cfg.N, cfg.H, cfg.window(), cfg.gains(), grad=False, want_y=True)
    assert loss == pytest.approx(float(((y.astype(np.float64) - x) ** 2).sum() / cfg.T), rel=1e-6)


def test_fp32_build_close_to_fp64():
    cfg = StftConfig(S=2, T=1 << 14)
    x = cfg.inputs()
    g = np.random.default_rng(3).uniform(0.5, 1.5, cfg.bins)
    _, _, y32 = O.stft_step(x, cfg.N, cfg.H, cfg.window(), g, grad=False, want_y=True, prec="f32")
    _, _, y64 = O.stft_step(x, cfg.N, cfg.H, cfg.window(), g, grad=False, want_y=True, prec="f64")
    assert np.abs(y32 - y64).max() < 1e-5


# ---------------------------------------------------------------- gradient
def test_gain_gradient_matches_central_differences():
    cfg = StftConfig(S=2, T=1500, N=64, H=16)
    x = cfg.inputs()
    win = cfg.window()
    g = np.random.default_rng(11).uniform(0.5, 1.5, cfg.bins)
    _, dg, _ = O.stft_step(x, cfg.N, cfg.H, win, g)
    for k in (0, 1, 7, cfg.N // 4, cfg.N // 2 - 1, cfg.N // 2):
        e = np.zeros_like(g)
        e[k] = 1e-6
        fd = (O.stft_step(x, cfg.N, cfg.H, win, g + e, grad=False)[0]
              - O.stft_step(x, cfg.N, cfg.H, win, g - e, grad=False)[0]) / 2e-6
        assert abs(dg[k] - fd) <= 1e-6 * abs(fd) + 1e-10, (k, dg[k], fd)
    u = dg / np.linalg.norm(dg)
    fd = (O.stft_step(x, cfg.N, cfg.H, win, g + 1e-6 * u, grad=False)[0]
          - O.stft_step(x, cfg.N, cfg.H, win, g - 1e-6 * u, grad=False)[0]) / 2e-6
    assert abs(dg @ u - fd) <= 1e-6 * abs(fd)
