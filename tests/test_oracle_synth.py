"""Pins of the oracle's config-3 synth forward (dgen_oracle_synth_fwd,
oracle/dgen_oracle.c synth_core) against closed forms of the reference graph
(Examples/HarmonicE2E/Synth.swift:47-102, nyquistNormalizedHarmonicsBatched
:158-167).  Each case is built so that the graph reduces to something the
mathematics fixes:

- one harmonic with constant controls is gain * uv * sin(2 pi phase);
- two harmonics are mixed in proportion to their amplitudes (renormalised);
- a harmonic exactly at sr/2 is masked (the reference's `<`), one below is not;
- a one-hot FIR tap i is the noise stream delayed by NF-1-i frames, times
  noise gain * 0.12 * noisePathScale, and zero before frame 0;
- control rows that are linear in the control frame interpolate to the
  (pinned) playhead;
- a non-finite control row zeroes exactly the frames whose lerp reads it.

The phase, noise and playhead used here are themselves pinned in
tests/test_oracle.py (reference known answers, exact integer recurrence).
CPU only."""
import numpy as np
import pytest

import oracle as O

SR = 16000.0


def _ctrl(B, F, K, NF, amps=None, gain=1.0, ngain=0.0, taps=None):
    """Control rows [B*F][K+2+NF] (row m = b*F + f), every row equal unless a
    per-(b, f) array is passed."""
    NC = K + 2 + NF
    c = np.zeros((B, F, NC), np.float64)
    if amps is not None:
        c[:, :, :K] = np.broadcast_to(np.asarray(amps, np.float64), (B, F, K))
    c[:, :, K] = np.broadcast_to(np.asarray(gain, np.float64), (B, F)) if np.ndim(gain) else gain
    c[:, :, K + 1] = np.broadcast_to(np.asarray(ngain, np.float64), (B, F)) if np.ndim(ngain) else ngain
    if taps is not None:
        c[:, :, K + 2:] = np.broadcast_to(np.asarray(taps, np.float64), (B, F, NF))
    return c.reshape(B * F, NC).astype(np.float32)


def _data(B, F, f0, uv=1.0):
    """f0, uv tables [F][B]: per-lane constants (or given [F][B] arrays)."""
    f0t = np.broadcast_to(np.asarray(f0, np.float32), (F, B)).astype(np.float32).copy()
    uvt = np.broadcast_to(np.asarray(uv, np.float32), (F, B)).astype(np.float32).copy()
    return f0t, uvt


def _sine(freq, T):
    """sin(2 pi phasor) of a constant frequency, through the pinned phasor."""
    ph = O.phasor(np.full(T, freq, np.float32), SR).astype(np.float64)
    return np.sin(2.0 * np.pi * ph)


def _f0_frames(f0, B, F, T):
    """Frame-rate f0 [B][T] through the pinned sampleRow lerp (fp32: a
    constant table can come back one ulp off at some frames)."""
    return O.lerp_frames(f0, B, F, T)


def _harm_sine(f0i, k):
    """sin(2 pi phasor) of harmonic k (1-based) of a per-frame f0 [T]."""
    freq = (np.float32(k) * f0i).astype(np.float32)
    return np.sin(2.0 * np.pi * O.phasor(freq, SR).astype(np.float64)), freq


def _exact_sine(freq, T):
    n = np.arange(T, dtype=np.float64)
    return np.sin(2.0 * np.pi * ((np.float64(np.float32(freq)) * n / SR) % 1.0))


def test_one_harmonic_is_a_scaled_sine():
    # lane 0: harmonic 3 of 220 Hz, gain 0.7, uv 1; lane 1: harmonic 1 of
    # 331 Hz, gain 1.3, uv 0.5 -- y = gain * uv * sin(2 pi phase) exactly
    # (den = 1 + 1e-8 rounds to 1 in fp32)
    B, F, T, K, NF = 2, 16, 1024, 5, 9
    amps = np.zeros((B, 1, K))
    amps[0, 0, 2] = 1.0
    amps[1, 0, 0] = 1.0
    gain = np.array([[0.7], [1.3]]) * np.ones((B, F))
    c = _ctrl(B, F, K, NF, amps=amps, gain=gain)
    f0, uv = _data(B, F, [220.0, 331.0], [1.0, 0.5])
    y = O.synth_fwd(c, f0, uv, B, F, T, K, NF, SR).astype(np.float64)
    ref0 = np.float32(0.7) * _sine(np.float32(3.0) * np.float32(220.0), T)
    ref1 = np.float32(1.3) * 0.5 * _sine(331.0, T)
    assert np.abs(y[0] - ref0).max() < 2e-6
    assert np.abs(y[1] - ref1).max() < 2e-6
    # and the closed form frac(f t / sr) within the fp32 phase drift
    assert np.abs(y[0] - np.float32(0.7) * _exact_sine(660.0, T)).max() < 2e-3
    assert np.abs(y[1] - np.float32(1.3) * 0.5 * _exact_sine(331.0, T)).max() < 2e-3


def test_harmonics_mix_in_proportion_to_their_amplitudes():
    # amps (1, 3) on harmonics 1 and 2: y = (s1 + 3 s2) / 4 (renormalised)
    B, F, T, K, NF = 1, 8, 512, 4, 5
    c = _ctrl(B, F, K, NF, amps=[1.0, 3.0, 0.0, 0.0], gain=2.0)
    f0, uv = _data(B, F, 200.0)
    y = O.synth_fwd(c, f0, uv, B, F, T, K, NF, SR)[0].astype(np.float64)
    ref = 2.0 * (_sine(200.0, T) + 3.0 * _sine(400.0, T)) / 4.0
    assert np.abs(y - ref).max() < 4e-6


def test_harmonic_at_nyquist_is_masked_and_the_rest_renormalised():
    # f0 = 4000 Hz at sr 16 kHz: harmonic 2 sits exactly on sr/2 and harmonic
    # 3 above it; both are masked (freq < nyquist is strict), so harmonic 1
    # alone carries the full gain.  With `<=` the output would halve.
    B, F, T, K, NF = 1, 4, 256, 3, 5
    c = _ctrl(B, F, K, NF, amps=[1.0, 1.0, 1.0], gain=1.0)
    f0, uv = _data(B, F, 4000.0)
    y = O.synth_fwd(c, f0, uv, B, F, T, K, NF, SR)[0].astype(np.float64)
    f0i = _f0_frames(f0, B, F, T)[0]
    s1, _ = _harm_sine(f0i, 1)
    s2, fr2 = _harm_sine(f0i, 2)
    on = fr2 == np.float32(8000.0)  # the fp32 lerp of a constant row is exact at most frames
    assert on.sum() > T // 2
    assert np.abs(y[on] - s1[on]).max() < 2e-6
    # where the lerp rounds f0 one ulp down, harmonic 2 drops below sr/2 and is kept
    assert np.abs(y[~on] - (s1[~on] + s2[~on]) / 2.0).max() < 2e-6
    # just below: harmonic 2 at 7999 Hz is kept, harmonic 3 (11998.5) is not
    f0b, uvb = _data(B, F, 3999.5)
    yb = O.synth_fwd(c, f0b, uvb, B, F, T, K, NF, SR)[0].astype(np.float64)
    f0ib = _f0_frames(f0b, B, F, T)[0]
    refb = (_harm_sine(f0ib, 1)[0] + _harm_sine(f0ib, 2)[0]) / 2.0
    assert np.abs(yb - refb).max() < 2e-6


@pytest.mark.parametrize("tap", [0, 3, 12])
def test_one_fir_tap_is_the_delayed_noise(tap):
    # harmonic gain 0, noise gain 2, one-hot tap i: the window is oldest
    # first and ends at the current frame, so y[t] = 2 * 0.12 * noise[t - (NF-1) + i]
    # (zero before frame 0); noisePathScale multiplies it
    B, F, T, K, NF = 1, 8, 600, 2, 13
    taps = np.zeros(NF)
    taps[tap] = 1.0
    for nscale in (1.0, 0.5):
        c = _ctrl(B, F, K, NF, amps=[1.0, 0.0], gain=0.0, ngain=2.0, taps=taps)
        f0, uv = _data(B, F, 300.0)
        y = O.synth_fwd(c, f0, uv, B, F, T, K, NF, SR, nscale=nscale)[0].astype(np.float64)
        noise = O.noise_stream(T).astype(np.float64)
        d = NF - 1 - tap
        ref = np.zeros(T)
        ref[d:] = noise[:T - d]
        ref *= 2.0 * np.float32(0.12) * nscale
        assert np.abs(y - ref).max() < 1e-7
        assert np.all(y[:d] == 0.0)


def test_noise_path_is_shared_by_lanes_and_harmonic_scale_applies():
    # two lanes with the same taps see the same noise stream; hscale scales
    # only the harmonic path
    B, F, T, K, NF = 2, 8, 400, 1, 4
    taps = [0.0, 0.0, 0.0, 1.0]
    c = _ctrl(B, F, K, NF, amps=[1.0], gain=1.0, ngain=1.0, taps=taps)
    f0, uv = _data(B, F, [250.0, 250.0])
    y = O.synth_fwd(c, f0, uv, B, F, T, K, NF, SR, hscale=0.25).astype(np.float64)
    noise = O.noise_stream(T).astype(np.float64)
    ref = 0.25 * _sine(250.0, T) + np.float32(0.12) * noise
    assert np.abs(y[0] - ref).max() < 1e-6
    assert np.array_equal(y[0], y[1])


def test_control_rows_interpolate_along_the_playhead():
    # noise gain row f of lane b = (b + 1) * (1 + f), a ramp: linear
    # interpolation between rows gives (b + 1) * (1 + playhead[t]) exactly;
    # uv row f = f / (F - 1) gives playhead / (F - 1) on the harmonic path
    B, F, T, K, NF = 2, 16, 1024, 1, 3
    f = np.arange(F, dtype=np.float64)
    ng = np.stack([(b + 1) * (1.0 + f) for b in range(B)])
    taps = [0.0, 0.0, 1.0]  # current frame's noise
    c = _ctrl(B, F, K, NF, amps=[1.0], gain=0.0, ngain=ng, taps=taps)
    f0, _ = _data(B, F, 500.0)
    uv = np.zeros((F, B), np.float32)
    y = O.synth_fwd(c, f0, uv, B, F, T, K, NF, SR).astype(np.float64)
    play = O.playhead(F, T).astype(np.float64)
    noise = O.noise_stream(T).astype(np.float64)
    for b in range(B):
        ref = np.float32(0.12) * noise * (b + 1) * (1.0 + play)
        assert np.abs(y[b] - ref).max() < 2e-6
    # harmonic path with a uv ramp
    c2 = _ctrl(B, F, K, NF, amps=[1.0], gain=1.0, ngain=0.0, taps=taps)
    uv2 = np.repeat((f / (F - 1))[:, None], B, axis=1).astype(np.float32)
    y2 = O.synth_fwd(c2, f0, uv2, B, F, T, K, NF, SR)[0].astype(np.float64)
    ref2 = _sine(500.0, T) * play / (F - 1)
    assert np.abs(y2 - ref2).max() < 2e-6


def test_f0_is_interpolated_per_lane_from_its_own_column():
    # f0 table [F][B]: lane 1 at 2x lane 0's frequency; with one harmonic the
    # two outputs are sines of the two pinned phase sequences
    B, F, T, K, NF = 2, 8, 512, 1, 3
    c = _ctrl(B, F, K, NF, amps=[1.0], gain=1.0)
    f0, uv = _data(B, F, [150.0, 300.0])
    y = O.synth_fwd(c, f0, uv, B, F, T, K, NF, SR).astype(np.float64)
    assert np.abs(y[0] - _sine(150.0, T)).max() < 2e-6
    assert np.abs(y[1] - _sine(300.0, T)).max() < 2e-6


def test_non_finite_control_row_zeroes_exactly_the_frames_that_read_it():
    # CRenderer.swift:1021-1039: every output store maps non-finite to 0.
    # A NaN gain in row f of lane 0 reaches exactly the frames whose lerp
    # reads row f (as lo or hi, whatever its weight); other frames and the
    # other lane keep their values.
    B, F, T, K, NF = 2, 8, 512, 1, 3
    taps = [0.0, 0.0, 1.0]
    c = _ctrl(B, F, K, NF, amps=[1.0], gain=1.0, ngain=1.0, taps=taps)
    f0, uv = _data(B, F, 200.0)
    clean = O.synth_fwd(c, f0, uv, B, F, T, K, NF, SR)
    bad = c.copy()
    row = 3
    bad[0 * F + row, K] = np.nan
    y = O.synth_fwd(bad, f0, uv, B, F, T, K, NF, SR)
    play = O.playhead(F, T)
    lo = np.floor(play).astype(int)
    hi = np.where(lo + 1 >= F, 0, lo + 1)
    hit = (lo == row) | (hi == row)
    assert hit.any() and (~hit).any()
    assert np.all(y[0][hit] == 0.0)
    assert np.array_equal(y[0][~hit], clean[0][~hit])
    assert np.array_equal(y[1], clean[1])
    # +inf gain with a zero sine (frame 0, phase 0) is NaN; elsewhere +-inf: all 0
    inf = c.copy()
    inf[0 * F + 0, K] = np.inf
    yi = O.synth_fwd(inf, f0, uv, B, F, T, K, NF, SR)
    assert np.all(yi[0][(lo == 0) | (hi == 0)] == 0.0)


def test_host_rate_drives_the_phase_and_graph_rate_the_nyquist_mask():
    # dgen_process_v1's context.sample_rate divides the phase increments
    # (u_phasor / hostSampleRate); the mask compares with the graph's
    # DGenConfig.sampleRate / 2.  f0 = 4000: harmonics 4000, 8000, 12000 Hz.
    B, F, T, K, NF = 1, 4, 256, 3, 5
    c = _ctrl(B, F, K, NF, amps=[1.0, 1.0, 1.0], gain=1.0)
    f0, uv = _data(B, F, 4000.0)
    f0i = _f0_frames(f0, B, F, T)[0]

    def sines(rate, k):
        freq = (np.float32(k) * f0i).astype(np.float32)
        return np.sin(2.0 * np.pi * O.phasor(freq, rate).astype(np.float64)), freq

    # graph rate 16 kHz masks harmonics 2 and 3 wherever 2*f0 is exactly 8000
    y = O.synth_fwd_rates(c, f0, uv, B, F, T, K, NF, 32000.0, 16000.0)[0].astype(np.float64)
    s1, _ = sines(32000.0, 1)
    s2, fr2 = sines(32000.0, 2)
    on = fr2 == np.float32(8000.0)
    assert on.sum() > T // 2
    assert np.abs(y[on] - s1[on]).max() < 2e-6
    # graph rate 32 kHz keeps harmonics 1..3 (all below 16 kHz)
    y2 = O.synth_fwd_rates(c, f0, uv, B, F, T, K, NF, 32000.0, 32000.0)[0].astype(np.float64)
    ref2 = (s1 + s2 + sines(32000.0, 3)[0]) / 3.0
    assert np.abs(y2 - ref2).max() < 2e-6
    # equal rates reduce to the plain forward
    assert np.array_equal(O.synth_fwd_rates(c, f0, uv, B, F, T, K, NF, SR, SR), O.synth_fwd(c, f0, uv, B, F, T, K,
                                                                                            NF, SR))
