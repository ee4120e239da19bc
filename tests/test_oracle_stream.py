"""Pins of the oracle's streaming blocks (dgen_oracle_oscbank_stream,
dgen_oracle_biquad_stream): a dgen_process_v1 call with preserveState
(Sources/DGenLazy/Realize.swift:553-563) carries the graph's state cells
from one call to the next.  Checked against closed forms (phase sums, the
one-pole's geometric kernel and its linearity), scipy.signal.lfilter with a
carried initial state, and the invariant that any split of a run into calls
gives the same samples.  CPU only."""
import numpy as np
import scipy.signal as ss

import oracle as O

SR = 44100.0


def bank():
    freqs = (np.arange(1, 17, dtype=np.float32) * np.float32(220.0)).astype(np.float32)
    rng = np.random.default_rng(1)
    amps = rng.uniform(0, 1, 16).astype(np.float32)
    return freqs, (amps / amps.sum()).astype(np.float32)


def run_calls(freqs, amps, sizes, stateful):
    st = np.zeros(len(freqs) + 1, np.float32)
    return np.concatenate([O.oscbank_stream(freqs, amps, SR, 0.9, n, stateful, st) for n in sizes]), st


def test_stateful_bank_is_the_phase_sum_through_the_one_pole():
    freqs, amps = bank()
    T = 4096
    y, st = run_calls(freqs, amps, [T], 1)
    x = sum(a * np.sin(2 * np.pi * O.phasor(np.full(T, f, np.float32), SR).astype(np.float64))
            for f, a in zip(freqs, amps.astype(np.float64)))
    ref = np.convolve(x, 0.9 ** np.arange(T))[:T]
    assert np.abs(y - ref).max() < 1e-5
    # the carried state: each oscillator's phase after T frames, and y[T-1]
    np.testing.assert_array_equal(st[:16], np.array([O.phasor(np.full(T + 1, f, np.float32), SR)[T] for f in freqs]))
    assert st[16] == y[-1]


def test_any_split_into_calls_gives_the_same_samples_when_state_carries():
    freqs, amps = bank()
    one, st1 = run_calls(freqs, amps, [6000], 1)
    for sizes in ([3000, 3000], [1, 999, 4000, 1000], [17] * 352 + [16]):
        got, st = run_calls(freqs, amps, sizes, 1)
        np.testing.assert_array_equal(got, one)
        np.testing.assert_array_equal(st, st1)


def test_deterministic_bank_phases_depend_on_the_split():
    # the deterministic phasor restarts its frame index in every call
    freqs, amps = bank()
    a, _ = run_calls(freqs, amps, [3000, 3000], 0)
    b, _ = run_calls(freqs, amps, [6000], 0)
    assert np.array_equal(a[:3000], b[:3000]) and not np.array_equal(a[3000:], b[3000:])


def test_deterministic_bank_restarts_its_phases_and_carries_the_one_pole():
    # call 2 = the zero-state bank of call 1's phases (frame index from 0)
    # plus the carried y through the one-pole: pole^(n+1) * y_prev (linearity)
    freqs, amps = bank()
    st = np.zeros(17, np.float32)
    y1 = O.oscbank_stream(freqs, amps, SR, 0.9, 2048, 0, st)
    np.testing.assert_array_equal(y1, O.oscbank(freqs, amps, SR, 0.9, 2048))
    yprev = float(st[16])
    y2 = O.oscbank_stream(freqs, amps, SR, 0.9, 2048, 0, st)
    ref = y1.astype(np.float64) + yprev * 0.9 ** np.arange(1, 2049)
    assert np.abs(y2 - ref).max() < 1e-5


def test_biquad_block_continues_like_lfilter_with_the_carried_state():
    # constant cutoff: an LTI RBJ low-pass, so block 2 from the carried
    # history equals scipy's lfilter with lfiltic initial conditions
    B, T = 3, 3000
    rng = np.random.default_rng(4)
    x = rng.uniform(-1, 1, (2 * T, B)).astype(np.float32)
    base = np.array([300.0, 1000.0, 5000.0], np.float32)
    Q = np.array([0.707, 2.0, 0.5], np.float32)
    st = np.zeros((B, 4), np.float32)
    y1 = O.biquad_stream(x[:T], None, base, Q, st)
    y2 = O.biquad_stream(x[T:], None, base, Q, st)
    np.testing.assert_array_equal(np.concatenate([y1, y2]), O.biquad_fwd(x, None, base, Q))
    for k in range(B):
        w0 = abs(float(base[k])) * 2 * np.pi / 44100.0
        alpha = np.sin(w0) / (2 * abs(float(Q[k])))
        b = np.array([(1 - np.cos(w0)) / 2, 1 - np.cos(w0), (1 - np.cos(w0)) / 2]) / (1 + alpha)
        a = np.array([1.0, -2 * np.cos(w0) / (1 + alpha), (1 - alpha) / (1 + alpha)])
        zi = ss.lfiltic(b, a, y1[::-1, k].astype(np.float64), x[:T][::-1, k].astype(np.float64))
        ref, _ = ss.lfilter(b, a, x[T:, k].astype(np.float64), zi=zi)
        assert np.abs(y2[:, k] - ref).max() < 1e-5


def test_biquad_any_split_is_the_same_and_outputs_are_contained():
    B, T = 5, 2000
    rng = np.random.default_rng(5)
    x = rng.uniform(-1, 1, (T, B)).astype(np.float32)
    m = np.exp2(rng.uniform(0, 4, T)).astype(np.float32)
    base = np.full(B, 200.0, np.float32)
    Q = np.full(B, 0.707, np.float32)
    ref = O.biquad_fwd(x, m, base, Q)
    st = np.zeros((B, 4), np.float32)
    parts, n0 = [], 0
    for n in (1, 700, 13, 1286):
        parts.append(O.biquad_stream(x[n0:n0 + n], m[n0:n0 + n], base, Q, st))
        n0 += n
    np.testing.assert_array_equal(np.concatenate(parts), ref)
    # a non-finite input: the out stores read 0 where y is non-finite
    xb = x.copy()
    xb[100, 2] = np.inf
    yb = O.biquad_stream(xb, m, base, Q, np.zeros((B, 4), np.float32))
    assert np.all(np.isfinite(yb)) and np.all(yb[100:, 2] == 0.0) and np.array_equal(yb[:, 0], ref[:, 0])
