"""ctypes view of the CPU oracle (``liboracle.so``).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP backend.  Only the
test suite, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module; the product library never calls it.

Each wrapper takes/returns numpy float32 arrays and selects the fp32
(emission-faithful) or fp64 (finite-difference) build with ``prec``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS: dict[str, ctypes.CDLL] = {}

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_c_int, _c_float, _c_size = ctypes.c_int, ctypes.c_float, ctypes.c_size_t
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")


def rp_(sfx):
    """Pointer type of the build's REAL arrays."""
    return _f32p if sfx == "_f32" else _f64p


def build() -> None:
    """Compile liboracle.so / liboracle_bench.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)


def lib(name: str = "liboracle.so") -> ctypes.CDLL:
    if name not in _LIBS:
        path = os.path.join(_HERE, name)
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        for sfx in ("_f32", "_f64"):
            if not hasattr(L, "dgen_oracle_oscbank" + sfx):
                continue
            _sig(L, "dgen_oracle_oscbank" + sfx, [_f32p, _f32p, _c_int, _c_float, _c_float, _c_int, _f32p])
            _sig(L, "dgen_oracle_oscbank_stream" + sfx,
                 [_f32p, _f32p, _c_int, _c_float, _c_float, _c_int, _c_int, rp_(sfx), _f32p])
            _sig(L, "dgen_oracle_playhead" + sfx, [_c_int, _c_int, _f32p])
            syn = [_f32p, _f32p, _f32p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_float, _c_float, _f32p]
            _sig(L, "dgen_oracle_synth_fwd" + sfx, syn)
            _sig(L, "dgen_oracle_synth_bwd" + sfx, syn[:3] + [_f32p] + syn[3:])
            _sig(L, "dgen_oracle_synth_fwd_rates" + sfx, syn[:9] + [_c_float] + syn[9:])
            _sig(L, "dgen_oracle_mlp_param_count" + sfx, [_c_int] * 4, _c_size)
            _sig(L, "dgen_oracle_mlp_fwd" + sfx, [_f32p, _f32p] + [_c_int] * 6 + [_f32p])
            _sig(L, "dgen_oracle_mlp_bwd" + sfx, [_f32p, _f32p, _f32p] + [_c_int] * 6 + [_f32p])
            mss = [_f32p, _f32p, _c_int, _c_int, _i32p, _c_int, _c_int, _c_float, _c_float, _c_float, _c_int,
                   _c_float]
            _sig(L, "dgen_oracle_mss_fwd" + sfx, mss + [ctypes.c_void_p], ctypes.c_double)
            _sig(L, "dgen_oracle_mss_bwd" + sfx, mss + [_f32p])
            _sig(L, "dgen_oracle_mss_fwd_real" + sfx, [rp_(sfx), _f32p] + mss[2:], ctypes.c_double)
            rp = _f32p if sfx == "_f32" else np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
            _sig(L, "dgen_oracle_harmonic_step" + sfx,
                 [_f32p, rp, _f32p, _f32p, _f32p] + [_c_int] * 8 + [_c_float] * 3 + [_i32p, _c_int, _c_int]
                 + [_c_float] * 3 + [_c_int, _c_float, ctypes.c_void_p, ctypes.c_void_p], ctypes.c_double)
            _sig(L, "dgen_oracle_adam" + sfx, [_f32p, _f32p, _f32p, _f32p, _c_size] + [_c_float] * 4 + [_c_int])
            vp = ctypes.c_void_p
            _sig(L, "dgen_oracle_biquad_fwd" + sfx, [_f32p, vp, rp, rp, _c_int, _c_int, _f32p])
            _sig(L, "dgen_oracle_biquad_stream" + sfx, [_f32p, vp, rp, rp, _c_int, _c_int, rp, _f32p])
            _sig(L, "dgen_oracle_biquad_step" + sfx, [_f32p, vp, rp, rp, _f32p, _c_int, _c_int, vp, vp],
                 ctypes.c_double)
            _sig(L, "dgen_oracle_tensor_fft" + sfx, [_c_int, _c_int, rp, rp])
            rs = ctypes.c_float if sfx == "_f32" else ctypes.c_double
            _sig(L, "dgen_oracle_membrane_step" + sfx, [_f32p, _c_int, _c_int, _c_int, rs, rs, _c_int, _c_int, _f32p,
                                                        vp, vp], ctypes.c_double)
            _sig(L, "dgen_oracle_stft_step" + sfx, [_f32p, _c_int, _c_int, _c_int, _c_int, _f32p, rp, vp, vp],
                 ctypes.c_double)
            _sig(L, "dgen_oracle_swept_phasor_step" + sfx,
                 [rp_(sfx), _c_int, _c_int, _c_float, _c_float, _c_float, _c_int, _c_int, ctypes.c_void_p,
                  ctypes.c_void_p],
                 ctypes.c_double)
            _sig(L, "dgen_oracle_svf_fwd" + sfx, [_f32p, vp, vp, rp, rp, vp, _c_int, _c_int, _c_float, vp, _f32p])
            _sig(L, "dgen_oracle_svf_step" + sfx,
                 [_f32p, vp, vp, rp, rp, vp, _f32p, _c_int, _c_int, _c_float, vp, vp, vp], ctypes.c_double)
        if hasattr(L, "dgen_oracle_temporal_scan"):
            _sig(L, "dgen_oracle_temporal_scan", [_f32p, ctypes.c_void_p, _c_int, _c_int, _f32p])
        if hasattr(L, "dgen_oracle_noise_stream"):
            _sig(L, "dgen_oracle_noise_stream", [_c_int, _f32p])
            _sig(L, "dgen_oracle_phasor", [_f32p, _c_int, _c_float, _f32p])
            _sig(L, "dgen_oracle_lerp_frames", [_f32p, _c_int, _c_int, _c_int, _f32p])
            _sig(L, "dgen_oracle_phase_checkpoints", [_f32p, _c_int, _c_int, _c_int, _c_float, _c_int, _f32p])
        _LIBS[name] = L
    return _LIBS[name]


def _sig(L, name, args, res=None):
    fn = getattr(L, name)
    fn.argtypes = args
    fn.restype = res


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fn(name: str, prec: str, libname: str = "liboracle.so"):
    return getattr(lib(libname), f"{name}_{prec}")


# -- config 1 -------------------------------------------------------------
def oscbank(freqs, amps, sr, pole, frames, prec="f32", libname="liboracle.so"):
    out = np.zeros(frames, np.float32)
    _fn("dgen_oracle_oscbank", prec, libname)(_f(freqs), _f(amps), len(freqs), sr, pole, frames, out)
    return out


def oscbank_stream(freqs, amps, sr, pole, frames, stateful, state, prec="f32"):
    """One streaming block of the bank; `state` ([n_osc] phases + y[n-1],
    float32 for prec f32, float64 for f64) is updated in place."""
    out = np.zeros(frames, np.float32)
    _fn("dgen_oracle_oscbank_stream", prec)(_f(freqs), _f(amps), len(freqs), sr, pole, frames, int(stateful), state,
                                            out)
    return out


# -- temporal gradient of stateful accumulators -----------------------------
def temporal_scan(g, reset=None):
    """Reset-aware exclusive suffix scan of g [T][E] (reset [T] or None)."""
    g = _f(g)
    T, E = g.shape
    out = np.zeros((T, E), np.float32)
    r = None if reset is None else _f(reset)
    lib().dgen_oracle_temporal_scan(g, None if r is None else r.ctypes.data_as(ctypes.c_void_p), T, E, out)
    return out


def swept_phasor_step(slope, T, sr, base, target, reset_from=-1, smooth=False, grad=True, want_phase=False,
                      prec="f64"):
    """Swept-phasor bank (loss on the phase, or with smooth on sin(2 pi
    phase)): returns (loss, d loss / d slope or None, phase [T][E] or None)."""
    dt = np.float32 if prec == "f32" else np.float64
    slope = np.ascontiguousarray(slope, dt)
    E = len(slope)
    g = np.zeros(E, dt) if grad else None
    ph = np.zeros((T, E), np.float32) if want_phase else None
    loss = _fn("dgen_oracle_swept_phasor_step", prec)(slope, E, T, sr, base, target, reset_from, int(smooth),
                                                      g.ctypes.data_as(ctypes.c_void_p) if grad else None,
                                                      ph.ctypes.data_as(ctypes.c_void_p) if want_phase else None)
    return loss, g, ph


# -- config 3 -------------------------------------------------------------
def playhead(F, T, prec="f32"):
    out = np.zeros(T, np.float32)
    _fn("dgen_oracle_playhead", prec)(F, T, out)
    return out


def noise_stream(T):
    out = np.zeros(T, np.float32)
    lib().dgen_oracle_noise_stream(T, out)
    return out


def phasor(freq, sr):
    """Stateful phasor outputs (pre-increment) for a per-frame frequency."""
    freq = _f(freq)
    out = np.zeros(len(freq), np.float32)
    lib().dgen_oracle_phasor(freq, len(freq), sr, out)
    return out


def lerp_frames(src, B, F, T):
    """[B][T] frame-rate interpolation of a [F][B] data table along the playhead."""
    out = np.zeros((B, T), np.float32)
    lib().dgen_oracle_lerp_frames(_f(src), B, F, T, out)
    return out


def phase_checkpoints(f0f, B, K, T, sr, seg=64):
    """[nseg][B][K] harmonic phases at every segment start."""
    nseg = (T + seg - 1) // seg
    out = np.zeros((nseg, B, K), np.float32)
    lib().dgen_oracle_phase_checkpoints(_f(f0f), B, K, T, sr, seg, out)
    return out


def synth_fwd(ctrl, f0, uv, B, F, T, K, NF, sr, hscale=1.0, nscale=1.0, prec="f32", libname="liboracle.so"):
    y = np.zeros((B, T), np.float32)
    _fn("dgen_oracle_synth_fwd", prec, libname)(_f(ctrl), _f(f0), _f(uv), B, F, T, K, NF, sr, hscale, nscale, y)
    return y


def synth_fwd_rates(ctrl, f0, uv, B, F, T, K, NF, host_sr, graph_sr, hscale=1.0, nscale=1.0, prec="f32"):
    """Synth forward with phase increments over host_sr and the Nyquist mask at graph_sr / 2."""
    y = np.zeros((B, T), np.float32)
    _fn("dgen_oracle_synth_fwd_rates", prec)(_f(ctrl), _f(f0), _f(uv), B, F, T, K, NF, host_sr, graph_sr, hscale,
                                              nscale, y)
    return y


def synth_bwd(ctrl, f0, uv, dy, B, F, T, K, NF, sr, hscale=1.0, nscale=1.0, prec="f32"):
    NC = K + 2 + NF
    d = np.zeros((B * F, NC), np.float32)
    _fn("dgen_oracle_synth_bwd", prec)(_f(ctrl), _f(f0), _f(uv), _f(dy), B, F, T, K, NF, sr, hscale, nscale, d)
    return d


def mlp_param_count(din, hid, layers, nc):
    return int(lib().dgen_oracle_mlp_param_count_f32(din, hid, layers, nc))


def mlp_fwd(X, P, M, din, hid, layers, K, NF, prec="f32", libname="liboracle.so"):
    ctrl = np.zeros((M, K + 2 + NF), np.float32)
    _fn("dgen_oracle_mlp_fwd", prec, libname)(_f(X), _f(P), M, din, hid, layers, K, NF, ctrl)
    return ctrl


def mlp_bwd(X, P, dctrl, M, din, hid, layers, K, NF, prec="f32"):
    dP = np.zeros(len(P), np.float32)
    _fn("dgen_oracle_mlp_bwd", prec)(_f(X), _f(P), _f(dctrl), M, din, hid, layers, K, NF, dP)
    return dP


# loss-mode bits of the multi-scale loss (dgen_oracle.c MSS_*): the
# magnitude and log-magnitude terms' lossMode .l2 (else .l1),
# useSmoothLogMagnitude, useHannWindow: false
MSS_L2_LIN, MSS_L2_LOG, MSS_SMOOTH_LOG, MSS_RECT_WINDOW = 1, 2, 4, 8


def mss_fwd(x, tgt, B, T, sizes, hop_div, w_lin, w_log, max_frames, prec="f32", frames=False,
            libname="liboracle.so", mode=0, w_mse=0.0):
    sizes = np.ascontiguousarray(sizes, np.int32)
    lf = np.zeros(T, np.float32) if frames else None
    ptr = lf.ctypes.data_as(ctypes.c_void_p) if frames else None
    tot = _fn("dgen_oracle_mss_fwd", prec, libname)(_f(x), _f(tgt), B, T, sizes, len(sizes), hop_div, w_lin,
                                                    w_log, max_frames, int(mode), float(w_mse), ptr)
    return (tot, lf) if frames else tot


def mss_fwd_x64(x, tgt, B, T, sizes, hop_div, w_lin, w_log, max_frames, mode=0, w_mse=0.0):
    """fp64 spectral loss with a float64 prediction (finite differences)."""
    sizes = np.ascontiguousarray(sizes, np.int32)
    return lib().dgen_oracle_mss_fwd_real_f64(np.ascontiguousarray(x, np.float64), _f(tgt), B, T, sizes, len(sizes),
                                              hop_div, w_lin, w_log, max_frames, int(mode), float(w_mse))


def mss_bwd(x, tgt, B, T, sizes, hop_div, w_lin, w_log, max_frames, prec="f32", mode=0, w_mse=0.0):
    sizes = np.ascontiguousarray(sizes, np.int32)
    dx = np.zeros((B, T), np.float32)
    _fn("dgen_oracle_mss_bwd", prec)(_f(x), _f(tgt), B, T, sizes, len(sizes), hop_div, w_lin, w_log,
                                     max_frames, int(mode), float(w_mse), dx)
    return dx


def adam(p, g, m, v, lr, b1, b2, eps, step, prec="f32"):
    p, m, v = _f(p).copy(), _f(m).copy(), _f(v).copy()
    _fn("dgen_oracle_adam", prec)(p, _f(g), m, v, len(p), lr, b1, b2, eps, step)
    return p, m, v


def harmonic_step(cfg, X, P, f0, uv, tgt, grad=True, want_y=False, prec="f64", libname="liboracle.so"):
    """Whole config-3 step (MLP -> synth -> MSS loss [-> backward]) in one
    oracle call.  For prec="f64" the parameters are float64, so finite
    differences can use steps far below fp32 resolution.
    Returns (loss, dP or None, y or None)."""
    dt = np.float32 if prec == "f32" else np.float64
    P = np.ascontiguousarray(P, dtype=dt)
    dP = np.zeros(len(P), dt) if grad else None
    y = np.zeros((cfg.B, cfg.T), np.float32) if want_y else None
    sizes = np.ascontiguousarray(cfg.fft_sizes, np.int32)
    fn = _fn("dgen_oracle_harmonic_step", prec, libname)
    loss = fn(_f(X), P, _f(f0), _f(uv), _f(tgt), cfg.B, cfg.F, cfg.T, cfg.K, cfg.NF, cfg.din, cfg.hidden,
              cfg.layers, cfg.sr, cfg.hscale, cfg.nscale, sizes, len(sizes), cfg.hop_div, cfg.w_lin, cfg.w_log,
              float(cfg.T), int(getattr(cfg, "mss_mode", 0)), float(getattr(cfg, "w_mse", 0.0)),
              dP.ctypes.data_as(ctypes.c_void_p) if grad else None,
              y.ctypes.data_as(ctypes.c_void_p) if want_y else None)
    return loss, dP, y


# -- config 4 -------------------------------------------------------------
def _mod_ptr(m, T):
    if m is None:
        return None, None
    m = _f(m)
    if m.shape != (T,):
        raise ValueError(f"modulation must have shape ({T},)")
    return m, m.ctypes.data_as(ctypes.c_void_p)


def biquad_fwd(x, m, base, Q, prec="f32"):
    """Biquad bank forward: x [T][B] -> y [T][B]; cutoff[n][k] = base[k]*m[n]
    (m None: unmodulated)."""
    x = _f(x)
    T, B = x.shape
    dt = np.float32 if prec == "f32" else np.float64
    m, mp = _mod_ptr(m, T)
    y = np.zeros((T, B), np.float32)
    _fn("dgen_oracle_biquad_fwd", prec)(x, mp, np.ascontiguousarray(base, dt), np.ascontiguousarray(Q, dt), B, T, y)
    return y


def biquad_stream(x, m, base, Q, state, prec="f32"):
    """One streaming block of the bank: x [T][B] -> y [T][B], the history
    state [B][4] (x[n-1], x[n-2], y[n-1], y[n-2]) updated in place."""
    x = _f(x)
    T, B = x.shape
    dt = np.float32 if prec == "f32" else np.float64
    m, mp = _mod_ptr(m, T)
    y = np.zeros((T, B), np.float32)
    _fn("dgen_oracle_biquad_stream", prec)(x, mp, np.ascontiguousarray(base, dt), np.ascontiguousarray(Q, dt), B, T,
                                           state, y)
    return y


def biquad_step(x, m, base, Q, tgt, grad=True, want_y=False, prec="f64"):
    """Config-4 step: forward, loss sum (y - tgt)^2, and (grad) the BPTT
    gradient [2][B] = (d/d base, d/d Q) in the build's precision.
    Returns (loss, grad or None, y or None)."""
    x = _f(x)
    T, B = x.shape
    dt = np.float32 if prec == "f32" else np.float64
    m, mp = _mod_ptr(m, T)
    g = np.zeros(2 * B, dt) if grad else None
    y = np.zeros((T, B), np.float32) if want_y else None
    loss = _fn("dgen_oracle_biquad_step", prec)(
        x, mp, np.ascontiguousarray(base, dt), np.ascontiguousarray(Q, dt), _f(tgt).reshape(T, B), B, T,
        y.ctypes.data_as(ctypes.c_void_p) if want_y else None, g.ctypes.data_as(ctypes.c_void_p) if grad else None)
    return loss, g, y


def _vp(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def svf_fwd(x, base, res, ks=None, m=None, env=None, sr=44100.0, state=None, prec="f32"):
    """The ZDF SVF low-pass bank: x [T][B] -> y [T][B] (float32).  base, res,
    ks [B] (ks None: kSat is the constant 0); m, env [T] or None (cutoff =
    clip(base * m + env, 20, 20000)); state [2][B] (ic1 | ic2, the build's
    precision) is carried in place when given."""
    x = _f(x)
    T, B = x.shape
    dt = np.float32 if prec == "f32" else np.float64
    ksa = None if ks is None else np.ascontiguousarray(ks, dt)
    ma = None if m is None else _f(m)
    ea = None if env is None else _f(env)
    if state is not None:
        assert state.dtype == dt and state.shape == (2, B) and state.flags.c_contiguous
    y = np.zeros((T, B), np.float32)
    _fn("dgen_oracle_svf_fwd", prec)(x, _vp(ma), _vp(ea), np.ascontiguousarray(base, dt),
                                     np.ascontiguousarray(res, dt), _vp(ksa), B, T, sr, _vp(state), y)
    return y


def svf_step(x, base, res, tgt, ks=None, m=None, env=None, sr=44100.0, grad=True, want_y=False, want_xbar=False,
             prec="f64"):
    """SVF bank step: forward, loss sum (y - tgt)^2, and (grad) the BPTT
    gradient [3][B] = (d/d base, d/d res, d/d ks).  Returns (loss, grad or
    None, y or None, xbar or None)."""
    x = _f(x)
    T, B = x.shape
    dt = np.float32 if prec == "f32" else np.float64
    ksa = None if ks is None else np.ascontiguousarray(ks, dt)
    ma = None if m is None else _f(m)
    ea = None if env is None else _f(env)
    g = np.zeros(3 * B, dt) if grad else None
    y = np.zeros((T, B), np.float32) if want_y else None
    xb = np.zeros((T, B), dt) if want_xbar else None
    loss = _fn("dgen_oracle_svf_step", prec)(
        x, _vp(ma), _vp(ea), np.ascontiguousarray(base, dt), np.ascontiguousarray(res, dt), _vp(ksa),
        _f(tgt).reshape(T, B), B, T, sr, _vp(y), _vp(g), _vp(xb))
    return loss, g, y, xb


# -- config 2 -------------------------------------------------------------
def tensor_fft(re, im=None, inverse=False, prec="f64"):
    """tensorFFT (inverse=False) or tensorIFFT without taking the real part
    (inverse=True, includes the 1/N scale).  Returns (re, im)."""
    dt = np.float32 if prec == "f32" else np.float64
    re = np.array(re, dtype=dt)
    im = np.zeros_like(re) if im is None else np.array(im, dtype=dt)
    _fn("dgen_oracle_tensor_fft", prec)(len(re), int(inverse), re, im)
    return re, im


def stft_step(x, N, H, win, g, grad=True, want_y=False, prec="f64"):
    """Config-2 step over x [S][T]: window -> FFT -> gains -> IFFT ->
    overlap-add; loss sum (y - x)^2 / T.  Returns (loss, dg or None, y or None)."""
    x = _f(x)
    S, T = x.shape
    dt = np.float32 if prec == "f32" else np.float64
    g = np.ascontiguousarray(g, dtype=dt)
    if g.shape != (N // 2 + 1,):
        raise ValueError(f"gains must have shape ({N // 2 + 1},)")
    dg = np.zeros(N // 2 + 1, dt) if grad else None
    y = np.zeros((S, T), np.float32) if want_y else None
    loss = _fn("dgen_oracle_stft_step", prec)(x, S, T, N, H, _f(win), g,
                                               y.ctypes.data_as(ctypes.c_void_p) if want_y else None,
                                               dg.ctypes.data_as(ctypes.c_void_p) if grad else None)
    return loss, dg, y


# -- config 5 -------------------------------------------------------------
def membrane_step(u0, T, c2, d, pickup, tgt, grad=True, want_out=False, prec="f64"):
    """Config-5 step on the grid u0 [R][C]: T steps of the damped wave
    equation, pickup out[n] = u_{n+1}[p], loss sum (out - tgt)^2.
    Returns (loss, grad [2] = (d/dc2, d/dd) or None, out [T] or None)."""
    u0 = _f(u0)
    R, C = u0.shape
    dt = np.float32 if prec == "f32" else np.float64
    g = np.zeros(2, dt) if grad else None
    out = np.zeros(T, np.float32) if want_out else None
    loss = _fn("dgen_oracle_membrane_step", prec)(
        u0, R, C, T, float(c2), float(d), int(pickup[0]), int(pickup[1]), _f(tgt).reshape(-1)[:T].copy()
        if tgt is not None else np.zeros(T, np.float32),
        out.ctypes.data_as(ctypes.c_void_p) if want_out else None, g.ctypes.data_as(ctypes.c_void_p) if grad else None)
    return loss, g, out
