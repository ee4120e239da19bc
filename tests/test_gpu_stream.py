"""The streaming process path (dgen_hip_process_v1, the reference's
dgen_process_v1 with realize(preserveState: true), Realize.swift:553-563):
any split of a signal into calls gives the same samples as one call, bit for
bit, and the samples match the oracle's streaming blocks
(dgen_oracle_oscbank_stream / dgen_oracle_biquad_stream) fed the same calls.
Configs 1 and 4.  Needs a GPU."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import BiquadConfig, OscBankConfig
from dgen_hip.programs import stream_biquad_program, stream_oscbank_program
from dgen_hip.runtime import HIPError, HIPLazyRuntime

pytestmark = pytest.mark.gpu


def osc_runtime(cfg, stateful):
    prog = stream_oscbank_program(cfg, stateful=stateful)
    rt = HIPLazyRuntime(prog, 0)
    freqs, amps = cfg.inputs()
    rt.write("freqs", freqs)
    rt.write("amps", amps)
    rt.setProcessPorts(*prog.meta["ports"])
    return rt


def osc_calls(rt, sizes, sr=0.0):
    return np.concatenate([rt.process([], n, sample_rate=sr)[0] for n in sizes])


def osc_oracle(cfg, sizes, stateful, sr=None):
    freqs, amps = cfg.inputs()
    st = np.zeros(cfg.n_osc + 1, np.float32)
    return np.concatenate([O.oscbank_stream(freqs, amps, sr or cfg.sr, cfg.pole, n, int(stateful), st)
                           for n in sizes])


SPLITS = ([16384] * 4, [1, 999, 4000, 60000, 536], [4096] * 16)


@pytest.mark.parametrize("stateful", [True, False])
def test_oscillator_bank_calls(gpu, stateful):
    cfg = OscBankConfig()
    print(f"streaming osc bank, stateful={stateful}", flush=True)
    rt = osc_runtime(cfg, stateful)
    try:
        one = osc_calls(rt, [cfg.frames])
        ref = osc_oracle(cfg, [cfg.frames], stateful)
        err = np.abs(one - ref).max()
        print(f"one call of {cfg.frames}: max|y - oracle| = {err:.3e}")
        assert err < 1e-4
        for sizes in SPLITS:
            first = rt.process([], sizes[0], reset=True)[0]  # restart from zero state, then the calls
            got = np.concatenate([first, osc_calls(rt, sizes[1:])])
            if stateful:
                np.testing.assert_array_equal(got, one)
            ref_s = osc_oracle(cfg, sizes, stateful)
            assert np.abs(got - ref_s).max() < 1e-4
    finally:
        rt.close()


def test_oscillator_bank_host_rate_and_reset(gpu):
    cfg = OscBankConfig()
    rt = osc_runtime(cfg, True)
    try:
        a = osc_calls(rt, [3000, 3000], sr=22050.0)
        ref = osc_oracle(cfg, [3000, 3000], True, sr=22050.0)
        assert np.abs(a - ref).max() < 1e-4
        again = rt.process([], 3000, sample_rate=22050.0, reset=True)[0]
        np.testing.assert_array_equal(again, a[:3000])
    finally:
        rt.close()


def test_runs_preserve_state_like_process_calls(gpu):
    # dgen_hip_run on a streaming schedule carries the state too (runNoCopy
    # with preserveState): two runs of 3000 frames = one process call of 6000
    cfg = OscBankConfig()
    rt = osc_runtime(cfg, True)
    try:
        one = rt.process([], 6000, reset=True)[0]
        rt.zeroAllBuffers()
        freqs, amps = cfg.inputs()
        rt.write("freqs", freqs)
        rt.write("amps", amps)
        parts = []
        for _ in range(2):
            rt.runNoCopy(3000)
            parts.append(rt.read("out")[:3000])
        np.testing.assert_array_equal(np.concatenate(parts), one)
        with pytest.raises(HIPError, match="max_frames"):
            rt.process([], cfg.frames + 1)
    finally:
        rt.close()


def bq_runtime(cfg):
    prog = stream_biquad_program(cfg)
    rt = HIPLazyRuntime(prog, 0)
    rt.write("params", cfg.params())
    rt.setProcessPorts(*prog.meta["ports"])
    return rt


def bq_calls(rt, x, mod, sizes, reset=True):
    out, n0 = [], 0
    for i, n in enumerate(sizes):
        ins = [x[n0:n0 + n, k] for k in range(x.shape[1])] + [mod[n0:n0 + n]]
        out.append(rt.process(ins, n, reset=reset and i == 0).T)
        n0 += n
    return np.concatenate(out)


def test_biquad_bank_calls(gpu):
    cfg = BiquadConfig(B=256, T=1 << 15)
    x, mod = cfg.inputs(), cfg.modulation()
    print(f"streaming biquad bank B={cfg.B} T={cfg.T}", flush=True)
    rt = bq_runtime(cfg)
    try:
        one = bq_calls(rt, x, mod, [cfg.T])
        for sizes in ([8192] * 4, [1, 4095, 20000, 8672]):
            np.testing.assert_array_equal(bq_calls(rt, x, mod, sizes), one)
    finally:
        rt.close()
    p = cfg.params()
    st = np.zeros((cfg.B, 4), np.float32)
    ref = O.biquad_stream(x, mod, p[:cfg.B], p[cfg.B:], st)
    ref64 = O.biquad_fwd(x, mod, p[:cfg.B].astype(np.float64), p[cfg.B:].astype(np.float64), prec="f64")
    e_hip = np.abs(one - ref64).max()
    e_o32 = np.abs(ref - ref64).max()
    print(f"max|y - fp64 oracle|: HIP {e_hip:.3e}, fp32 oracle {e_o32:.3e}; HIP vs fp32 oracle "
          f"{np.abs(one - ref).max():.3e}")
    assert np.abs(one - ref).max() < 1e-4
    assert e_hip <= 2.0 * e_o32 + 1e-7
