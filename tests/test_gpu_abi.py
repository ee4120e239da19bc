"""The run contract of the C ABI on the GPU: which frame counts a schedule
runs (LazyRuntime.runNoCopy(frameCount:), Realize.swift:12-19), the declared
output cells (outputsPointer), the host sample rate of a run
(DGenProcessContextV1.sample_rate, dgen_runtime.h:252-291) and non-finite
output containment (CRenderer.swift:1021-1039).  Needs a GPU."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import HarmonicConfig, HIPError, OscBankConfig
from dgen_hip.programs import check_row_schedule, harmonic_program, oscbank_program
from dgen_hip.runtime import HIPLazyRuntime

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def osc(gpu):
    cfg = OscBankConfig()
    freqs, amps = cfg.inputs()
    rt = HIPLazyRuntime(oscbank_program(cfg), 0)
    rt.write("freqs", freqs)
    rt.write("amps", amps)
    yield cfg, freqs, amps, rt
    rt.close()


def test_exact_frame_count_classes_reject_other_counts(gpu):
    cfg = HarmonicConfig(B=1, T=1024, hidden=16, fft_sizes=(64,))
    with HIPLazyRuntime(harmonic_program(cfg, train=False), 0) as rt:
        for n in (cfg.T - 1, cfg.T // 2):
            with pytest.raises(HIPError, match="must equal"):
                rt.runNoCopy(n)
        with pytest.raises(HIPError, match="max_frames"):
            rt.runNoCopy(0)
        rt.runNoCopy(cfg.T)


def test_oscillator_bank_runs_a_prefix_of_its_frames(osc):
    cfg, freqs, amps, rt = osc
    rt.runNoCopy()
    full = rt.read("out")
    for n in (1, 1000, 4096, cfg.frames - 3):
        rt.write("out", np.zeros(cfg.frames, np.float32))
        rt.runNoCopy(n)
        got = rt.read("out")
        np.testing.assert_array_equal(got[:n], full[:n])
        assert not got[n:].any()
    with pytest.raises(HIPError, match="max_frames"):
        rt.runNoCopy(cfg.frames + 1)


def test_outputs_are_host_visible_after_a_run(osc):
    cfg, freqs, amps, rt = osc
    rt.runNoCopy()
    ref = rt.read("out")
    view = rt.outputsPointer()
    assert view.shape == (cfg.frames,)
    view[:] = -7.0  # host mirror only; the next run copies the device cells back
    rt.runNoCopy()
    np.testing.assert_array_equal(rt.outputsPointer(), ref)


def test_outputs_can_be_undeclared_and_declared_again(osc):
    # (the bench's timed region declares none, so its closing sync copies
    # nothing; the sync after a run_async copies the declared cells)
    cfg, freqs, amps, rt = osc
    rt.runNoCopy()
    ref = rt.read("out")
    try:
        rt.setOutputs(None)
        with pytest.raises(HIPError, match="no output cells"):
            rt.outputsPointer()
        rt.run_async()
        rt.sync()
    finally:
        rt.setOutputs("out")
    view = rt.outputsPointer()
    view[:] = -7.0
    rt.run_async()
    rt.sync()
    np.testing.assert_array_equal(rt.outputsPointer(), ref)


def test_host_sample_rate_drives_the_oscillator_phases(osc):
    cfg, freqs, amps, rt = osc
    rt.runNoCopy()
    base = rt.read("out")
    try:
        rt.setSampleRate(22050.0)
        rt.runNoCopy()
        got = rt.read("out")
        ref = O.oscbank(freqs, amps, 22050.0, cfg.pole, cfg.frames)
        err = np.abs(got - ref).max()
        print(f"osc bank at a 22.05 kHz host rate: max|y - oracle| = {err:.3e}")
        assert err < 1e-4
        assert np.abs(got - base).max() > 0.1
        with pytest.raises(HIPError, match="outside"):
            rt.setSampleRate(-1.0)
    finally:
        rt.setSampleRate(0.0)
    rt.runNoCopy()
    np.testing.assert_array_equal(rt.read("out"), base)


def _render(cfg, X, f0, uv, params, host_sr=0.0, graphs=False):
    with HIPLazyRuntime(harmonic_program(cfg, train=False), 0) as rt:
        check_row_schedule(rt)
        rt.write("X", X)
        rt.write("f0", f0)
        rt.write("uv", uv)
        rt.write("params", params)
        if graphs:
            rt.set_graphs(True)
            rt.runNoCopy()  # captured at the rendered rate
        rt.setSampleRate(host_sr)
        rt.runNoCopy()
        return {k: rt.read(k) for k in ("y", "ctrl", "f0_frames", "checkpoints")}


def test_host_sample_rate_drives_the_harmonic_phases_not_the_nyquist_mask(gpu):
    cfg = HarmonicConfig(B=2, T=4096, hidden=32, fft_sizes=(64,))
    f0, uv, X = cfg.data()
    for graphs in (False, True):
        out = _render(cfg, X, f0, uv, cfg.weights(), host_sr=22050.0, graphs=graphs)
        f0f = out["f0_frames"].reshape(cfg.B, cfg.T)
        ck = O.phase_checkpoints(f0f, cfg.B, cfg.K, cfg.T, 22050.0)
        np.testing.assert_array_equal(out["checkpoints"].reshape(ck.shape), ck)
        ctrl = out["ctrl"].reshape(cfg.M, cfg.ldc)[:, :cfg.NC]
        ref = O.synth_fwd_rates(ctrl, f0, uv, cfg.B, cfg.F, cfg.T, cfg.K, cfg.NF, 22050.0, cfg.sr)
        err = np.abs(out["y"].reshape(cfg.B, cfg.T) - ref).max()
        print(f"harmonic render at a 22.05 kHz host rate (graphs {graphs}): max|y - oracle| = {err:.3e}")
        assert err < 1e-5


def test_non_finite_controls_zero_exactly_the_frames_that_read_them(gpu):
    # a NaN feature row (b = 1, control frame f) makes that control row NaN;
    # every frame whose sampleRow lerp reads row f is stored as 0, all others
    # are unchanged, and lane 0 is untouched
    cfg = HarmonicConfig(B=2, T=4096, hidden=32, fft_sizes=(64,))
    f0, uv, X = cfg.data()
    P = cfg.weights()
    clean = _render(cfg, X, f0, uv, P)["y"].reshape(cfg.B, cfg.T)
    row = 17
    Xb = X.copy().reshape(cfg.B, cfg.F, cfg.din)
    Xb[1, row, :] = np.nan
    Xb = Xb.reshape(X.shape)
    y = _render(cfg, Xb, f0, uv, P)["y"].reshape(cfg.B, cfg.T)
    play = O.playhead(cfg.F, cfg.T)
    lo = np.floor(play).astype(int)
    hi = np.where(lo + 1 >= cfg.F, 0, lo + 1)
    hit = (lo == row) | (hi == row)
    assert hit.sum() > 64
    assert np.all(y[1][hit] == 0.0)
    np.testing.assert_array_equal(y[1][~hit], clean[1][~hit])
    np.testing.assert_array_equal(y[0], clean[0])
    ctrl = O.mlp_fwd(Xb, P, cfg.M, cfg.din, cfg.hidden, cfg.layers, cfg.K, cfg.NF)
    ref = O.synth_fwd(ctrl, f0, uv, cfg.B, cfg.F, cfg.T, cfg.K, cfg.NF, cfg.sr)
    assert np.all(ref[1][hit] == 0.0)
    assert np.abs(y - ref).max() < 1e-4
    # an infinite harmonic-gain bias makes every frame non-finite: all zero
    P2 = P.copy()
    off = cfg.param_count() - cfg.NC  # bh
    P2[off + cfg.K] = np.inf
    y2 = _render(cfg, X, f0, uv, P2)["y"]
    assert np.all(y2 == 0.0)


def test_non_finite_oscillator_input_zeroes_the_output(osc):
    cfg, freqs, amps, rt = osc
    try:
        bad = amps.copy()
        bad[3] = np.nan
        rt.write("amps", bad)
        rt.runNoCopy()
        assert np.all(rt.read("out") == 0.0)
        assert np.all(O.oscbank(freqs, bad, cfg.sr, cfg.pole, 4096) == 0.0)
        badf = freqs.copy()
        badf[2] = np.inf
        rt.write("amps", amps)
        rt.write("freqs", badf)
        rt.runNoCopy()
        assert np.all(rt.read("out") == 0.0)
    finally:
        rt.write("amps", amps)
        rt.write("freqs", freqs)
