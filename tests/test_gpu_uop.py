"""Generic UOp blocks on the GPU (dgen_hip_set_blocks + DGEN_HIP_K_UOP_BLOCK):
schedules built from the compiler's block vocabulary, rendered to HIP C++ and
compiled with hiprtc, against the CPU oracle and numpy:
- config 1 as two generic blocks (phasor bank -> sum -> history one-pole)
  within 1e-4 of the oracle and of the config-1 kernel class, and with a
  tanh waveshaper (one elementwise block more) against tanh of the oracle;
- a hop counter and a hop-gated block (Temporality .hopBased);
- Signal.noise()'s xorshift32 stream, bit for bit;
- the arithmetic / comparison / logic / selection / math UOps against numpy;
- a static block run at configure, read through a static global;
- the harmonic synth's kernel-class schedule with one generic block
  appended;
- runs of fewer frames than the cells hold, and graph replay.
Needs a GPU."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import HarmonicConfig, OscBankConfig
from dgen_hip.programs import harmonic_program, oscbank_program
from dgen_hip.runtime import HIPLazyRuntime
from dgen_hip.uop_programs import (append_lane_shaper, expr_reference, expr_uop_program, frame_count_uop_block,
                                   hop_uop_program, noise_uop_program, oscbank_uop_program, table_uop_program)

pytestmark = pytest.mark.gpu


def run_oscbank(cfg, drive=None, frames=None):
    prog = oscbank_uop_program(cfg, drive=drive)
    freqs, amps = cfg.inputs()
    with HIPLazyRuntime(prog, 0) as rt:
        rt.write("freqs", freqs)
        rt.write("amps", amps)
        rt.runNoCopy(frames)
        return rt.read("out")[:frames or cfg.frames]


def test_config1_as_generic_blocks_matches_the_oracle_and_the_kernel_class(gpu):
    cfg = OscBankConfig()
    print(f"generic-block oscillator bank: {cfg.n_osc} oscillators x {cfg.frames} frames", flush=True)
    y = run_oscbank(cfg)
    freqs, amps = cfg.inputs()
    ref = O.oscbank(freqs, amps, cfg.sr, cfg.pole, cfg.frames)
    with HIPLazyRuntime(oscbank_program(cfg), 0) as rt:
        rt.write("freqs", freqs)
        rt.write("amps", amps)
        rt.runNoCopy()
        kc = rt.read("out")
    e_o, e_k = np.abs(y - ref).max(), np.abs(y - kc).max()
    print(f"max|y - oracle| {e_o:.3e}, max|y - kernel class| {e_k:.3e}")
    assert e_o < 1e-4 and e_k < 1e-4
    # a run of fewer frames computes the same first frames
    part = run_oscbank(cfg, frames=5000)
    np.testing.assert_array_equal(part, y[:5000])


def test_one_elementwise_block_more(gpu):
    cfg = OscBankConfig()
    y = run_oscbank(cfg, drive=2.0)
    freqs, amps = cfg.inputs()
    ref = np.tanh(2.0 * O.oscbank(freqs, amps, cfg.sr, cfg.pole, cfg.frames).astype(np.float64))
    err = np.abs(y - ref).max()
    print(f"tanh(2 y): max|y - tanh(2 oracle)| {err:.3e}")
    assert err < 1e-4


def test_hop_gated_block(gpu):
    T, hop = 10007, 256
    prog = hop_uop_program(T, hop)
    x = np.random.default_rng(5).standard_normal(T).astype(np.float32)
    with HIPLazyRuntime(prog, 0) as rt:
        rt.write("x", x)
        rt.runNoCopy()
        dec, hits, cnt = rt.read("decimated"), rt.read("hits")[0], rt.read("counter")[0]
    np.testing.assert_array_equal(dec, x[::hop])
    assert hits == len(range(0, T, hop))
    assert cnt == T % hop  # the accum's state after T increments, wrapped at the hop


def test_noise_stream_bit_exact(gpu):
    T = 70000
    with HIPLazyRuntime(noise_uop_program(T), 0) as rt:
        rt.runNoCopy()
        out = rt.read("out")
    np.testing.assert_array_equal(out, O.noise_stream(T))


def test_expression_uops_against_numpy(gpu):
    T = 4096
    prog = expr_uop_program(T)
    x = np.random.default_rng(9).uniform(-2, 2, T).astype(np.float32)
    with HIPLazyRuntime(prog, 0) as rt:
        rt.write("x", x)
        rt.runNoCopy()
        out = rt.read("out").reshape(8, T)
    ref = expr_reference(x)
    for ch in range(8):
        err = np.abs(out[ch] - ref[ch]) / (1.0 + np.abs(ref[ch]))
        print(f"channel {ch}: max rel err {err.max():.2e}")
        assert err.max() < 2e-6, ch


def test_static_block_and_static_global(gpu):
    T, N = 3000, 64
    with HIPLazyRuntime(table_uop_program(T, N), 0) as rt:
        rt.runNoCopy()
        out, tab = rt.read("out"), rt.read("table")
    ref = 0.5 * np.sin(2 * np.pi * np.arange(N) / N)
    assert np.abs(tab - ref).max() < 1e-6
    np.testing.assert_array_equal(out, tab[np.arange(T) % N])


def test_kernel_class_schedule_with_a_generic_block_appended(gpu):
    cfg = HarmonicConfig(B=4, T=8192, hidden=64, fft_sizes=(512, 256))
    prog = harmonic_program(cfg, train=False)
    prog.alloc("y_shaped", cfg.B * cfg.T)
    append_lane_shaper(prog, "y", "y_shaped", cfg.B, cfg.T, 3.0)
    f0, uv, X = cfg.data()
    with HIPLazyRuntime(prog, 0) as rt:
        rt.write("X", X)
        rt.write("f0", f0)
        rt.write("uv", uv)
        rt.write("params", cfg.weights())
        rt.runNoCopy()
        y, ys = rt.read("y"), rt.read("y_shaped")
    np.testing.assert_allclose(ys, np.tanh(3.0 * y.astype(np.float64)), rtol=0, atol=2e-7)
    ctrl = O.mlp_fwd(X, cfg.weights(), cfg.M, cfg.din, cfg.hidden, cfg.layers, cfg.K, cfg.NF)
    ref = O.synth_fwd(ctrl, f0, uv, cfg.B, cfg.F, cfg.T, cfg.K, cfg.NF, cfg.sr).reshape(-1)
    assert np.abs(ys - np.tanh(3.0 * ref.astype(np.float64))).max() < 1e-4


def test_generic_blocks_replay_as_a_graph_and_see_the_frame_count(gpu):
    cfg = OscBankConfig(frames=20000)
    prog = oscbank_uop_program(cfg)
    fc = prog.alloc("frames_seen", 1)
    frame_count_uop_block(prog, fc)
    freqs, amps = cfg.inputs()
    with HIPLazyRuntime(prog, 0) as rt:
        rt.write("freqs", freqs)
        rt.write("amps", amps)
        rt.runNoCopy(12345)
        assert rt.read("frames_seen")[0] == 12345.0
        outs = []
        for graphs in (False, True):
            rt.set_graphs(graphs)
            rt.write("history", np.zeros(1, np.float32))
            for _ in range(3):
                rt.runNoCopy()
            outs.append(rt.read("out"))
        np.testing.assert_array_equal(outs[0], outs[1])
        assert rt.read("frames_seen")[0] == cfg.frames
