"""HIP training step against the committed golden step and the oracle's
finite differences; bit-exact static and frame tables; determinism; the
optimiser; error paths.  Needs a GPU."""
import os

import numpy as np
import pytest

import oracle as O
from dgen_hip import HarmonicConfig, HIPError
from dgen_hip.programs import HarmonicSession, harmonic_program
from dgen_hip.runtime import HIPLazyRuntime

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "harmonic_small.npz")


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.fixture(scope="module")
def golden(gpu):
    g = np.load(GOLDEN, allow_pickle=False)
    c = g["config"]
    cfg = HarmonicConfig(B=int(c[0]), T=int(c[1]), hidden=int(c[2]), fft_sizes=tuple(int(v) for v in c[3:]))
    s = HarmonicSession(cfg, optimizer=False, target=g["target"])
    s.step()
    out = {k: s.rt.read(k) for k in ("y", "loss_frames", "grads", "f0_frames", "checkpoints", "dy")}
    out["loss"] = s.loss()
    s.step()
    out["y2"] = s.rt.read("y")
    out["grads2"] = s.rt.read("grads")
    s.close()
    return cfg, g, out


def test_frame_tables_bit_exact(golden):
    cfg, g, out = golden
    np.testing.assert_array_equal(out["f0_frames"].reshape(cfg.B, cfg.T), g["f0_frames"])
    # the phase-carry chain reproduces the sequential fp32 phasor exactly
    np.testing.assert_array_equal(out["checkpoints"].reshape(g["checkpoints"].shape), g["checkpoints"])


def test_golden_forward_and_loss(golden):
    cfg, g, out = golden
    y = out["y"].reshape(cfg.B, cfg.T)
    err = np.abs(y - g["y"]).max()
    print(f"golden max|y - y_ref| = {err:.3e}")
    assert err < 1e-4
    assert abs(out["loss"] - float(g["loss"])) / float(g["loss"]) < 1e-5


def test_golden_gradient_close_to_fp64(golden):
    """fp32 HIP gradient vs the fp64 oracle gradient: within the fp32 noise
    of the fp32 oracle itself (plus a small floor)."""
    cfg, g, out = golden
    _, g32, _ = O.harmonic_step(cfg, g["X"], g["params"], g["f0"], g["uv"], g["target"], grad=True, prec="f32")
    e_gpu, e_o32 = rel(out["grads"], g["grad"]), rel(g32, g["grad"])
    print(f"grad rel L2 vs fp64 oracle: HIP {e_gpu:.3e}, fp32 oracle {e_o32:.3e}")
    assert e_gpu <= 2.0 * e_o32 + 1e-4


def test_gradient_matches_finite_differences(golden):
    """Parity bar: the HIP gradient of sum(loss) within 1e-2 relative of
    central finite differences of the fp64 oracle forward, measured
    (a) along the gradient direction, (b) on the 8 largest components one by
    one, (c) along random unit directions relative to |grad| (a random
    projection of an fp32 gradient can be arbitrarily small, so its own
    relative error is not a meaningful bar)."""
    cfg, g, out = golden
    P = g["params"].astype(np.float64)
    hip = out["grads"].astype(np.float64)

    def fd(v, eps):
        lp = O.harmonic_step(cfg, g["X"], P + eps * v, g["f0"], g["uv"], g["target"], grad=False, prec="f64")[0]
        lm = O.harmonic_step(cfg, g["X"], P - eps * v, g["f0"], g["uv"], g["target"], grad=False, prec="f64")[0]
        return (lp - lm) / (2 * eps)

    u = g["grad"] / np.linalg.norm(g["grad"])
    d = fd(u, 1e-6)
    print(f"along grad: HIP {hip @ u:.6e}, FD {d:.6e}")
    assert abs(hip @ u - d) / abs(d) < 1e-2
    for i in np.argsort(-np.abs(g["grad"]))[:8]:
        e = np.zeros_like(P)
        e[i] = 1.0
        d = fd(e, 1e-7)
        print(f"param {i}: HIP {hip[i]:.6e}, FD {d:.6e}")
        assert abs(hip[i] - d) / abs(d) < 1e-2
    rng = np.random.default_rng(21)
    gn = np.linalg.norm(hip)
    for _ in range(3):
        v = rng.standard_normal(len(P))
        v /= np.linalg.norm(v)
        d = fd(v, 1e-6)
        print(f"random direction: HIP {hip @ v:.6e}, FD {d:.6e}, |diff|/|grad| {abs(hip @ v - d) / gn:.2e}")
        assert abs(hip @ v - d) / gn < 1e-2


def test_runs_are_deterministic(golden):
    cfg, g, out = golden
    np.testing.assert_array_equal(out["y"], out["y2"])
    np.testing.assert_array_equal(out["grads"], out["grads2"])


def test_adam_step_matches_oracle(gpu):
    g = np.load(GOLDEN, allow_pickle=False)
    c = g["config"]
    cfg = HarmonicConfig(B=int(c[0]), T=int(c[1]), hidden=int(c[2]), fft_sizes=tuple(int(v) for v in c[3:]))
    s = HarmonicSession(cfg, optimizer=True, target=g["target"])
    try:
        s.step()
        grads = s.rt.read("grads")
        p1 = s.rt.read("params")
        m1, v1 = s.rt.read("adam_m"), s.rt.read("adam_v")
    finally:
        s.close()
    n = len(grads)
    ref_p, ref_m, ref_v = O.adam(g["params"], grads, np.zeros(n, np.float32), np.zeros(n, np.float32), cfg.lr, 0.9,
                                 0.999, 1e-8, 1, prec="f32")
    np.testing.assert_allclose(m1, ref_m, rtol=1e-6, atol=1e-12)
    np.testing.assert_allclose(v1, ref_v, rtol=1e-6, atol=1e-14)
    np.testing.assert_allclose(p1, ref_p, rtol=1e-6, atol=1e-7)


def test_frame_count_beyond_max_is_an_error(gpu):
    cfg = HarmonicConfig(B=1, T=1024, hidden=16, fft_sizes=(64,))
    with HIPLazyRuntime(harmonic_program(cfg, train=False), 0) as rt:
        with pytest.raises(HIPError, match="max_frames"):
            rt.runNoCopy(cfg.T + 1)


def test_operand_outside_arena_is_rejected_at_configure(gpu):
    cfg = HarmonicConfig(B=1, T=1024, hidden=16, fft_sizes=(64,))
    p = harmonic_program(cfg, train=False)
    p.size = p.cells["y"].off + 10  # arena too small for the synth output
    with pytest.raises(HIPError, match="outside arena"):
        HIPLazyRuntime(p, 0)
