"""HIP 2D membrane (config 5: time-blocked stencil forward and discrete
adjoint) against the CPU oracle: the pickup series within the
1e-4 max-abs of the fp32 oracle (held here to 1e-3 of the series' peak),
gradients against the fp64 oracle and central finite differences, at small
ragged grids and launch splits and at the full 512^2 x 4800 configuration.
Needs a GPU."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import MembraneConfig
from dgen_hip.programs import MembraneSession, membrane_program
from dgen_hip.runtime import HIPLazyRuntime

pytestmark = pytest.mark.gpu


def render(cfg, u0, params, steps):
    with HIPLazyRuntime(membrane_program(cfg, train=False, steps=steps), 0) as rt:
        rt.write("u0", u0)
        rt.write("params", params)
        rt.runNoCopy()
        out = rt.read("pickup")
        last = rt.read("states").reshape(cfg.T + 2, cfg.R, cfg.C)[-1]
        return out, last


@pytest.mark.parametrize("R,C,T,steps", [(64, 64, 300, 16), (70, 45, 257, 16), (32, 32, 16, 16), (100, 64, 1, 16),
                                         (48, 80, 100, 5), (33, 31, 40, 1)])
def test_forward_matches_oracle(gpu, R, C, T, steps):
    cfg = MembraneConfig(R=R, C=C, T=T)
    u0 = cfg.bump()
    print(f"case R={R} C={C} T={T} steps={steps}", flush=True)
    out, _ = render(cfg, u0, cfg.params(), steps)
    _, _, o32 = O.membrane_step(u0, T, np.float32(cfg.c2), np.float32(cfg.d), cfg.pickup, None, grad=False,
                                want_out=True, prec="f32")
    err = np.abs(out - o32).max()
    print(f"max|out - out_oracle| = {err:.3e} (peak {np.abs(o32).max():.3e})")
    assert err < 1e-4
    assert err <= 1e-3 * np.abs(o32).max() + 1e-7


def test_eigenmode_keeps_its_shape(gpu):
    """Size-independent property on the full 512^2 grid: a Dirichlet
    eigenmode evolves by the scalar recurrence of its eigenvalue, so the
    final state is the initial mode times that scalar."""
    cfg = MembraneConfig(T=400)
    y = np.arange(cfg.R)[:, None] + 1.0
    x = np.arange(cfg.C)[None, :] + 1.0
    a, b = 5, 3
    phi = (np.sin(np.pi * a * y / (cfg.R + 1)) * np.sin(np.pi * b * x / (cfg.C + 1))).astype(np.float32)
    mu = -4 * np.sin(np.pi * a / (2 * (cfg.R + 1))) ** 2 - 4 * np.sin(np.pi * b / (2 * (cfg.C + 1))) ** 2
    c2, d = 0.2, 0.001
    _, last = render(cfg, phi, np.array([c2, d], np.float32), 16)
    M = np.array([[2 - d + c2 * mu, -(1 - d)], [1.0, 0.0]])
    s = np.array([1.0, 1.0])
    for _ in range(cfg.T):
        s = M @ s
    err = np.abs(last - s[0] * phi.astype(np.float64)).max()
    print(f"eigenmode max err {err:.3e} (scale {abs(s[0]):.3e})")
    assert err < 1e-4


def small_session(R=48, C=40, T=200, steps=16, optimizer=False):
    cfg = MembraneConfig(R=R, C=C, T=T)
    return cfg, MembraneSession(cfg, optimizer=optimizer, steps=steps)


@pytest.mark.parametrize("steps", [16, 7])
def test_loss_and_gradient_match_oracle(gpu, steps):
    cfg, s = small_session(steps=steps)
    try:
        s.step()
        loss, g = s.loss(), s.rt.read("grads")
        s.step()
        g2 = s.rt.read("grads")
    finally:
        s.close()
    p = cfg.params().astype(np.float64)
    l64, g64, _ = O.membrane_step(s.u0, cfg.T, p[0], p[1], cfg.pickup, s.target, prec="f64")
    _, g32, _ = O.membrane_step(s.u0, cfg.T, p[0], p[1], cfg.pickup, s.target, prec="f32")
    print(f"loss HIP {loss:.8e} fp64 {l64:.8e}; grad HIP {g} fp64 {g64} fp32 oracle {g32}")
    assert abs(loss - l64) / l64 < 1e-4
    e_hip = np.abs(g - g64) / np.abs(g64)
    e_o32 = np.abs(g32 - g64) / np.abs(g64)
    assert e_hip.max() <= max(4 * e_o32.max(), 1e-4)
    np.testing.assert_array_equal(g, g2)  # deterministic


def test_gradient_matches_finite_differences(gpu):
    """Parity bar: within 1e-2 of central differences of the fp64
    oracle forward."""
    cfg, s = small_session(R=40, C=36, T=150)
    try:
        s.step()
        g = s.rt.read("grads").astype(np.float64)
    finally:
        s.close()
    p = cfg.params().astype(np.float64)
    for j in range(2):
        eps = 1e-6 * abs(p[j])
        pp, pm = p.copy(), p.copy()
        pp[j] += eps
        pm[j] -= eps
        fd = (O.membrane_step(s.u0, cfg.T, *pp, cfg.pickup, s.target, grad=False)[0]
              - O.membrane_step(s.u0, cfg.T, *pm, cfg.pickup, s.target, grad=False)[0]) / (2 * eps)
        print(f"param {j}: HIP {g[j]:.6e} FD {fd:.6e}")
        assert abs(g[j] - fd) <= 1e-2 * abs(fd)


def test_adam_step_matches_oracle(gpu):
    cfg, s = small_session(optimizer=True)
    try:
        s.step()
        g = s.rt.read("grads")
        p1 = s.rt.read("params")
    finally:
        s.close()
    ref_p, _, _ = O.adam(cfg.params(), g, np.zeros(2, np.float32), np.zeros(2, np.float32), cfg.lr, 0.9, 0.999,
                         1e-8, 1, prec="f32")
    np.testing.assert_allclose(p1, ref_p, rtol=1e-6, atol=1e-9)


def test_full_configuration_matches_oracle(gpu):
    """512 x 512 grid, 4800 frames (benchmark config 5): target and pickup
    series within 1e-4 of the fp32 oracle, loss and both gradients against
    the fp64 oracle within the 1e-2 parity bar.  dL/dc2 (-2.51) is a small
    residue of much larger oscillating terms; the sequential fp32 oracle's
    own gradient is 3.1% (c2) and 0.9% (d) from fp64 here, this kernel's
    about 0.6% and 0.004%."""
    cfg = MembraneConfig()
    s = MembraneSession(cfg, optimizer=False)
    try:
        s.step()
        out = s.rt.read("pickup")
        loss, g = s.loss(), s.rt.read("grads")
    finally:
        s.close()
    _, _, t32 = O.membrane_step(s.u0, cfg.T, np.float32(cfg.tgt_c2), np.float32(cfg.tgt_d), cfg.pickup, None,
                                grad=False, want_out=True, prec="f32")
    _, _, o32 = O.membrane_step(s.u0, cfg.T, np.float32(cfg.c2), np.float32(cfg.d), cfg.pickup, None, grad=False,
                                want_out=True, prec="f32")
    print(f"target max err {np.abs(s.target - t32).max():.3e}, pickup max err {np.abs(out - o32).max():.3e}")
    assert np.abs(s.target - t32).max() < 1e-4
    assert np.abs(out - o32).max() < 1e-4
    p = cfg.params().astype(np.float64)
    l64, g64, _ = O.membrane_step(s.u0, cfg.T, p[0], p[1], cfg.pickup, s.target, prec="f64")
    e = np.abs(g - g64) / np.abs(g64)
    print(f"loss HIP {loss:.8e} fp64 {l64:.8e}; grad rel err {e}")
    assert abs(loss - l64) / l64 < 1e-4
    assert e.max() < 1e-2
