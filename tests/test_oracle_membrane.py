"""Pins of the config-5 membrane oracle (oracle/dgen_oracle.c, mem_* and
dgen_oracle_membrane_step): the discrete Dirichlet eigenmode closed form
(stencil, update coefficients, u_{-1} = u_0 start and the u_{n+1} pickup),
mirror symmetry of the zero padding, and central finite differences of the
loss for the adjoint.  CPU only."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import MembraneConfig


def eigenmode(R, C, a, b):
    y = np.arange(R)[:, None] + 1.0
    x = np.arange(C)[None, :] + 1.0
    phi = np.sin(np.pi * a * y / (R + 1)) * np.sin(np.pi * b * x / (C + 1))
    mu = -4 * np.sin(np.pi * a / (2 * (R + 1))) ** 2 - 4 * np.sin(np.pi * b / (2 * (C + 1))) ** 2
    return phi, mu


@pytest.mark.parametrize("c2,d", [(0.2, 0.0), (0.25, 0.002), (0.1, 0.05)])
def test_eigenmode_evolves_by_the_scalar_recurrence(c2, d):
    # L phi = mu phi for the zero-padded 5-point stencil, so u_n = T_n phi with
    # T_{n+1} = (2 - d + c2 mu) T_n - (1 - d) T_{n-1}, T_{-1} = T_0 = 1
    R, C, T = 24, 20, 300
    phi, mu = eigenmode(R, C, 3, 2)
    p = (7, 11)
    _, _, out = O.membrane_step(phi.astype(np.float32), T, c2, d, p, None, grad=False, want_out=True)
    M = np.array([[2 - d + c2 * mu, -(1 - d)], [1.0, 0.0]])
    s = np.array([1.0, 1.0])  # (T_0, T_{-1})
    ref = []
    for _ in range(T):
        s = M @ s
        ref.append(s[0])
    ref = np.array(ref) * float(np.float32(phi[p]))
    # the mode is given in fp32, so it is an eigenvector to fp32 accuracy only
    assert np.abs(out - ref).max() < 1e-5 * np.abs(phi).max()


def test_closed_form_cosine_without_damping():
    # d = 0: T_n = cos((n + 1/2) theta) / cos(theta/2), cos theta = 1 + c2 mu / 2
    R, C, T, c2 = 16, 16, 200, 0.22
    phi, mu = eigenmode(R, C, 1, 1)
    p = (8, 8)
    _, _, out = O.membrane_step(phi.astype(np.float32), T, c2, 0.0, p, None, grad=False, want_out=True)
    th = np.arccos(1 + c2 * mu / 2)
    n = np.arange(T) + 1  # out[n] = u_{n+1}
    ref = float(np.float32(phi[p])) * np.cos((n + 0.5) * th) / np.cos(th / 2)
    assert np.abs(out - ref).max() < 1e-5


def test_zero_padding_is_mirror_symmetric():
    cfg = MembraneConfig(R=40, C=40, T=150)
    u0 = cfg.bump()
    p = (10, 31)
    _, _, a = O.membrane_step(u0, cfg.T, 0.2, 0.01, p, None, grad=False, want_out=True)
    _, _, b = O.membrane_step(np.ascontiguousarray(u0[::-1, ::-1]), cfg.T, 0.2, 0.01,
                              (39 - p[0], 39 - p[1]), None, grad=False, want_out=True)
    np.testing.assert_allclose(a, b, atol=1e-12)


def test_fp32_build_close_to_fp64():
    cfg = MembraneConfig(R=64, C=64, T=600)
    u0 = cfg.bump()
    _, _, o32 = O.membrane_step(u0, cfg.T, cfg.c2, cfg.d, cfg.pickup, None, grad=False, want_out=True, prec="f32")
    _, _, o64 = O.membrane_step(u0, cfg.T, cfg.c2, cfg.d, cfg.pickup, None, grad=False, want_out=True, prec="f64")
    assert np.abs(o32 - o64).max() < 1e-5 * np.abs(o64).max()


@pytest.mark.parametrize("T", [300, 7, 1])
def test_gradient_matches_central_differences(T):
    cfg = MembraneConfig(R=32, C=28, T=T)
    u0 = cfg.bump()
    _, _, tgt = O.membrane_step(u0, T, cfg.tgt_c2, cfg.tgt_d, cfg.pickup, None, grad=False, want_out=True)
    p0 = np.array([cfg.c2, cfg.d])
    _, g, _ = O.membrane_step(u0, T, p0[0], p0[1], cfg.pickup, tgt)
    for j in range(2):
        eps = 1e-6 * abs(p0[j])
        pp, pm = p0.copy(), p0.copy()
        pp[j] += eps
        pm[j] -= eps
        fd = (O.membrane_step(u0, T, *pp, cfg.pickup, tgt, grad=False)[0]
              - O.membrane_step(u0, T, *pm, cfg.pickup, tgt, grad=False)[0]) / (2 * eps)
        assert abs(g[j] - fd) <= 1e-6 * abs(fd) + 1e-12, (j, g[j], fd)


def test_loss_is_sum_of_squared_pickup_error():
    cfg = MembraneConfig(R=24, C=24, T=50)
    u0 = cfg.bump()
    tgt = np.random.default_rng(1).standard_normal(cfg.T).astype(np.float32) * 0.01
    loss, _, out = O.membrane_step(u0, cfg.T, cfg.c2, cfg.d, cfg.pickup, tgt, grad=False, want_out=True)
    assert loss == pytest.approx(float(((out.astype(np.float64) - tgt) ** 2).sum()), rel=1e-6)
