"""HIP tensor biquad bank (config 4: chunked forward scan + BPTT adjoint)
against the CPU oracle: forward within the 1e-4 max-abs parity bar of the
fp32 oracle and no further from the fp64 oracle than twice the fp32 oracle's
own rounding, gradients against the fp64 oracle and central finite
differences, at small ragged shapes and at the full 256 x 2^18
configuration.  Needs a GPU."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import BiquadConfig, HIPError
from dgen_hip.programs import BiquadSession, biquad_program
from dgen_hip.runtime import HIPLazyRuntime

pytestmark = pytest.mark.gpu


def render(cfg, params, x, mod, chunk):
    prog = biquad_program(cfg, train=False, modulated=mod is not None, chunk=chunk)
    with HIPLazyRuntime(prog, 0) as rt:
        rt.write("x", x)
        if mod is not None:
            rt.write("mod", mod)
        rt.write("params", params)
        rt.runNoCopy()
        return rt.read("y").reshape(cfg.T, cfg.B)


def lane_params(B, seed):
    rng = np.random.default_rng(seed)
    return rng.uniform(60.0, 400.0, B).astype(np.float32), rng.uniform(0.4, 3.0, B).astype(np.float32)


@pytest.mark.parametrize("B,T,chunk", [(8, 4096, 256), (3, 1000, 256), (5, 4097, 64), (1, 1, 256), (70, 2000, 7),
                                       (300, 3000, 512), (64, 5000, 1)])
def test_forward_matches_oracle(gpu, B, T, chunk):
    cfg = BiquadConfig(B=B, T=T)
    x, m = cfg.inputs(), cfg.modulation()
    base, Q = lane_params(B, B * 7919 + T)
    print(f"case B={B} T={T} chunk={chunk}", flush=True)
    y = render(cfg, np.concatenate([base, Q]), x, m, chunk)
    y32 = O.biquad_fwd(x, m, base, Q, prec="f32")
    y64 = O.biquad_fwd(x, m, base, Q, prec="f64")
    err, e_hip, e_o32 = (np.abs(y - y32).max(), np.abs(y - y64).max(), np.abs(y32 - y64).max())
    print(f"max|y - y_oracle32| = {err:.3e}; vs fp64: HIP {e_hip:.3e}, fp32 oracle {e_o32:.3e}")
    assert err < 1e-4                      # parity bar
    assert e_hip <= 2.0 * e_o32 + 1e-6     # no worse than the reference's own fp32 rounding


def test_unmodulated_target_bank(gpu):
    cfg = BiquadConfig(B=16, T=6000)
    x = cfg.inputs()
    y = render(cfg, cfg.target_params(), x, None, 256)
    ref = O.biquad_fwd(x, None, cfg.target_params()[:16], cfg.target_params()[16:], prec="f32")
    assert np.abs(y - ref).max() < 1e-5


def small_session(B=6, T=3000, chunk=128, optimizer=False):
    cfg = BiquadConfig(B=B, T=T)
    s = BiquadSession(cfg, optimizer=optimizer, chunk=chunk)
    return cfg, s


def test_loss_and_gradient_match_oracle(gpu):
    cfg, s = small_session()
    try:
        s.step()
        y = s.rt.read("y").reshape(cfg.T, cfg.B)
        loss = s.loss()
        g = s.rt.read("grads")
        y2_run = (s.step(), s.rt.read("y"))[1]
        g2 = s.rt.read("grads")
    finally:
        s.close()
    p = cfg.params()
    l64, g64, y64 = O.biquad_step(s.x, s.mod, p[:cfg.B], p[cfg.B:], s.target, want_y=True, prec="f64")
    _, g32, _ = O.biquad_step(s.x, s.mod, p[:cfg.B], p[cfg.B:], s.target, prec="f32")
    assert np.abs(y - y64).max() < 1e-5
    assert abs(loss - l64) / l64 < 1e-5
    e_hip = np.abs(g - g64) / np.abs(g64)
    e_o32 = np.abs(g32 - g64) / np.abs(g64)
    print(f"grad rel err per component: HIP max {e_hip.max():.2e}, fp32 oracle max {e_o32.max():.2e}")
    assert e_hip.max() < max(4 * e_o32.max(), 1e-4)
    # deterministic: a second run gives identical bits
    np.testing.assert_array_equal(y.reshape(-1), y2_run)
    np.testing.assert_array_equal(g, g2)


@pytest.mark.parametrize("B,T,chunk", [(6, 3000, 128), (70, 2000, 7), (64, 4097, 64)])
def test_fused_adjoint_summaries_equal_the_reverse_pass(gpu, B, T, chunk):
    """The forward replay's prefix-product adjoint summaries and the
    separate reverse pass compose the same affine chunk maps: equal to fp64
    rounding, and the gradients equal to fp32 rounding."""
    cfg = BiquadConfig(B=B, T=T)
    print(f"case B={B} T={T} chunk={chunk}", flush=True)
    target = O.biquad_fwd(cfg.inputs(), None, cfg.target_params()[:B], cfg.target_params()[B:], prec="f32")
    out = {}
    for fused in (True, False):
        s = BiquadSession(cfg, optimizer=False, chunk=chunk, target=target, fuse_adjoint=fused)
        try:
            s.step()
            out[fused] = (s.rt.read("adj_summary").view(np.float64), s.rt.read("grads"), s.loss())
        finally:
            s.close()
    (a1, g1, l1), (a0, g0, l0) = out[True], out[False]
    assert abs(l1 - l0) <= 1e-6 * abs(l0)
    scale = np.abs(a0).max()
    print(f"summary max diff {np.abs(a1 - a0).max():.3e} (scale {scale:.3e})")
    np.testing.assert_allclose(a1, a0, rtol=0, atol=1e-12 * scale)
    np.testing.assert_allclose(g1, g0, rtol=1e-5, atol=1e-6 * np.abs(g0).max())


def test_gradient_matches_finite_differences(gpu):
    """Parity bar: within 1e-2 relative of central differences of the
    fp64 oracle forward, per parameter and along the gradient."""
    cfg, s = small_session(B=4, T=2500, chunk=100)
    try:
        s.step()
        g = s.rt.read("grads").astype(np.float64)
    finally:
        s.close()
    p = cfg.params().astype(np.float64)
    B = cfg.B

    def loss_at(q):
        return O.biquad_step(s.x, s.mod, q[:B], q[B:], s.target, grad=False, prec="f64")[0]

    for j in range(2 * B):
        eps = 1e-6 * abs(p[j])
        e = np.zeros_like(p)
        e[j] = eps
        fd = (loss_at(p + e) - loss_at(p - e)) / (2 * eps)
        print(f"param {j}: HIP {g[j]:.6e} FD {fd:.6e}")
        assert abs(g[j] - fd) <= 1e-2 * abs(fd)
    u = g / np.linalg.norm(g)
    h = 1e-6 * np.linalg.norm(p)
    fd = (loss_at(p + h * u) - loss_at(p - h * u)) / (2 * h)
    assert abs(g @ u - fd) <= 1e-2 * abs(fd)


def test_adam_step_matches_oracle(gpu):
    cfg, s = small_session(optimizer=True)
    try:
        s.step()
        g = s.rt.read("grads")
        p1 = s.rt.read("params")
    finally:
        s.close()
    n = 2 * cfg.B
    ref_p, _, _ = O.adam(cfg.params(), g, np.zeros(n, np.float32), np.zeros(n, np.float32), cfg.lr, 0.9, 0.999,
                         1e-8, 1, prec="f32")
    np.testing.assert_allclose(p1, ref_p, rtol=1e-6, atol=1e-7)


def test_full_configuration_matches_oracle(gpu):
    """256 lanes x 2^18 frames (benchmark config 4): forward within 1e-4
    max-abs of the fp32 oracle over all 2^26 samples, loss and both
    gradients against the fp64 oracle."""
    cfg = BiquadConfig()
    s = BiquadSession(cfg, optimizer=False)
    try:
        s.step()
        y = s.rt.read("y").reshape(cfg.T, cfg.B)
        loss = s.loss()
        g = s.rt.read("grads")
    finally:
        s.close()
    p = cfg.params()
    tgt_ref = O.biquad_fwd(s.x, None, cfg.target_params()[:cfg.B], cfg.target_params()[cfg.B:], prec="f32")
    print(f"target max err {np.abs(s.target - tgt_ref).max():.3e}")
    assert np.abs(s.target - tgt_ref).max() < 1e-4
    l32, _, y32 = O.biquad_step(s.x, s.mod, p[:cfg.B], p[cfg.B:], s.target, grad=False, want_y=True, prec="f32")
    err = np.abs(y - y32).max()
    print(f"forward max|y - y_oracle| over {y.size} samples = {err:.3e}")
    assert err < 1e-4
    l64, g64, _ = O.biquad_step(s.x, s.mod, p[:cfg.B], p[cfg.B:], s.target, prec="f64")
    print(f"loss HIP {loss:.8e} fp64 {l64:.8e}")
    assert abs(loss - l64) / l64 < 1e-5
    e = np.abs(g - g64) / np.abs(g64)
    print(f"grad rel err: base max {e[:cfg.B].max():.2e}, Q max {e[cfg.B:].max():.2e}")
    assert e.max() < 1e-3


def test_chunk_limit_is_an_error(gpu):
    cfg = BiquadConfig(B=1, T=70000)
    with pytest.raises(HIPError, match="chunks"):
        HIPLazyRuntime(biquad_program(cfg, train=False, chunk=1), 0)
