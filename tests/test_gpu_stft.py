"""HIP STFT round trip (config 2: window -> FFT -> gains -> IFFT ->
overlap-add, and the gain gradient) against the CPU oracle: forward within
the 1e-4 max-abs parity bar against the fp32 oracle and within a small multiple
of the fp32 oracle's own distance from the fp64 oracle, gradients against the
fp64 oracle and central finite differences, at small ragged shapes and at
the full 8 x 2^20 configuration.  Needs a GPU."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import StftConfig
from dgen_hip.programs import StftSession, stft_program
from dgen_hip.runtime import HIPLazyRuntime

pytestmark = pytest.mark.gpu


def render(cfg, x, gains):
    with HIPLazyRuntime(stft_program(cfg, train=False), 0) as rt:
        rt.write("x", x)
        rt.write("window", cfg.window())
        rt.write("gains", gains)
        rt.runNoCopy()
        return rt.read("y").reshape(cfg.S, cfg.T)


def random_gains(n, seed):
    return np.random.default_rng(seed).uniform(0.3, 1.7, n).astype(np.float32)


@pytest.mark.parametrize("S,T,N,H", [(2, 3000, 64, 16), (3, 10000, 256, 64), (2, 20000, 1024, 256),
                                     (1, 9000, 2048, 512), (2, 5001, 128, 48), (1, 1, 64, 16), (1, 16500, 512, 512)])
def test_forward_matches_oracle(gpu, S, T, N, H):
    cfg = StftConfig(S=S, T=T, N=N, H=H)
    x = cfg.inputs()
    g = random_gains(cfg.bins, N + T)
    print(f"case S={S} T={T} N={N} H={H}", flush=True)
    y = render(cfg, x, g)
    _, _, y32 = O.stft_step(x, N, H, cfg.window(), g, grad=False, want_y=True, prec="f32")
    _, _, y64 = O.stft_step(x, N, H, cfg.window(), g, grad=False, want_y=True, prec="f64")
    err, e_hip, e_o32 = np.abs(y - y32).max(), np.abs(y - y64).max(), np.abs(y32 - y64).max()
    print(f"max|y - y_oracle32| = {err:.3e}; vs fp64: HIP {e_hip:.3e}, fp32 oracle {e_o32:.3e}")
    assert err < 1e-4
    # the GPU FFT takes its twiddles from the hardware sin/cos (~1e-7 absolute)
    # and builds radix-8 powers by products, the oracle's are correctly rounded
    assert e_hip <= 8.0 * e_o32 + 2e-6


def test_identity_gains_reproduce_twice_the_delayed_input(gpu):
    """Size-independent property at the full length: with unit gains the
    periodic-Hann round trip is y[t] = 2 x[t - N + 1]."""
    cfg = StftConfig(S=2)
    x = cfg.inputs()
    y = render(cfg, x, cfg.gains())
    d = cfg.N - 1
    err = max(np.abs(y[:, :d]).max(), np.abs(y[:, d:] - 2.0 * x[:, :cfg.T - d]).max())
    print(f"identity max err {err:.3e}")
    assert err < 1e-5


def small_session(S=2, T=6000, N=256, H=64, optimizer=False, seed=5):
    cfg = StftConfig(S=S, T=T, N=N, H=H)
    return cfg, StftSession(cfg, optimizer=optimizer, gains=random_gains(cfg.bins, seed))


def test_loss_and_gradient_match_oracle(gpu):
    cfg, s = small_session()
    try:
        s.step()
        loss, g = s.loss(), s.rt.read("grads")
        s.step()
        g2 = s.rt.read("grads")
    finally:
        s.close()
    l64, g64, _ = O.stft_step(s.x, cfg.N, cfg.H, s.window, s.gains0, prec="f64")
    _, g32, _ = O.stft_step(s.x, cfg.N, cfg.H, s.window, s.gains0, prec="f32")
    assert abs(loss - l64) / l64 < 1e-5
    e_hip = np.linalg.norm(g - g64) / np.linalg.norm(g64)
    e_o32 = np.linalg.norm(g32 - g64) / np.linalg.norm(g64)
    print(f"grad rel L2 err: HIP {e_hip:.2e}, fp32 oracle {e_o32:.2e}")
    assert e_hip <= max(4 * e_o32, 1e-5)
    np.testing.assert_array_equal(g, g2)  # deterministic


def test_gradient_matches_finite_differences(gpu):
    """Parity bar: within 1e-2 of central differences of the fp64 oracle
    forward, per bin and along the gradient."""
    cfg, s = small_session(S=1, T=3000, N=128, H=32)
    try:
        s.step()
        g = s.rt.read("grads").astype(np.float64)
    finally:
        s.close()
    p = s.gains0.astype(np.float64)

    def loss_at(q):
        return O.stft_step(s.x, cfg.N, cfg.H, s.window, q, grad=False, prec="f64")[0]

    for k in (0, 1, 5, cfg.N // 4, cfg.N // 2 - 1, cfg.N // 2):
        e = np.zeros_like(p)
        e[k] = 1e-6
        fd = (loss_at(p + e) - loss_at(p - e)) / 2e-6
        print(f"bin {k}: HIP {g[k]:.6e} FD {fd:.6e}")
        assert abs(g[k] - fd) <= 1e-2 * abs(fd)
    u = g / np.linalg.norm(g)
    fd = (loss_at(p + 1e-6 * u) - loss_at(p - 1e-6 * u)) / 2e-6
    assert abs(g @ u - fd) <= 1e-2 * abs(fd)


def test_adam_step_matches_oracle(gpu):
    cfg, s = small_session(optimizer=True)
    try:
        s.step()
        g = s.rt.read("grads")
        p1 = s.rt.read("gains")
    finally:
        s.close()
    n = cfg.bins
    ref_p, _, _ = O.adam(s.gains0, g, np.zeros(n, np.float32), np.zeros(n, np.float32), cfg.lr, 0.9, 0.999, 1e-8, 1,
                         prec="f32")
    np.testing.assert_allclose(p1, ref_p, rtol=1e-6, atol=1e-7)


def test_full_configuration_matches_oracle(gpu):
    """8 signals x 2^20 samples, N = 1024, H = 256 (benchmark config 2) at the
    initial unit gains: forward within 1e-4 of the fp32 oracle, loss and
    gain gradient against the fp64 oracle."""
    cfg = StftConfig()
    s = StftSession(cfg, optimizer=False)
    try:
        s.step()
        y = s.rt.read("y").reshape(cfg.S, cfg.T)
        loss, g = s.loss(), s.rt.read("grads")
    finally:
        s.close()
    _, _, y32 = O.stft_step(s.x, cfg.N, cfg.H, s.window, s.gains0, grad=False, want_y=True, prec="f32")
    err = np.abs(y - y32).max()
    print(f"forward max|y - y_oracle| over {y.size} samples = {err:.3e}")
    assert err < 1e-4
    l64, g64, _ = O.stft_step(s.x, cfg.N, cfg.H, s.window, s.gains0, prec="f64")
    print(f"loss HIP {loss:.8e} fp64 {l64:.8e}")
    assert abs(loss - l64) / l64 < 1e-5
    e = np.linalg.norm(g - g64) / np.linalg.norm(g64)
    print(f"grad rel L2 err {e:.2e}, max abs {np.abs(g - g64).max():.2e} of max {np.abs(g64).max():.2e}")
    assert e < 1e-4
