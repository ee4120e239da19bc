"""Config 3 at the size the bench times: B=32 lanes x T=64000 frames, hidden
512, all six FFT sizes, against the CPU oracle; and the north-star gradient
bar (central finite differences of the fp64 oracle forward within 1e-2) at
the full per-lane shape (B=4, T=64000, hidden 512, six sizes).

The oracle runs one lane per call (its loss is the batch mean, so a lane's
call with B=1 gives that lane's share times B), the lanes spread over host
threads (the oracle is plain C behind ctypes, which releases the GIL).
Needs a GPU."""
import dataclasses
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle as O
from dgen_hip import HarmonicConfig
from dgen_hip.programs import HarmonicSession

pytestmark = pytest.mark.gpu

WORKERS = max(1, min(16, os.cpu_count() or 1))


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


class Lanes:
    """The oracle over a batch, one lane per call, lanes on host threads."""

    def __init__(self, cfg, X, f0, uv):
        self.cfg, self.one = cfg, dataclasses.replace(cfg, B=1)
        self.X = X.reshape(cfg.B, cfg.F, cfg.din)
        self.f0, self.uv = f0, uv
        self.pool = ThreadPoolExecutor(WORKERS)

    def lane(self, b):
        return (np.ascontiguousarray(self.X[b]), np.ascontiguousarray(self.f0[:, b:b + 1]),
                np.ascontiguousarray(self.uv[:, b:b + 1]))

    def step(self, P, tgt, grad, prec, want_y=False):
        """Batch loss (mean of lanes), gradient (mean), y [B][T]."""
        def one(b):
            Xb, fb, ub = self.lane(b)
            return O.harmonic_step(self.one, Xb, P, fb, ub, np.ascontiguousarray(tgt[b:b + 1]), grad=grad,
                                   want_y=want_y, prec=prec)
        res = list(self.pool.map(one, range(self.cfg.B)))
        loss = sum(r[0] for r in res) / self.cfg.B
        g = sum(r[1].astype(np.float64) for r in res) / self.cfg.B if grad else None
        y = np.concatenate([r[2] for r in res]) if want_y else None
        return loss, g, y

    def close(self):
        self.pool.shutdown()


@pytest.fixture(scope="module")
def full(gpu):
    cfg = HarmonicConfig()  # B=32, T=64000, hidden 512, FFT 2048..64
    f0, uv, X = cfg.data()
    print(f"config 3 full size: B={cfg.B} T={cfg.T} hidden={cfg.hidden} fft={cfg.fft_sizes}", flush=True)
    s = HarmonicSession(cfg, optimizer=False)  # target rendered on the GPU from the target seed's weights
    try:
        s.step()
        out = {k: s.rt.read(k) for k in ("y", "loss_frames", "f0_frames", "uv_frames", "checkpoints", "playhead",
                                          "noise")}
        out["loss"] = s.loss()
        out["target"] = s.target
    finally:
        s.close()
    lanes = Lanes(cfg, X, f0, uv)
    zeros = np.zeros((cfg.B, cfg.T), np.float32)
    _, _, tgt_ref = lanes.step(cfg.weights(seed=cfg.target_seed), zeros, False, "f32", want_y=True)
    l32, _, y_ref = lanes.step(cfg.weights(), out["target"], False, "f32", want_y=True)
    l64, _, _ = lanes.step(cfg.weights().astype(np.float64), out["target"], False, "f64")
    lanes.close()
    return cfg, f0, uv, out, dict(target=tgt_ref, y=y_ref, l32=l32, l64=l64)


def test_full_size_tables_and_phases_bit_exact(full):
    cfg, f0, uv, out, ref = full
    np.testing.assert_array_equal(out["playhead"], O.playhead(cfg.F, cfg.T))
    np.testing.assert_array_equal(out["noise"], O.noise_stream(cfg.T))
    f0f = O.lerp_frames(f0, cfg.B, cfg.F, cfg.T)
    np.testing.assert_array_equal(out["f0_frames"].reshape(cfg.B, cfg.T), f0f)
    np.testing.assert_array_equal(out["uv_frames"].reshape(cfg.B, cfg.T), O.lerp_frames(uv, cfg.B, cfg.F, cfg.T))
    # all 1000 x 32 x 60 segment-start phases of the sequential fp32 chain
    ck = O.phase_checkpoints(f0f, cfg.B, cfg.K, cfg.T, cfg.sr)
    np.testing.assert_array_equal(out["checkpoints"].reshape(ck.shape), ck)
    # the fp32 playhead drifts and wraps to row 0 in the last frame (reference behaviour)
    print(f"last playhead values {out['playhead'][-3:]}")


def test_full_size_forward_within_1e4(full):
    cfg, f0, uv, out, ref = full
    y = out["y"].reshape(cfg.B, cfg.T)
    err = np.abs(y - ref["y"])
    errt = np.abs(out["target"] - ref["target"]).max()
    print(f"y over {y.size} samples: max|y - oracle| = {err.max():.3e} (last 64 frames {err[:, -64:].max():.3e}); "
          f"GPU-rendered target {errt:.3e}")
    assert err.max() < 1e-4
    assert errt < 1e-4


def test_full_size_loss(full):
    cfg, f0, uv, out, ref = full
    e_hip = abs(out["loss"] - ref["l64"]) / abs(ref["l64"])
    e_o32 = abs(ref["l32"] - ref["l64"]) / abs(ref["l64"])
    print(f"loss {out['loss']:.7f}: rel to fp64 oracle HIP {e_hip:.2e}, fp32 oracle {e_o32:.2e}")
    assert e_hip < 1e-5


@pytest.fixture(scope="module")
def lane4(gpu):
    cfg = HarmonicConfig(B=4)
    f0, uv, X = cfg.data()
    print(f"gradient at the per-lane shape: B={cfg.B} T={cfg.T} hidden={cfg.hidden} fft={cfg.fft_sizes}", flush=True)
    s = HarmonicSession(cfg, optimizer=False)
    try:
        s.step()
        g = s.rt.read("grads").astype(np.float64)
        tgt = s.target
    finally:
        s.close()
    lanes = Lanes(cfg, X, f0, uv)
    P64 = cfg.weights().astype(np.float64)
    _, g64, _ = lanes.step(P64, tgt, True, "f64")
    _, g32, _ = lanes.step(cfg.weights(), tgt, True, "f32")
    yield cfg, lanes, P64, tgt, g, g64, g32
    lanes.close()


def _fd(lanes, P64, tgt, v, eps):
    lp = lanes.step(P64 + eps * v, tgt, False, "f64")[0]
    lm = lanes.step(P64 - eps * v, tgt, False, "f64")[0]
    return (lp - lm) / (2 * eps)


def test_full_shape_gradient_along_gradient_and_random_directions(lane4):
    cfg, lanes, P64, tgt, g, g64, g32 = lane4
    print(f"grad rel L2 vs fp64 oracle: HIP {rel(g, g64):.3e}, fp32 oracle {rel(g32, g64):.3e}")
    u = g64 / np.linalg.norm(g64)
    d = _fd(lanes, P64, tgt, u, 1e-6)
    print(f"along grad: HIP {g @ u:.6e}, fp32 oracle {g32 @ u:.6e}, FD {d:.6e}")
    assert abs(g @ u - d) / abs(d) < 1e-2
    rng = np.random.default_rng(22)
    gn = np.linalg.norm(g)
    for _ in range(3):
        v = rng.standard_normal(len(P64))
        v /= np.linalg.norm(v)
        d = _fd(lanes, P64, tgt, v, 1e-6)
        print(f"random direction: HIP {g @ v:.6e}, FD {d:.6e}, |diff|/|grad| {abs(g @ v - d) / gn:.2e}")
        assert abs(g @ v - d) / gn < 1e-2


def test_full_shape_gradient_largest_components(lane4):
    cfg, lanes, P64, tgt, g, g64, g32 = lane4
    worst = 0.0
    for i in np.argsort(-np.abs(g64))[:8]:
        e = np.zeros_like(P64)
        e[i] = 1.0
        d = _fd(lanes, P64, tgt, e, 1e-7)
        eh, eo = abs(g[i] - d) / abs(d), abs(g32[i] - d) / abs(d)
        print(f"param {i}: HIP {g[i]:.6e}, fp32 oracle {g32[i]:.6e}, FD {d:.6e}; rel err HIP {eh:.2e}, "
              f"fp32 oracle {eo:.2e}")
        worst = max(worst, eh)
    assert worst < 1e-2
