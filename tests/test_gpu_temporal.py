"""Temporal gradient of stateful accumulators on the GPU: the chunked
reset-aware suffix scan (DGEN_HIP_K_TEMPORAL_GRAD_SCAN) against the oracle's
sequential scan (Emit+TemporalGradient.swift:56-81), and the swept-phasor
bank's gradient to its learnable sweep rates against the fp64 oracle and
central finite differences of it (TemporalGradientTests.swift:24-60 scaled
to 256 lanes x 2^16 frames).  Needs a GPU."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import SweptPhasorConfig
from dgen_hip import runtime as R
from dgen_hip.program import Program
from dgen_hip.programs import SweptPhasorSession

pytestmark = pytest.mark.gpu


def scan_program(E, T):
    p = Program(max_frames=T)
    g = p.alloc("g", T * E)
    rs = p.alloc("reset", T)
    out = p.alloc("out", T * E)
    C = (T + 255) // 256
    ws = p.alloc("ws", 2 * C * E + C)
    p.add(R.K_TEMPORAL_GRAD_SCAN, [g, rs, out, E, T, ws, 0], [44100.0], label="scan")
    p.output_cell = "out"
    return p


def scan64(g, rs):
    """The same scan in fp64 (the rounding-free value both fp32 scans approximate)."""
    out = np.zeros(g.shape)
    carry = np.zeros(g.shape[1])
    for n in range(g.shape[0] - 1, -1, -1):
        active = 0.0 * carry if rs[n] > 0 else carry
        out[n] = active
        carry = g[n] + active
    return out


@pytest.mark.parametrize("E,T", [(256, (1 << 16) + 123), (1, 5000), (70, 256)])
def test_scan_matches_oracle(gpu, E, T):
    rng = np.random.default_rng(E + T)
    g = rng.standard_normal((T, E)).astype(np.float32)
    n = np.arange(T)
    resets = {"none": np.zeros(T), "every 1000": (n % 1000 == 999), "from half": n >= T // 2,
              "isolated": np.isin(n, [0, 255, 256, T - 1]), "all": np.ones(T)}
    with R.HIPLazyRuntime(scan_program(E, T), 0) as rt:
        rt.write("g", g)
        for name, rs in resets.items():
            rs = np.asarray(rs, np.float32)
            rt.write("reset", rs)
            rt.runNoCopy()
            got = rt.read("out").reshape(T, E)
            ref = O.temporal_scan(g, rs)
            ref64 = scan64(g, rs)
            e_hip, e_o32 = np.abs(got - ref64).max(), np.abs(ref - ref64).max()
            scale = np.abs(ref64).max() + 1.0
            print(f"E={E} T={T} resets {name}: max|out - fp64| HIP {e_hip:.3e}, fp32 oracle {e_o32:.3e} "
                  f"(max |out| {scale - 1:.3e})")
            # the chunked scan reassociates only the carries between chunks:
            # within 2x the sequential fp32 oracle's rounding
            assert e_hip <= 2.0 * e_o32 + 1e-6 * scale
            assert np.all(got[rs > 0] == 0.0)  # a reset frame discards its increment


@pytest.mark.parametrize("reset_from", [-1, 40000])
def test_swept_phasor_gradient(gpu, reset_from):
    cfg = SweptPhasorConfig(reset_from=reset_from)
    print(f"swept phasor bank E={cfg.E} T={cfg.T} reset_from={reset_from}", flush=True)
    s = SweptPhasorSession(cfg, optimizer=False)
    try:
        s.step()
        loss, g = s.loss(), s.rt.read("grads").astype(np.float64)
    finally:
        s.close()
    slopes = cfg.slopes()
    args = (cfg.T, cfg.sr, cfg.base, cfg.target, reset_from, cfg.smooth)
    l64, g64, _ = O.swept_phasor_step(slopes.astype(np.float64), *args)
    l32, g32, _ = O.swept_phasor_step(slopes, *args, prec="f32")
    e_hip, e_o32 = np.linalg.norm(g - g64) / np.linalg.norm(g64), np.linalg.norm(g32 - g64) / np.linalg.norm(g64)
    print(f"loss {loss:.6e} (fp64 oracle {l64:.6e}); grad rel L2 vs fp64: HIP {e_hip:.3e}, fp32 oracle {e_o32:.3e}")
    assert abs(loss - l64) <= 1e-4 * abs(l64)
    assert e_hip <= 2.0 * e_o32 + 1e-5
    for e in (0, cfg.E // 2, cfg.E - 1):  # central differences of the fp64 oracle, one lane at a time
        sl = np.array([slopes[e]], np.float64)
        eps = 1e-7 * sl[0]
        lp = O.swept_phasor_step(sl + eps, *args, grad=False)[0]
        lm = O.swept_phasor_step(sl - eps, *args, grad=False)[0]
        d = (lp - lm) / (2 * eps)
        print(f"lane {e} slope {sl[0]:.1f}: HIP {g[e]:.6e}, FD {d:.6e}")
        # fp32 phases: lanes whose gradient cancels to a few units carry the
        # bank's absolute fp32 error, hence the floor at 1e-3 of the largest
        assert abs(g[e] - d) <= 1e-2 * abs(d) + 1e-3 * np.abs(g64).max()
