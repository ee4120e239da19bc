"""The phase chain (DGEN_HIP_K_PHASOR_CARRY) in its general form, bit for
bit against the oracle's stateful phasor (Emit+State.swift:322-369): f0
blocks holding values outside the fast-step range (tiny, huge) beside
zero and ordinary ones, and lengths that end in a partial interval and a
partial segment; one and two harmonic groups; and the timed build, which
must step the same phases.  The f0 frames the chain reads (the sampleRow
lerp of the f0 rows, Emit+RowSelection.swift:164-197) are checked bit for
bit too, down to a single control row.  Needs a GPU."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import HarmonicConfig
from dgen_hip.programs import harmonic_program
from dgen_hip.runtime import HIPLazyRuntime

pytestmark = pytest.mark.gpu


def render_checkpoints(cfg, f0, uv, X, chain_timer=False):
    with HIPLazyRuntime(harmonic_program(cfg, train=False, chain_timer=chain_timer), 0) as rt:
        rt.write("X", X)
        rt.write("f0", f0)
        rt.write("uv", uv)
        rt.write("params", cfg.weights())
        rt.runNoCopy()
        out = {k: rt.read(k) for k in ("f0_frames", "checkpoints")}
        if chain_timer:
            out["timer"] = rt.read("chain_timer").view(np.uint64).reshape(-1, 8)
        return out


def with_slow_blocks(cfg, f0):
    """f0 [F][B] with runs of control frames outside the fast range: tiny
    (below 2^-20 Hz), huge (above 2^24 / (64 G) Hz) and zero."""
    f0 = f0.copy()
    F = cfg.F
    f0[F // 5:F // 5 + 3, 0] = 1e-30
    f0[F // 2:F // 2 + 2, cfg.B - 1] = 3.0e6
    f0[(3 * F) // 4:(3 * F) // 4 + 40, 0] = 0.0
    return f0


# (T, K): whole intervals; a partial last interval of whole segments; a
# partial last segment; two harmonic groups with a partial segment; fewer
# segments than the producers' lead; one f0 block and a partial second
CASES = [(6400, 60), (6400 + 3 * 64, 60), (6400 + 100, 60), (4096 + 17, 100), (100, 60), (64 * 13 + 5, 60)]


@pytest.mark.parametrize("T,K", CASES, ids=[f"T{t}-K{k}" for t, k in CASES])
def test_checkpoints_bit_exact_with_slow_blocks_and_ragged_ends(gpu, T, K):
    cfg = HarmonicConfig(B=3, T=T, K=K, hidden=32, fft_sizes=(64,))
    print(f"T={T} K={K} B={cfg.B} F={cfg.F}", flush=True)
    f0, uv, X = cfg.data()
    for name, f in (("ordinary f0", f0), ("slow blocks", with_slow_blocks(cfg, f0))):
        out = render_checkpoints(cfg, f, uv, X)
        f0f = out["f0_frames"].reshape(cfg.B, cfg.T)
        np.testing.assert_array_equal(f0f, O.lerp_frames(f, cfg.B, cfg.F, cfg.T))
        slow = ~((f0f == 0) | ((f0f >= 2.0 ** -20) & (f0f < 2.0 ** 24 / (64 * ((K + 63) // 64)))))
        ck = O.phase_checkpoints(f0f, cfg.B, cfg.K, cfg.T, cfg.sr)
        print(f"  {name}: {int(slow.sum())} frames outside the fast range", flush=True)
        np.testing.assert_array_equal(out["checkpoints"].reshape(ck.shape), ck)


def test_timed_build_steps_the_same_phases(gpu):
    cfg = HarmonicConfig(B=2, T=6400 + 100, hidden=32, fft_sizes=(64,))
    f0, uv, X = cfg.data()
    f0 = with_slow_blocks(cfg, f0)
    plain = render_checkpoints(cfg, f0, uv, X)
    timed = render_checkpoints(cfg, f0, uv, X, chain_timer=True)
    np.testing.assert_array_equal(timed["checkpoints"], plain["checkpoints"])
    rec = timed["timer"]
    nseg = (cfg.T + 63) // 64
    assert rec.shape == (cfg.B, 8)
    assert (rec[:, 6] == (nseg + 3) // 4).all()        # intervals
    assert (rec[:, 3] > rec[:, 2]).all() and (rec[:, 5] > rec[:, 4]).all()
    assert (rec[:, 0] < rec[:, 3] - rec[:, 2]).all()   # barrier waits within the run
