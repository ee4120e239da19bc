"""Runs replayed as a captured HIP graph (dgen_hip_set_graphs) against the
same schedule enqueued kernel by kernel.  Two sessions start from the same
state; each takes several training steps (forward, loss, backward, Adam),
the graph session with the program's own eager work between its replays
(downloads, an upload, synchronisation, a profiled eager run); after every
step the trained parameters, gradients and outputs must be bit-identical
(every kernel here is deterministic).  The harmonic schedule also forks a
side stream, so its capture exercises the fork/join.  Needs a GPU."""
import numpy as np
import pytest

from dgen_hip import BiquadConfig, HarmonicConfig, MembraneConfig, StftConfig
from dgen_hip.programs import BiquadSession, HarmonicSession, MembraneSession, StftSession

pytestmark = pytest.mark.gpu


def _harmonic():
    cfg = HarmonicConfig(B=2, T=2048, hidden=64, fft_sizes=(512, 256, 128, 64))
    tgt = np.sin(np.arange(cfg.B * cfg.T, dtype=np.float64) * 0.05).astype(np.float32).reshape(cfg.B, cfg.T) * 0.1
    return (lambda: HarmonicSession(cfg, optimizer=True, target=tgt)), ["params", "grads", "y", "loss_frames"]


def _biquad():
    cfg = BiquadConfig(B=8, T=3000)
    tgt = np.zeros((cfg.T, cfg.B), np.float32)
    return (lambda: BiquadSession(cfg, optimizer=True, target=tgt)), ["params", "y"]


def _stft():
    cfg = StftConfig(S=2, T=16384, N=1024, H=256)
    return (lambda: StftSession(cfg, optimizer=True)), ["gains", "loss"]


def _membrane(R, C, T):
    cfg = MembraneConfig(R=R, C=C, T=T)
    tgt = np.zeros(cfg.T, np.float32)
    return (lambda: MembraneSession(cfg, optimizer=True, target=tgt)), ["params", "grads", "pickup", "loss"]


CASES = {
    "harmonic": _harmonic,
    "biquad": _biquad,
    "stft": _stft,
    "membrane_centred": lambda: _membrane(48, 40, 150),
    "membrane_inside": lambda: _membrane(64, 96, 150),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_graph_replay_matches_eager(gpu, case):
    make, cells = CASES[case]()
    print(f"case {case}", flush=True)
    eager, graph = make(), make()
    try:
        graph.rt.set_graphs(True)
        for step in range(4):
            eager.rt.runNoCopy()
            graph.rt.run_async()
            graph.rt.sync()
            for name in cells:
                a, b = eager.rt.read(name), graph.rt.read(name)
                assert np.array_equal(a, b), f"{case}: step {step}: cell {name} differs (max {np.abs(a - b).max()})"
            if step == 1:
                # eager work between replays: re-upload the parameters the
                # graph session holds, and an op-by-op profiled run on both
                graph.rt.write("params" if "params" in graph.program.cells else "gains",
                               graph.rt.read("params" if "params" in graph.program.cells else "gains"))
                eager.rt.profileKernels()
                graph.rt.profileKernels()
    finally:
        eager.close()
        graph.close()
