"""Config 1: deterministic phasor bank -> sin -> sum -> history one-pole on
the GPU against the oracle, at the benchmark size (65536 frames) and at
ragged lengths."""
import numpy as np
import pytest

import oracle as O
from dgen_hip import OscBankConfig
from dgen_hip.programs import oscbank_program
from dgen_hip.runtime import HIPLazyRuntime

pytestmark = pytest.mark.gpu


def run(cfg):
    freqs, amps = cfg.inputs()
    with HIPLazyRuntime(oscbank_program(cfg), 0) as rt:
        rt.write("freqs", freqs)
        rt.write("amps", amps)
        rt.runNoCopy()
        return rt.read("out"), freqs, amps


@pytest.mark.parametrize("frames", [65536, 1, 255, 257, 10000])
def test_oscbank_matches_oracle(gpu, frames):
    cfg = OscBankConfig(frames=frames)
    y, freqs, amps = run(cfg)
    ref = O.oscbank(freqs, amps, cfg.sr, cfg.pole, frames)
    err = np.abs(y - ref).max()
    print(f"frames {frames}: max|y - oracle| = {err:.3e}")
    assert err < 1e-4

