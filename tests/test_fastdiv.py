"""The phase kernels divide by the sample rate with a reciprocal product and
two fma corrections (k_harmonic.hip div_sr); it must equal the IEEE quotient
bit for bit on the range they use it on.  Exhaustive for the sample rates of
the benchmark workloads, every 7th float for other common rates."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("fastdiv") / "fastdiv_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, os.path.join(HERE, "fastdiv_check.c"), "-lm"],
                   check=True)
    return exe


def run(exe, *args):
    p = subprocess.run([exe, *args], capture_output=True, text=True)
    return p.returncode, {float(a): int(b) for a, b in (l.split() for l in p.stdout.split("\n") if l.strip())}


def test_exhaustive_for_workload_rates(checker):
    rc, res = run(checker, "16000", "44100")
    assert rc == 0 and res == {16000.0: 0, 44100.0: 0}


def test_sampled_for_common_rates(checker):
    # common rates, the ends of the host-rate range dgen_hip_set_sample_rate
    # accepts ([1, 1e7] Hz) and a few arbitrary ones
    rates = ["8000", "11025", "22050", "24000", "32000", "48000", "88200", "96000", "192000", "1000", "4", "1",
             "10000000", "12345.678", "37011.5", "44099.99"]
    rc, res = run(checker, "sample", *rates)
    assert rc == 0 and all(v == 0 for v in res.values()) and len(res) == len(rates)
