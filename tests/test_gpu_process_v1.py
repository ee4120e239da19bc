"""The reference-named process-function exports dgen_process_v1 /
dgen_set_param_value_v1 (include/dgen_process_v1.h), driven as the
reference's host drives a process-function library
(CCompiledKernel.runWithMemory, Sources/DGen/Runtime.swift:728-787): the
symbols are looked up by name, a state block of getMemorySize() floats is
allocated and zeroed, the parameters are written into it at their cell
offsets (injectTensorData, Sources/DGen/Tensor.swift:320-330), and every
block passes channel pointer arrays and a DGenProcessContextV1.

Any split of a signal into blocks reproduces the context-level streaming
path (dgen_hip_process_v1) bit for bit for configs 1 and 4; re-zeroing the
block resets the graph; two blocks are two independent instances.
Needs a GPU."""
import ctypes

import numpy as np
import pytest

from dgen_hip import BiquadConfig, OscBankConfig
from dgen_hip import runtime as R
from dgen_hip.programs import stream_biquad_program, stream_oscbank_program
from dgen_hip.runtime import HIPLazyRuntime, process_v1

pytestmark = pytest.mark.gpu


def inject(prog, block, **cells):
    """Write parameter cells into a host state block at their offsets."""
    for name, a in cells.items():
        c = prog.cells[name]
        block[c.off:c.off + c.n] = np.asarray(a, np.float32).ravel()


def test_symbols_resolve_by_name(gpu):
    lib = ctypes.CDLL(R.LIB_PATH)
    for name in R.PROCESS_V1_SYMBOLS:
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_oscillator_bank_blocks_reproduce_the_streaming_path(gpu):
    cfg = OscBankConfig()
    prog = stream_oscbank_program(cfg, stateful=True)
    freqs, amps = cfg.inputs()
    rt = HIPLazyRuntime(prog, 0)
    try:
        rt.write("freqs", freqs)
        rt.write("amps", amps)
        rt.setProcessPorts(*prog.meta["ports"])
        one = rt.process([], cfg.frames, reset=True)[0]
        n = rt.bindProcess()
        assert n == max(1024, prog.meta["memory"][1])
        block = np.zeros(n, np.float32)
        inject(prog, block, freqs=freqs, amps=amps)
        fresh = block.copy()
        for sizes in ([cfg.frames], [16384] * 4, [1, 999, 4000, 60000, 536], [512] * 128):
            block[:] = fresh  # the host re-zeroes the block (and re-injects its parameters): a reset
            got = np.concatenate([process_v1([], 1, k, block)[0] for k in sizes])
            print(f"blocks {sizes[:5]}{'...' if len(sizes) > 5 else ''}: max|diff| {np.abs(got - one).max():.3e}")
            np.testing.assert_array_equal(got, one)
        # the carried state is in the block: phases and the one-pole's y[n-1]
        st = prog.cells["state"]
        assert np.any(block[st.off:st.off + st.n] != 0)
        # the parameter entry point is the reference C backend's no-op
        R.load_library().dgen_set_param_value_v1(prog.cells["amps"].off, 123.0)
        block[:] = fresh
        np.testing.assert_array_equal(process_v1([], 1, 4096, block)[0], one[:4096])
    finally:
        rt.close()
    assert R.load_library().dgen_hip_process_memory_size() == 0  # destroying the bound context unbinds it


def test_oscillator_bank_host_rate_and_context_check(gpu):
    cfg = OscBankConfig()
    prog = stream_oscbank_program(cfg, stateful=True)
    freqs, amps = cfg.inputs()
    rt = HIPLazyRuntime(prog, 0)
    try:
        rt.write("freqs", freqs)
        rt.write("amps", amps)
        rt.setProcessPorts(*prog.meta["ports"])
        at_22k = rt.process([], 6000, sample_rate=22050.0, reset=True)[0]
        rendered = rt.process([], 6000, reset=True)[0]
        block = np.zeros(rt.bindProcess(), np.float32)
        inject(prog, block, freqs=freqs, amps=amps)
        fresh = block.copy()
        got = np.concatenate([process_v1([], 1, 3000, block, sample_rate=22050.0)[0] for _ in range(2)])
        np.testing.assert_array_equal(got, at_22k)
        # no context (or one that fails the v1 check) runs at the graph's rate
        block[:] = fresh
        np.testing.assert_array_equal(process_v1([], 1, 6000, block, context=False)[0], rendered)
        # a failing block leaves silence and a message, not an abort
        block[:] = fresh
        out = process_v1([], 1, cfg.frames + 1, block)
        assert np.all(out == 0.0)
        assert b"max_frames" in R.load_library().dgen_hip_last_error()
    finally:
        rt.close()


def test_biquad_bank_blocks_and_independent_instances(gpu):
    cfg = BiquadConfig(B=256, T=1 << 15)
    prog = stream_biquad_program(cfg)
    x, mod, p = cfg.inputs(), cfg.modulation(), cfg.params()
    print(f"process_v1 biquad bank B={cfg.B} T={cfg.T}", flush=True)
    rt = HIPLazyRuntime(prog, 0)
    try:
        rt.write("params", p)
        rt.setProcessPorts(*prog.meta["ports"])
        ins = [x[:, k] for k in range(cfg.B)] + [mod]
        one = rt.process(ins, cfg.T, reset=True).T
        blocks = [np.zeros(rt.bindProcess(), np.float32) for _ in range(2)]
        for b in blocks:
            inject(prog, b, params=p)

        def call(block, n0, n):
            return process_v1([a[n0:n0 + n] for a in ins], cfg.B, n, block).T

        # two instances interleaved block by block, with different splits
        a_parts, b_parts, na, nb = [], [], 0, 0
        for sa, sb in zip([8192] * 4, [1, 4095, 20000, 8672]):
            a_parts.append(call(blocks[0], na, sa))
            na += sa
            b_parts.append(call(blocks[1], nb, sb))
            nb += sb
        np.testing.assert_array_equal(np.concatenate(a_parts), one)
        np.testing.assert_array_equal(np.concatenate(b_parts), one)
        # the block holds the four history cells of every lane
        st = prog.cells["state"]
        assert np.array_equal(blocks[0][st.off:st.off + st.n], blocks[1][st.off:st.off + st.n])
    finally:
        rt.close()
