"""The no-allocation bank forward (dgen_hip_biquad_forward_noalloc) against
the schedule's own forward (configure + dgen_hip_run of the biquad render
program, the same kernels on arena cells): bit-identical, on two calls in a
row (the second smaller, so the fixed scratch keeps the first call's
contents), and the size limit of the fixed scratch.  The test's own device
buffers come from the HIP runtime the library links (hipMalloc through
ctypes).  Needs a GPU."""
import ctypes

import numpy as np
import pytest

from dgen_hip import BiquadConfig
from dgen_hip.programs import biquad_program
from dgen_hip.runtime import HIPLazyRuntime, load_library

pytestmark = pytest.mark.gpu


def schedule_forward(cfg, x, mod, params, chunk):
    prog = biquad_program(cfg, train=False, modulated=mod is not None, chunk=chunk)
    with HIPLazyRuntime(prog, 0) as rt:
        rt.write("x", x)
        if mod is not None:
            rt.write("mod", mod)
        rt.write("params", params)
        rt.runNoCopy()
        return rt.read("y").reshape(cfg.T, cfg.B)


class DeviceBuffers:
    """hipMalloc'd copies of host arrays (the caller's buffers)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")  # the runtime libdgen_hip.so is linked against, already loaded
        self.hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.hip.hipFree.argtypes = [ctypes.c_void_p]
        self.ptrs = []

    def put(self, a):
        a = np.ascontiguousarray(a, np.float32)
        p = ctypes.c_void_p()
        assert self.hip.hipMalloc(ctypes.byref(p), a.nbytes) == 0
        self.ptrs.append(p)
        assert self.hip.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) == 0  # host to device
        return p

    def get(self, p, shape):
        out = np.empty(shape, np.float32)
        assert self.hip.hipDeviceSynchronize() == 0
        assert self.hip.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0  # device to host
        return out

    def free(self):
        for p in self.ptrs:
            self.hip.hipFree(p)
        self.ptrs = []


def noalloc_forward(x, mod, params, B, T, chunk):
    L = load_library()
    d = DeviceBuffers()
    try:
        dx, dp = d.put(x), d.put(params)
        dm = d.put(mod) if mod is not None else None
        dy = d.put(np.full((T, B), np.nan, np.float32))  # every output must be written
        rc = L.dgen_hip_biquad_forward_noalloc(0, dx, dm, dp, dy, B, T, chunk, None)
        assert rc == 0, L.dgen_hip_last_error()
        return d.get(dy, (T, B))
    finally:
        d.free()


def test_noalloc_forward_matches_the_schedule_forward_on_two_calls(gpu):
    cases = [(BiquadConfig(B=256, T=1 << 16), True, 512),   # modulated, the config-4 chunk
             (BiquadConfig(B=37, T=3001), False, 64)]         # smaller, ragged, unmodulated
    for cfg, modulated, chunk in cases:
        print(f"no-alloc biquad forward B={cfg.B} T={cfg.T} chunk={chunk} modulated={modulated}", flush=True)
        x, params = cfg.inputs(), cfg.params()
        mod = cfg.modulation() if modulated else None
        ref = schedule_forward(cfg, x, mod, params, chunk)
        got = noalloc_forward(x, mod, params, cfg.B, cfg.T, chunk)
        np.testing.assert_array_equal(got, ref)


def test_noalloc_forward_rejects_banks_beyond_its_scratch(gpu):
    L = load_library()
    # 256 lanes x 2^21 frames in 256-frame chunks need 117 MB of summaries
    rc = L.dgen_hip_biquad_forward_noalloc(0, 8, None, 8, 8, 256, 1 << 21, 256, None)
    assert rc == -4 and b"scratch" in L.dgen_hip_last_error()
    rc = L.dgen_hip_biquad_forward_noalloc(0, None, None, 8, 8, 4, 4, 0, None)
    assert rc == -1
