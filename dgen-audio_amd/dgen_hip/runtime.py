"""ctypes binding of libdgen_hip.so and the host-side runtime object.

``HIPLazyRuntime`` mirrors the reference's ``LazyRuntime`` protocol
(Sources/DGenLazy/Realize.swift:12-19): ``cellAllocations``,
``zeroAllBuffers()``, ``runNoCopy(frameCount)``, ``memoryPointer()``,
``outputsPointer()`` and ``profileKernels(frameCount)``.  It drives the C ABI
declared in include/dgen_hip.h; there is no CPU fallback: every call goes to
the HIP library, and a missing library or device raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

from .program import Program

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdgen_hip.so")

NARG, NFARG = 32, 8

# kernel classes (enum dgen_hip_kernel)
K_ACCUM_TABLE = 1
K_DENSE_SMALL = 2
K_GEMM = 3
K_HEADS_FWD = 4
K_PHASOR_CARRY = 5
K_SYNTH_FWD = 6
K_SPECTRAL_LOSS = 7
K_SPECTRAL_GATHER = 8
K_SYNTH_BWD = 9
K_SYNTH_BWD_REDUCE = 10
K_HEADS_BWD = 11
K_COLSUM = 12
K_DENSE_SMALL_WGRAD = 13
K_ADAM = 14
K_OSC_BANK = 15
K_NOISE_TABLE = 16
K_ROW_SCHEDULE = 17
K_FFT_TABLES = 18
K_LERP_FRAMES = 19
K_BIQUAD_CHUNK = 20
K_BIQUAD_CARRY = 21
K_BIQUAD_FWD = 22
K_BIQUAD_ADJ_CHUNK = 23
K_BIQUAD_BWD = 24
K_STFT_FWD = 25
K_STFT_BWD = 26
K_MEMBRANE_FWD = 27
K_MEMBRANE_BWD = 28
K_STREAM_OSC_BANK = 29
K_STREAM_BIQUAD = 30
K_TEMPORAL_GRAD_SCAN = 31
K_SWEPT_PHASOR = 32
K_SVF_CHUNK = 33
K_SVF_FWD = 34
K_SVF_SEQ = 35
K_SVF_ADJ_CHUNK = 36
K_SVF_BWD = 37
K_STREAM_SVF = 38
K_SPLIT_BF16 = 39
K_UOP_BLOCK = 40
K_RUN_TABLE = 41

KERNEL_NAMES = {v: k[2:].lower() for k, v in globals().items() if k.startswith("K_")}

EPI_NONE, EPI_BIAS, EPI_BIAS_TANH, EPI_TANH_GRAD = 0, 1, 2, 3
OP_STATIC, OP_SIDE, OP_JOIN, OP_FORK = 1, 2, 4, 8

EXPORTED_SYMBOLS = (
    "dgen_hip_abi_version", "dgen_hip_device_count", "dgen_hip_create", "dgen_hip_destroy",
    "dgen_hip_last_error", "dgen_hip_configure", "dgen_hip_host_memory", "dgen_hip_upload",
    "dgen_hip_download", "dgen_hip_zero", "dgen_hip_run", "dgen_hip_run_async", "dgen_hip_sync", "dgen_hip_set_graphs",
    "dgen_hip_profile", "dgen_hip_time_runs", "dgen_hip_time_op", "dgen_hip_time_op_alone", "dgen_hip_run_op",
    "dgen_hip_set_outputs",
    "dgen_hip_host_outputs", "dgen_hip_set_sample_rate", "dgen_hip_biquad_forward_noalloc",
    "dgen_hip_set_process_ports", "dgen_hip_process_v1", "dgen_hip_process_bind", "dgen_hip_process_memory_size",
    "dgen_hip_set_blocks", "dgen_hip_render_blocks",
)
# the reference-named process-function exports (include/dgen_process_v1.h)
PROCESS_V1_SYMBOLS = ("dgen_process_v1", "dgen_set_param_value_v1")
DGEN_ABI_VERSION_V1 = 1
PROCESS_RESET = 1


class HIPError(RuntimeError):
    """A libdgen_hip call returned a negative status."""


class COp(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_uint32), ("flags", ctypes.c_uint32),
                ("arg", ctypes.c_int64 * NARG), ("farg", ctypes.c_float * NFARG)]


class CProcessContext(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32), ("sample_rate", ctypes.c_float),
                ("flags", ctypes.c_uint32)]


class DGenProcessContextV1(ctypes.Structure):
    """The reference's process context (dgen_runtime.h:252-257)."""
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32), ("sample_rate", ctypes.c_float),
                ("reserved", ctypes.c_uint32)]


class CKernelTime(ctypes.Structure):
    _fields_ = [("index", ctypes.c_uint32), ("kernel", ctypes.c_uint32), ("gpu_ms", ctypes.c_float)]


_LIB: ctypes.CDLL | None = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libdgen_hip.so (built in-tree by __graft_entry__.build())."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise HIPError(f"{path} is missing: build the HIP extension first (python -c "
                       f"'import __graft_entry__ as g; g.build()')")
    L = ctypes.CDLL(path)
    vp, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
    sig = {
        "dgen_hip_abi_version": ([], i32),
        "dgen_hip_device_count": ([ctypes.POINTER(i32)], i32),
        "dgen_hip_create": ([i32, ctypes.POINTER(vp)], i32),
        "dgen_hip_destroy": ([vp], i32),
        "dgen_hip_last_error": ([], ctypes.c_char_p),
        "dgen_hip_configure": ([vp, ctypes.POINTER(COp), u32, u64, u32], i32),
        "dgen_hip_host_memory": ([vp], ctypes.POINTER(ctypes.c_float)),
        "dgen_hip_upload": ([vp, u64, u64], i32),
        "dgen_hip_download": ([vp, u64, u64], i32),
        "dgen_hip_zero": ([vp, u64, u64], i32),
        "dgen_hip_run": ([vp, u32], i32),
        "dgen_hip_run_async": ([vp, u32], i32),
        "dgen_hip_set_graphs": ([vp, i32], i32),
        "dgen_hip_sync": ([vp], i32),
        "dgen_hip_profile": ([vp, u32, ctypes.POINTER(CKernelTime), ctypes.c_size_t,
                              ctypes.POINTER(ctypes.c_size_t)], i32),
        "dgen_hip_time_runs": ([vp, u32, i32, i32, ctypes.POINTER(ctypes.c_double)], i32),
        "dgen_hip_time_op": ([vp, u32, u32, i32, ctypes.POINTER(ctypes.c_double)], i32),
        "dgen_hip_time_op_alone": ([vp, u32, u32, i32, ctypes.POINTER(ctypes.c_double)], i32),
        "dgen_hip_run_op": ([vp, u32, u32], i32),
        "dgen_hip_set_outputs": ([vp, u64, u64], i32),
        "dgen_hip_host_outputs": ([vp, ctypes.POINTER(u64)], ctypes.POINTER(ctypes.c_float)),
        "dgen_hip_set_sample_rate": ([vp, ctypes.c_float], i32),
        "dgen_hip_biquad_forward_noalloc": ([i32, vp, vp, vp, vp, u32, u32, u32, vp], i32),
        "dgen_hip_set_process_ports": ([vp, u32, ctypes.POINTER(u64), ctypes.POINTER(u32), u32,
                                        ctypes.POINTER(u64), ctypes.POINTER(u32)], i32),
        "dgen_hip_process_v1": ([vp, ctypes.POINTER(ctypes.POINTER(ctypes.c_float)),
                                 ctypes.POINTER(ctypes.POINTER(ctypes.c_float)), u32, ctypes.POINTER(CProcessContext)],
                                i32),
        "dgen_hip_process_bind": ([vp, u64, u64], i32),
        "dgen_hip_process_memory_size": ([], u64),
        "dgen_process_v1": ([ctypes.POINTER(ctypes.POINTER(ctypes.c_float)),
                             ctypes.POINTER(ctypes.POINTER(ctypes.c_float)), u32, vp,
                             ctypes.POINTER(DGenProcessContextV1), vp], None),
        "dgen_set_param_value_v1": ([ctypes.c_int32, ctypes.c_float], None),
        "dgen_hip_set_blocks": ([vp, vp, u32], i32),
        "dgen_hip_render_blocks": ([vp, u32, i32, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)],
                                   i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _LIB = L
    return L


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().dgen_hip_last_error().decode(errors="replace")
        raise HIPError(f"{what} failed ({rc}): {msg}")


def device_count() -> int:
    L = load_library()
    n = ctypes.c_int(0)
    rc = L.dgen_hip_device_count(ctypes.byref(n))
    return n.value if rc == 0 else 0


@dataclass
class KernelTiming:
    index: int
    name: str
    dispatch_info: str
    gpu_ms: float


class HIPLazyRuntime:
    """Runtime for one compiled program on one device (LazyRuntime mirror)."""

    def __init__(self, program: Program, device: int = 0):
        self.L = load_library()
        self.program = program
        self.cellAllocations = program.cells
        ctx = ctypes.c_void_p()
        _check(self.L.dgen_hip_create(device, ctypes.byref(ctx)), "dgen_hip_create")
        self._ctx = ctx
        ops = (COp * max(1, len(program.ops)))()
        for i, op in enumerate(program.ops):
            ops[i].kernel = op.kernel
            ops[i].flags = op.flags
            for j, a in enumerate(op.arg):
                ops[i].arg[j] = int(a)
            for j, a in enumerate(op.farg):
                ops[i].farg[j] = float(a)
        self._ops = ops
        if program.blocks:
            # generic UOp blocks: rendered, compiled and loaded before the
            # schedule that launches them is configured
            from .uop import SerializedBlocks
            self._blocks = SerializedBlocks(program.blocks)
            _check(self.L.dgen_hip_set_blocks(ctx, self._blocks.array, self._blocks.n), "dgen_hip_set_blocks")
        # Static ops run inside configure and may read data cells, so data
        # staged before configure would be lost; the program's static ops only
        # read constants, and inputs are written afterwards via write().
        _check(self.L.dgen_hip_configure(ctx, ops, len(program.ops), program.size, program.max_frames),
               "dgen_hip_configure")
        ptr = self.L.dgen_hip_host_memory(ctx)
        self._host = np.ctypeslib.as_array(ptr, shape=(program.size,))
        if program.output_cell:
            c = program.cells[program.output_cell]
            _check(self.L.dgen_hip_set_outputs(ctx, c.off, c.n), "dgen_hip_set_outputs")

    # -- LazyRuntime protocol -------------------------------------------
    def zeroAllBuffers(self) -> None:
        _check(self.L.dgen_hip_zero(self._ctx, 0, 0), "dgen_hip_zero")
        self._host[:] = 0.0

    def _frames(self, frameCount: int | None) -> int:
        """None means the frame count the program was rendered for; any
        other value goes to the library as is (it rejects what the schedule
        cannot run, 0 included)."""
        return self.program.max_frames if frameCount is None else int(frameCount)

    def runNoCopy(self, frameCount: int | None = None) -> None:
        _check(self.L.dgen_hip_run(self._ctx, self._frames(frameCount)), "dgen_hip_run")

    def memoryPointer(self) -> np.ndarray:
        return self._host

    def setOutputs(self, cell: str | None) -> None:
        """Declare the program's cell `cell` as the output cells that every
        dgen_hip_run (and the sync after a run_async) copies to the host, or
        none (None).  The program's output_cell is declared at configure."""
        if cell is None:
            _check(self.L.dgen_hip_set_outputs(self._ctx, 0, 0), "dgen_hip_set_outputs")
        else:
            c = self.program.cells[cell]
            _check(self.L.dgen_hip_set_outputs(self._ctx, c.off, c.n), "dgen_hip_set_outputs")

    def outputsPointer(self) -> np.ndarray:
        """The output cells in the host mirror, as the last run left them
        (dgen_hip_run copies them back; dgen_hip_host_outputs)."""
        n = ctypes.c_uint64(0)
        ptr = self.L.dgen_hip_host_outputs(self._ctx, ctypes.byref(n))
        if not ptr or n.value == 0:
            raise HIPError("the program declares no output cells")
        return np.ctypeslib.as_array(ptr, shape=(n.value,))

    def setSampleRate(self, sample_rate: float) -> None:
        """Host sample rate of later runs (0: the rendered rate); the
        DGenProcessContextV1.sample_rate of the reference's C backend."""
        _check(self.L.dgen_hip_set_sample_rate(self._ctx, float(sample_rate)), "dgen_hip_set_sample_rate")

    def profileKernels(self, frameCount: int | None = None) -> list[KernelTiming]:
        cap = len(self.program.ops)
        buf = (CKernelTime * max(1, cap))()
        n = ctypes.c_size_t(0)
        _check(self.L.dgen_hip_profile(self._ctx, self._frames(frameCount), buf, cap,
                                       ctypes.byref(n)), "dgen_hip_profile")
        out = []
        for i in range(min(n.value, cap)):
            op = self.program.ops[buf[i].index]
            out.append(KernelTiming(buf[i].index, op.label or KERNEL_NAMES.get(buf[i].kernel, "?"),
                                    op.dispatch, buf[i].gpu_ms))
        return out

    # -- cell helpers ---------------------------------------------------
    def write(self, name: str, data) -> None:
        c = self.program.cells[name]
        a = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        if a.size != c.n:
            raise ValueError(f"cell {name}: {a.size} values for {c.n} floats")
        self._host[c.off:c.off + c.n] = a
        _check(self.L.dgen_hip_upload(self._ctx, c.off, c.n), f"upload {name}")

    def download(self, name: str) -> None:
        c = self.program.cells[name]
        _check(self.L.dgen_hip_download(self._ctx, c.off, c.n), f"download {name}")

    def read(self, name: str) -> np.ndarray:
        c = self.program.cells[name]
        self.download(name)
        return self._host[c.off:c.off + c.n].copy()

    # -- streaming process calls (dgen_process_v1) ----------------------
    def setProcessPorts(self, inputs, outputs) -> None:
        """Channels of process(): lists of (cell name, lane, lanes) for
        [frames][lanes] cells (one channel per lane, stride lanes)."""
        def cells(ports):
            off = (ctypes.c_uint64 * max(1, len(ports)))()
            st = (ctypes.c_uint32 * max(1, len(ports)))()
            for i, (name, lane, lanes) in enumerate(ports):
                off[i] = self.program.cells[name].off + lane
                st[i] = lanes
            return off, st
        (io, ist), (oo, ost) = cells(inputs), cells(outputs)
        self._ports = (len(inputs), len(outputs))
        _check(self.L.dgen_hip_set_process_ports(self._ctx, len(inputs), io, ist, len(outputs), oo, ost),
               "dgen_hip_set_process_ports")

    def process(self, inputs, frames: int, sample_rate: float = 0.0, reset: bool = False) -> np.ndarray:
        """One dgen_hip_process_v1 block: inputs [n_in][frames] -> outputs [n_out][frames]."""
        n_in, n_out = self._ports
        fp = ctypes.POINTER(ctypes.c_float)
        ins = [np.ascontiguousarray(a, np.float32) for a in inputs]
        if len(ins) != n_in or any(a.shape != (frames,) for a in ins):
            raise ValueError(f"process: {n_in} input channels of {frames} frames expected")
        outs = np.zeros((n_out, frames), np.float32)
        ip = (fp * max(1, n_in))(*[a.ctypes.data_as(fp) for a in ins])
        op = (fp * max(1, n_out))(*[outs[i].ctypes.data_as(fp) for i in range(n_out)])
        ctxv = CProcessContext(2, ctypes.sizeof(CProcessContext), float(sample_rate), PROCESS_RESET if reset else 0)
        _check(self.L.dgen_hip_process_v1(self._ctx, ip, op, int(frames), ctypes.byref(ctxv)), "dgen_hip_process_v1")
        return outs

    def bindProcess(self) -> int:
        """Bind this runtime's schedule to the reference-named exports
        dgen_process_v1 / dgen_set_param_value_v1 (dgen_hip_process_bind), with
        the program's graph memory (``meta["memory"]``: the cells the reference
        keeps in the host's state block).  The process ports must be set.
        Returns the state block size in floats (dgen_hip_process_memory_size)."""
        off, end = self.program.meta["memory"]
        _check(self.L.dgen_hip_process_bind(self._ctx, off, end - off), "dgen_hip_process_bind")
        return int(self.L.dgen_hip_process_memory_size())

    def set_graphs(self, enable: bool = True) -> None:
        """Replay runs as a captured HIP graph (dgen_hip_set_graphs)."""
        _check(self.L.dgen_hip_set_graphs(self._ctx, 1 if enable else 0), "dgen_hip_set_graphs")

    def run_async(self, frameCount: int | None = None) -> None:
        _check(self.L.dgen_hip_run_async(self._ctx, self._frames(frameCount)), "dgen_hip_run_async")

    def sync(self) -> None:
        _check(self.L.dgen_hip_sync(self._ctx), "dgen_hip_sync")

    def time_runs(self, warmup: int, iters: int, frameCount: int | None = None) -> float:
        ms = ctypes.c_double(0.0)
        _check(self.L.dgen_hip_time_runs(self._ctx, self._frames(frameCount), warmup, iters,
                                         ctypes.byref(ms)), "dgen_hip_time_runs")
        return ms.value

    def time_op(self, index: int, iters: int, frameCount: int | None = None) -> float:
        ms = ctypes.c_double(0.0)
        _check(self.L.dgen_hip_time_op(self._ctx, self._frames(frameCount), index, iters,
                                       ctypes.byref(ms)), "dgen_hip_time_op")
        return ms.value

    def time_op_alone(self, index: int, iters: int, frameCount: int | None = None) -> float:
        """Average ms of op `index` run alone, back to back on stream 0."""
        ms = ctypes.c_double(0.0)
        _check(self.L.dgen_hip_time_op_alone(self._ctx, self._frames(frameCount), index, iters,
                                             ctypes.byref(ms)), "dgen_hip_time_op_alone")
        return ms.value

    def run_op(self, index: int, frameCount: int | None = None) -> None:
        """Run schedule op `index` alone on the current cell contents."""
        _check(self.L.dgen_hip_run_op(self._ctx, self._frames(frameCount), index), "dgen_hip_run_op")

    def close(self) -> None:
        if getattr(self, "_ctx", None):
            # (destroying the bound context unbinds the process exports)
            self.L.dgen_hip_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def process_v1(inputs, n_out: int, frames: int, state: np.ndarray, sample_rate: float | None = None,
               context: bool = True) -> np.ndarray:
    """Drive the reference-named export dgen_process_v1 as a host does
    (CCompiledKernel.runWithMemory, Runtime.swift:746-787): channel pointer
    arrays, the caller's state block (a float32 array of
    dgen_hip_process_memory_size() values, zeroed by the host for a fresh
    instance) and a DGenProcessContextV1 carrying the host rate.  Returns the
    output channels [n_out][frames].  Failures leave the outputs at 0 (the
    export returns nothing); the message is in dgen_hip_last_error()."""
    L = load_library()
    fp = ctypes.POINTER(ctypes.c_float)
    ins = [np.ascontiguousarray(a, np.float32) for a in inputs]
    outs = np.full((n_out, frames), np.nan, np.float32)
    ip = (fp * max(1, len(ins)))(*[a.ctypes.data_as(fp) for a in ins])
    op = (fp * max(1, n_out))(*[outs[i].ctypes.data_as(fp) for i in range(n_out)])
    if state.dtype != np.float32 or not state.flags["C_CONTIGUOUS"]:
        raise ValueError("state block: a contiguous float32 array")
    c = DGenProcessContextV1(DGEN_ABI_VERSION_V1, ctypes.sizeof(DGenProcessContextV1),
                             0.0 if sample_rate is None else float(sample_rate), 0)
    L.dgen_process_v1(ip, op, int(frames), state.ctypes.data_as(ctypes.c_void_p),
                      ctypes.byref(c) if context else None, None)
    return outs

