"""Generic UOp blocks: the schedule vocabulary a DGen renderer receives.

The reference compiler hands each backend ``[BlockUOps]``
(Sources/DGen/Renderer/Renderer.swift:3-24): the fused block's UOps
(Sources/DGen/UOps.swift:17-138), its frame order, temporality (frame-based,
hop-based with a counter, static) and ``DispatchMode``
(Renderer.swift:26-67).  This module mirrors that vocabulary on the host and
serialises it to the C ABI (``dgen_hip_block``, include/dgen_hip.h), where
the library renders every block to HIP C++ the way the Metal renderer
renders MSL, compiles it with hiprtc and launches it as a
``DGEN_HIP_K_UOP_BLOCK`` op.  It is the path for blocks that no kernel class
pattern-matches.

Operands are the reference's ``Lazy`` (UOps.swift:1-7): ``const(v)``,
``var(id)``, ``glob(slot)`` (a global, already resolved to its tape slot as
``IRContext.getGlobalId`` does) and ``FRAME_COUNT`` (the variable -1).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

from . import runtime as R

# enum dgen_hip_lazy_kind
L_EMPTY, L_CONST, L_VAR, L_GLOBAL, L_FRAME_COUNT = 0, 1, 2, 3, 4

# enum dgen_hip_uop_op, in the reference's Op order (UOps.swift:17-138)
OP_NAMES = [
    "nop", "load", "store", "delay1", "mutate", "add", "sub", "mul", "div", "abs", "sign", "sin", "cos", "and",
    "or", "xor", "tan", "atan", "tanh", "exp", "log", "log10", "sqrt", "pow", "atan2", "mod", "gt", "gte", "lte",
    "lt", "eq", "min", "max", "floor", "ceil", "round", "noise", "memoryRead", "memoryWrite", "memoryAccumulate",
    "simdBroadcastLoad", "broadcastScalar", "beginIf", "gswitch", "selector", "endIf", "defineGlobal", "loadGlobal",
    "beginLoop", "beginForLoop", "beginReverseLoop", "endLoop", "beginRange", "endRange", "beginParallelRange",
    "endParallelRange", "setThreadCountScale", "setFrameIndex", "output", "input", "frameCount", "hostSampleRate",
    "frameIndex", "threadIndex", "loadTape", "cast", "identity", "declareVar", "beginHopCheck", "endHopCheck",
    "threadgroupArrayDecl", "threadgroupRead", "threadgroupWrite", "threadgroupBarrier",
]
OP = {n: i for i, n in enumerate(OP_NAMES)}

# enum dgen_hip_dispatch (DispatchMode without the GEMM modes)
DISPATCH = {"singleThreaded": 0, "perFrame": 1, "perFrameScaled": 2, "fixedWithFrameLoop": 3, "staticThreads": 4,
            "selfManaged": 5, "selfManagedThreads": 6, "perFrameThreadgroup1": 7, "perFrameScaledThreadgroup1": 8}
FRAME_ORDER = {"sequential": 0, "parallel": 1}
TEMPORALITY = {"frame": 0, "hop": 1, "static": 2}


@dataclass(frozen=True)
class Lazy:
    kind: int
    id: int = 0
    value: float = 0.0


EMPTY = Lazy(L_EMPTY)
FRAME_COUNT = Lazy(L_FRAME_COUNT)


def const(v: float) -> Lazy:
    return Lazy(L_CONST, 0, float(v))


def var(i: int) -> Lazy:
    return Lazy(L_VAR, int(i))


def glob(slot: int) -> Lazy:
    return Lazy(L_GLOBAL, int(slot))


def _lz(x) -> Lazy:
    if isinstance(x, Lazy):
        return x
    if isinstance(x, (int, float)):
        return const(x)
    raise TypeError(f"operand {x!r}")


@dataclass
class UOp:
    op: str
    value: Lazy = EMPTY
    a: Lazy = EMPTY
    b: Lazy = EMPTY
    c: Lazy = EMPTY
    imm: tuple = (0, 0)
    int_typed: bool = False
    options: tuple = ()


@dataclass
class Block:
    """BlockUOps: ops + dispatch mode (name, n) + frame order + temporality."""
    ops: list = field(default_factory=list)
    dispatch: str = "perFrame"
    n: int = 0
    frame_order: str = "parallel"
    temporality: str = "frame"
    hop_size: int = 0
    hop_counter: Lazy = EMPTY


class BlockBuilder:
    """Appends UOps to a block and hands out fresh variable ids, in the
    style of the reference's IRBuilder (IRBuilder.swift): each value op
    returns the operand of its result."""

    def __init__(self, block: Block, first_var: int = 0):
        self.block = block
        self.next_var = first_var

    def _new(self) -> Lazy:
        v = var(self.next_var)
        self.next_var += 1
        return v

    def op(self, name: str, *args, imm=(0, 0), int_typed=False, options=(), value: Lazy | None = None) -> Lazy:
        if name not in OP:
            raise ValueError(f"unknown UOp {name}")
        v = self._new() if value is None else value
        ops = [_lz(a) for a in args] + [EMPTY] * (3 - len(args))
        self.block.ops.append(UOp(name, v, ops[0], ops[1], ops[2], tuple(imm), int_typed,
                                  tuple(_lz(o) for o in options)))
        return v

    def stmt(self, name: str, *args, imm=(0, 0), value: Lazy = EMPTY) -> None:
        ops = [_lz(a) for a in args] + [EMPTY] * (3 - len(args))
        self.block.ops.append(UOp(name, value, ops[0], ops[1], ops[2], tuple(imm)))

    # conveniences mirroring the Op cases
    def __getattr__(self, name):
        if name in OP:
            return lambda *a, **k: self.op(name, *a, **k)
        raise AttributeError(name)


# ---- C ABI structures (include/dgen_hip.h) ---------------------------------
class CLazy(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("id", ctypes.c_int32), ("value", ctypes.c_float),
                ("reserved", ctypes.c_int32)]


class CUop(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int32), ("int_typed", ctypes.c_int32), ("value", CLazy), ("a", CLazy), ("b", CLazy),
                ("c", CLazy), ("imm", ctypes.c_int64 * 2), ("list", ctypes.POINTER(CLazy)), ("n_list", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32)]


class CBlock(ctypes.Structure):
    _fields_ = [("dispatch", ctypes.c_int32), ("dispatch_n", ctypes.c_int32), ("frame_order", ctypes.c_int32),
                ("temporality", ctypes.c_int32), ("hop_size", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("hop_counter", CLazy), ("ops", ctypes.POINTER(CUop)), ("n_ops", ctypes.c_uint32),
                ("reserved2", ctypes.c_uint32)]


def _clazy(l: Lazy) -> CLazy:
    return CLazy(l.kind, l.id, l.value, 0)


class SerializedBlocks:
    """The blocks as C structures; keeps every array alive while in use."""

    def __init__(self, blocks: list):
        self._keep = []
        self.array = (CBlock * max(1, len(blocks)))()
        self.n = len(blocks)
        for i, b in enumerate(blocks):
            ops = (CUop * max(1, len(b.ops)))()
            for j, u in enumerate(b.ops):
                c = ops[j]
                c.op = OP[u.op]
                c.int_typed = 1 if u.int_typed else 0
                c.value, c.a, c.b, c.c = _clazy(u.value), _clazy(u.a), _clazy(u.b), _clazy(u.c)
                c.imm[0], c.imm[1] = int(u.imm[0]), int(u.imm[1])
                if u.options:
                    lst = (CLazy * len(u.options))(*[_clazy(o) for o in u.options])
                    self._keep.append(lst)
                    c.list = ctypes.cast(lst, ctypes.POINTER(CLazy))
                    c.n_list = len(u.options)
            self._keep.append(ops)
            cb = self.array[i]
            if b.dispatch not in DISPATCH:
                raise ValueError(f"dispatch mode {b.dispatch!r} (GEMM blocks go to the GEMM class)")
            cb.dispatch = DISPATCH[b.dispatch]
            cb.dispatch_n = int(b.n)
            cb.frame_order = FRAME_ORDER[b.frame_order]
            cb.temporality = TEMPORALITY[b.temporality]
            cb.hop_size = int(b.hop_size)
            cb.hop_counter = _clazy(b.hop_counter)
            cb.ops = ctypes.cast(ops, ctypes.POINTER(CUop))
            cb.n_ops = len(b.ops)


def render(blocks: list, compile: bool = False) -> str:
    """The HIP C++ source the library generates for these blocks
    (dgen_hip_render_blocks; with ``compile`` also compiled by hiprtc, no
    device needed)."""
    L = R.load_library()
    s = SerializedBlocks(blocks)
    n = ctypes.c_size_t(0)
    R._check(L.dgen_hip_render_blocks(s.array, s.n, 0, None, 0, ctypes.byref(n)), "dgen_hip_render_blocks")
    buf = ctypes.create_string_buffer(n.value + 1)
    R._check(L.dgen_hip_render_blocks(s.array, s.n, 1 if compile else 0, buf, n.value + 1, ctypes.byref(n)),
             "dgen_hip_render_blocks")
    return buf.value.decode()
