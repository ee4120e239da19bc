"""A compiled program for the HIP backend: cell allocations over one flat
float arena plus an ordered schedule of kernel-class launches.

This is the HIP analogue of the reference renderer's output: the
``CellAllocations`` of MemoryAllocation.swift and the ``[CompiledKernel]``
list of Renderer.swift:134-143, each op carrying its dispatch description
(Renderer.swift:26-67 ``DispatchMode``) for profiling output.
"""
from __future__ import annotations

from dataclasses import dataclass, field

ALIGN = 64  # floats: every cell starts on a 256-byte boundary


@dataclass
class Cell:
    name: str
    off: int
    n: int


@dataclass
class Op:
    kernel: int
    arg: list
    farg: list = field(default_factory=list)
    flags: int = 0
    label: str = ""
    dispatch: str = ""
    bytes: float = 0.0   # algorithmic HBM bytes per launch (interface read once + written once)
    flops: float = 0.0   # algorithmic flops per launch
    bound: str = "hbm"   # roof that bounds the op: "hbm", "mfma" (fp32 matrix), "mfma_x6" (split-bf16
                         # products on the bf16 matrix cores) or "valu" (fp32 vector)


@dataclass
class Program:
    cells: dict = field(default_factory=dict)
    ops: list = field(default_factory=list)
    size: int = 0
    max_frames: int = 0
    output_cell: str = ""
    meta: dict = field(default_factory=dict)
    # generic UOp blocks (dgen_hip.uop.Block) the DGEN_HIP_K_UOP_BLOCK ops index
    blocks: list = field(default_factory=list)

    def alloc(self, name: str, n: int) -> int:
        if name in self.cells:
            raise ValueError(f"cell {name} allocated twice")
        n = int(n)
        if n <= 0:
            raise ValueError(f"cell {name}: size {n}")
        off = (self.size + ALIGN - 1) // ALIGN * ALIGN
        self.cells[name] = Cell(name, off, n)
        self.size = off + n
        return off

    def off(self, name: str) -> int:
        return self.cells[name].off

    def add(self, kernel: int, arg, farg=(), flags: int = 0, label: str = "", dispatch: str = "",
            bytes: float = 0.0, flops: float = 0.0, bound: str = "hbm") -> int:
        arg = [int(a) for a in arg]
        farg = [float(a) for a in farg]
        if len(arg) > 32 or len(farg) > 8:
            raise ValueError("too many op arguments")
        if bound not in ("hbm", "mfma", "mfma_x6", "valu"):
            raise ValueError(f"unknown bound {bound}")
        self.ops.append(Op(kernel, arg + [0] * (32 - len(arg)), farg + [0.0] * (8 - len(farg)), flags, label,
                           dispatch, float(bytes), float(flops), bound))
        return len(self.ops) - 1

    def find(self, label: str) -> int:
        for i, op in enumerate(self.ops):
            if op.label == label:
                return i
        raise KeyError(label)
