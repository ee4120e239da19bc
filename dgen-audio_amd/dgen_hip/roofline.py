"""Roofline of a schedule: per-op algorithmic bytes and flops against the
MI355X peaks.

For each op k (one schedule entry, possibly several launches):

    T_roof,k = max(bytes_k / HBM, flops_k / P_k)

with P_k the fp32 matrix (MFMA) peak for fp32-product GEMMs, the bf16
matrix peak over six for split-bf16 GEMMs (six bf16 partial products per
fp32 product: ``flops_k`` counts fp32-product flops), and the fp32 vector
peak for VALU-bound ops.  ``bytes_k`` counts the op's interface traffic: every input
read once and every output written once, in fp32, with window overlap and
row reuse assumed served on chip.  The step fraction is
sum_k T_roof,k / sum_k T_meas,k.
"""
from __future__ import annotations

from dataclasses import dataclass

HBM_BYTES_PER_S = 8.0e12        # MI355X HBM3E
MFMA_FP32_FLOPS = 157.3e12      # dense fp32 matrix
MFMA_BF16_FLOPS = 2.5e15        # dense bf16 matrix
SPLIT_BF16_FLOPS = MFMA_BF16_FLOPS / 6  # fp32 products as six bf16 partial products
VALU_FP32_FLOPS = 157.3e12      # fp32 vector

PEAK = {"hbm": HBM_BYTES_PER_S, "mfma": MFMA_FP32_FLOPS, "mfma_x6": SPLIT_BF16_FLOPS, "valu": VALU_FP32_FLOPS}


def roof_seconds(op) -> float:
    """Roofline time of one op: the larger of its HBM and compute times."""
    t_mem = op.bytes / HBM_BYTES_PER_S
    t_cmp = op.flops / PEAK["valu" if op.bound == "hbm" else op.bound]
    return max(t_mem, t_cmp)


@dataclass
class OpRoof:
    index: int
    label: str
    bound: str
    bytes: float
    flops: float
    roof_ms: float
    meas_ms: float

    @property
    def frac(self) -> float:
        return self.roof_ms / self.meas_ms if self.meas_ms > 0 else 0.0

    def achieved(self) -> tuple[float, float, str]:
        """(achieved, peak, unit) against the op's own bound."""
        s = self.meas_ms * 1e-3
        if self.bound == "hbm":
            return self.bytes / s / 1e9, HBM_BYTES_PER_S / 1e9, "GB/s"
        return self.flops / s / 1e12, PEAK[self.bound] / 1e12, "TFLOP/s"


def table(program, timings) -> list[OpRoof]:
    """Join a program's cost model with measured per-op times (ms)."""
    out = []
    for t in timings:
        op = program.ops[t.index]
        out.append(OpRoof(t.index, op.label, op.bound, op.bytes, op.flops, roof_seconds(op) * 1e3, t.gpu_ms))
    return out


def step_roof_ms(program) -> float:
    """Sum of roofline times of every per-run op of the program."""
    from .runtime import OP_STATIC
    return sum(roof_seconds(op) for op in program.ops if not op.flags & OP_STATIC) * 1e3
