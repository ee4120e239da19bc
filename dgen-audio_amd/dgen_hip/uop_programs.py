"""Schedules built from generic UOp blocks (dgen_hip.uop): DGen graphs in
the form the reference compiler hands a renderer, i.e. blocks of UOps with a
dispatch mode, frame order and temporality, lowered here op by op as the
reference's emitters write them.  No kernel class is pattern-matched: every
block goes through the library's generic renderer (hiprtc).

- ``oscbank_uop_program``: config 1 (``Signal.phasor(Tensor)`` bank -> sin
  -> * amps -> sum -> ``history`` one-pole), optionally with a tanh
  waveshaper on the output: a graph that differs from the config-1 kernel
  class in one elementwise block.
- ``hop_uop_program``: an accum hop counter in a sequential block and a
  hop-gated block that runs only where the counter is 0 (Temporality
  .hopBased).
- ``noise_uop_program``: ``Signal.noise()``'s xorshift32 cell.
- ``expr_uop_program``: a frame-parallel block exercising the arithmetic,
  comparison, logic, selection and math UOps.
- ``table_uop_program``: a static block (run once at configure) filling a
  table cell, read by a frame block through a static global.
"""
from __future__ import annotations

import numpy as np

from . import runtime as R
from .program import Program
from .uop import FRAME_COUNT, Block, BlockBuilder, const, glob
from .workloads import OscBankConfig

TWO_PI_F32 = float(np.float32(2.0 * np.pi))  # the graphs' 2pi constant


def _block_op(p: Program, index: int, tape: int = -1, slots: int = 0, out: int = -1, nout: int = 0,
              inp: int = -1, nin: int = 0, frames: int | None = None, sr: float = 44100.0, flags: int = 0,
              label: str = "", dispatch: str = "", bytes: float = 0.0, flops: float = 0.0):
    return p.add(R.K_UOP_BLOCK, [index, tape, slots, out, nout, inp, nin, frames or p.max_frames], [sr], flags=flags,
                 label=label or f"uop_block_{index}", dispatch=dispatch, bytes=bytes, flops=flops, bound="valu")


def oscbank_uop_program(cfg: OscBankConfig, drive: float | None = None) -> Program:
    """Config 1 as two generic blocks.

    Block 0 (perFrame, parallel): the deterministic phasor of every
    oscillator, (f / sr) * n - floor(...) (Emit+State.swift:370-387), times
    2pi, sin, times its amplitude, summed in oscillator order over a
    parallel range (the tensor's element loop); the frame's sum goes to tape
    slot 0.  Block 1 (singleThreaded, sequential): the history one-pole y =
    x + pole * y[n-1] (historyRead / historyWrite, Emit+State.swift:150-224)
    and the output; with ``drive`` the output is tanh(drive * y) (the
    history keeps y)."""
    T, n = cfg.frames, cfg.n_osc
    p = Program(max_frames=T)
    freqs = p.alloc("freqs", n)
    amps = p.alloc("amps", n)
    hist = p.alloc("history", 1)
    tape = p.alloc("tape", T)
    out = p.alloc("out", T)

    a = Block(dispatch="perFrame", frame_order="parallel")
    b = BlockBuilder(a)
    fi = b.frameIndex()
    sr = b.hostSampleRate()
    acc = b.declareVar(0.0)
    k = b.beginParallelRange(imm=(n, 0))
    f = b.memoryRead(k, imm=(freqs, 0))
    inc = b.div(f, sr)
    raw = b.mul(inc, fi)
    ph = b.sub(raw, b.floor(raw))
    s = b.sin(b.mul(ph, TWO_PI_F32))
    acc2 = b.add(acc, b.mul(s, b.memoryRead(k, imm=(amps, 0))))
    b.stmt("mutate", acc, acc2)
    b.stmt("endParallelRange")
    b.identity(acc, value=glob(0))

    c = Block(dispatch="singleThreaded", frame_order="sequential")
    b = BlockBuilder(c, first_var=100)
    h = b.load(imm=(hist, 0))
    y = b.add(glob(0), b.mul(h, cfg.pole))
    b.stmt("store", y, imm=(hist, 0))
    if drive is not None:
        y = b.tanh(b.mul(y, float(drive)))
    b.stmt("output", y, imm=(0, 0))

    p.blocks = [a, c]
    _block_op(p, 0, tape, 1, sr=cfg.sr, label="phasor_bank_sum", dispatch=f"perFrame({T})",
              bytes=4.0 * T, flops=float(T) * 30.0 * n)
    _block_op(p, 1, tape, 1, out, 1, sr=cfg.sr, label="history_out", dispatch="singleThreaded",
              bytes=8.0 * T, flops=2.0 * T)
    p.output_cell = "out"
    p.meta.update(cfg=cfg, drive=drive)
    return p


def hop_uop_program(T: int, hop: int) -> Program:
    """A hop counter and a hop-gated block (Temporality .hopBased).

    Block 0 (singleThreaded): accum(1, reset 0, min 0, max hop) on a cell,
    its pre-increment value to tape slot 1 (u_accum, Definitions.swift:
    215-246: out = state; next = state + 1, wrapped by subtracting the span at
    max).  Block 1 (perFrame, hop-based on that counter): for the frames where
    the counter is 0, dec[n / hop] = x[n] and a hop count accumulates in a
    cell through memoryAccumulate."""
    p = Program(max_frames=T)
    x = p.alloc("x", T)
    cnt = p.alloc("counter", 1)
    dec = p.alloc("decimated", (T + hop - 1) // hop)
    hits = p.alloc("hits", 1)
    tape = p.alloc("tape", 2 * T)

    a = Block(dispatch="singleThreaded", frame_order="sequential")
    b = BlockBuilder(a)
    s = b.load(imm=(cnt, 0))
    b.identity(s, value=glob(1))
    n1 = b.add(s, 1.0)
    wrap = b.gte(n1, float(hop))
    n2 = b.gswitch(wrap, b.sub(n1, float(hop)), n1)
    b.stmt("store", n2, imm=(cnt, 0))

    c = Block(dispatch="perFrame", frame_order="parallel", temporality="hop", hop_size=hop, hop_counter=glob(1))
    b = BlockBuilder(c, first_var=100)
    fi = b.frameIndex(int_typed=True)
    q = b.div(fi, hop, int_typed=True)
    v = b.memoryRead(fi, imm=(x, 0))
    b.stmt("memoryWrite", q, v, imm=(dec, 0))
    b.stmt("memoryAccumulate", 0.0, 1.0, imm=(hits, 0))

    p.blocks = [a, c]
    _block_op(p, 0, tape, 2, label="hop_counter", dispatch="singleThreaded")
    _block_op(p, 1, tape, 2, label="hop_gated", dispatch=f"perFrame({T}) hop {hop}")
    p.meta.update(hop=hop)
    return p


def noise_uop_program(T: int) -> Program:
    """Signal.noise(): the xorshift32 stream of one cell (one sequential
    block), to output channel 0."""
    p = Program(max_frames=T)
    st = p.alloc("noise_state", 1)
    out = p.alloc("out", T)
    a = Block(dispatch="singleThreaded", frame_order="sequential")
    b = BlockBuilder(a)
    b.stmt("output", b.noise(imm=(st, 0)), imm=(0, 0))
    p.blocks = [a]
    _block_op(p, 0, out=out, nout=1, label="noise", dispatch="singleThreaded")
    p.output_cell = "out"
    return p


def expr_uop_program(T: int) -> Program:
    """One frame-parallel block over the input channel x and the frame index
    n, writing eight output channels:
      0: (x * 3 - 1) / 2 + n mod 5 (float mod)    1: |x|^1.5 + sqrt(|x|)
      2: sign(x) * atan2(x, 0.5) + tanh(x)         3: exp(-x^2) + log10(1 + |x|)
      4: x > 0 and n mod 3 < 1 ? floor(4x) : ceil(4x)  (and/or/xor as 0/1)
      5: selector(n mod 4, [x, 2x, 3x])             6: min(max(x, -0.5), 0.5) + round(3x)
      7: (int)(n / 7) * 7 + n % 7 - n  (integer ops; 0)"""
    p = Program(max_frames=T)
    x = p.alloc("x", T)
    out = p.alloc("out", 8 * T)
    a = Block(dispatch="perFrame", frame_order="parallel")
    b = BlockBuilder(a)
    xv = b.input(imm=(0, 0))
    n = b.frameIndex()
    ni = b.frameIndex(int_typed=True)
    o0 = b.add(b.div(b.sub(b.mul(xv, 3.0), 1.0), 2.0), b.mod(n, 5.0))
    ax = b.abs(xv)
    o1 = b.add(b.pow(ax, 1.5), b.sqrt(ax))
    o2 = b.add(b.mul(b.sign(xv), b.atan2(xv, 0.5)), b.tanh(xv))
    o3 = b.add(b.exp(b.sub(0.0, b.mul(xv, xv))), b.log10(b.add(1.0, ax)))
    c1 = b.gt(xv, 0.0)
    c2 = b.lt(b.mod(n, 3.0), 1.0)
    both = b.op("and", c1, c2)
    either = b.op("or", c1, c2)
    one = b.op("xor", both, either)  # exactly one of the two
    o4 = b.add(b.gswitch(both, b.floor(b.mul(xv, 4.0)), b.ceil(b.mul(xv, 4.0))), b.mul(one, 100.0))
    sel = b.add(b.mod(n, 4.0), 0.0)
    o5 = b.selector(sel, options=(xv, b.mul(xv, 2.0), b.mul(xv, 3.0)))
    o6 = b.add(b.min(b.max(xv, -0.5), 0.5), b.round(b.mul(xv, 3.0)))
    q = b.div(ni, 7, int_typed=True)
    r = b.mod(ni, 7, int_typed=True)
    o7 = b.sub(b.add(b.mul(q, 7, int_typed=True), r, int_typed=True), ni, int_typed=True)
    o7f = b.cast(o7, imm=(0, 0))
    for ch, v in enumerate((o0, o1, o2, o3, o4, o5, o6, o7f)):
        b.stmt("output", v, imm=(ch, 0))
    p.blocks = [a]
    _block_op(p, 0, out=out, nout=8, inp=x, nin=1, label="expr", dispatch=f"perFrame({T})")
    p.meta.update(x=x)
    return p


def expr_reference(x: np.ndarray) -> np.ndarray:
    """numpy evaluation of expr_uop_program's eight channels (float64)."""
    x = x.astype(np.float64)
    n = np.arange(len(x), dtype=np.float64)
    ax = np.abs(x)
    o = np.zeros((8, len(x)))
    o[0] = (x * 3 - 1) / 2 + np.fmod(n, 5)
    o[1] = ax ** 1.5 + np.sqrt(ax)
    o[2] = np.sign(x) * np.arctan2(x, 0.5) + np.tanh(x)
    o[3] = np.exp(-x * x) + np.log10(1 + ax)
    c1 = x > 0
    c2 = np.fmod(n, 3) < 1
    both, either = c1 & c2, c1 | c2
    o[4] = np.where(both, np.floor(4 * x), np.ceil(4 * x)) + 100.0 * (both != either)
    m = np.fmod(n, 4)
    o[5] = np.select([m <= 0, m <= 1, m <= 2, m <= 3], [0 * x, x, 2 * x, 3 * x], 0.0)
    # round half away from zero (roundf)
    r3 = np.sign(3 * x) * np.floor(np.abs(3 * x) + 0.5)
    o[6] = np.clip(x, -0.5, 0.5) + r3
    o[7] = 0.0
    return o


def table_uop_program(T: int, N: int) -> Program:
    """A static block (staticThreads(N), run once when the schedule is
    configured) writing table[i] = sin(2 pi i / N) * scale, with the scale a
    static global (tape slot 0, frame 0); a frame block reads the table at
    n mod N and writes it to output channel 0."""
    p = Program(max_frames=T)
    tab = p.alloc("table", N)
    tape = p.alloc("tape", T)
    out = p.alloc("out", T)
    s = Block(dispatch="staticThreads", n=N, frame_order="parallel", temporality="static")
    b = BlockBuilder(s)
    b.stmt("defineGlobal", glob(0))
    b.identity(0.5, value=glob(0))
    i = b.threadIndex(int_typed=True)
    ang = b.div(b.mul(b.cast(i, imm=(0, 0)), TWO_PI_F32), float(N))
    b.stmt("memoryWrite", i, b.mul(b.sin(ang), glob(0)), imm=(tab, 0))
    f = Block(dispatch="perFrame", frame_order="parallel")
    b = BlockBuilder(f, first_var=100)
    ni = b.frameIndex(int_typed=True)
    j = b.mod(ni, N, int_typed=True)
    b.stmt("output", b.memoryRead(j, imm=(tab, 0)), imm=(0, 0))
    p.blocks = [s, f]
    _block_op(p, 0, tape, 1, flags=R.OP_STATIC, label="table", dispatch=f"staticThreads({N})")
    _block_op(p, 1, tape, 1, out, 1, label="table_read", dispatch=f"perFrame({T})")
    p.output_cell = "out"
    return p


def frame_count_uop_block(p: Program, out_cell: int) -> None:
    """Append a block writing the run's frame count to a cell (the frameCount
    UOp; used to check that generic blocks run the run's frame count)."""
    blk = Block(dispatch="singleThreaded", frame_order="sequential")
    b = BlockBuilder(blk, first_var=500)
    b.stmt("store", b.identity(FRAME_COUNT), imm=(out_cell, 0))
    p.blocks.append(blk)
    _block_op(p, len(p.blocks) - 1, label="frame_count")


__all__ = ["oscbank_uop_program", "hop_uop_program", "noise_uop_program", "expr_uop_program", "expr_reference",
           "table_uop_program", "frame_count_uop_block", "const"]


def append_lane_shaper(p: Program, src: str, dst: str, lanes: int, frames: int, drive: float) -> None:
    """Append one generic block to a schedule: dst[b][n] = tanh(drive *
    src[b][n]) over a [lanes][frames] cell, as the compiler would emit an
    elementwise tanh on a [B] SignalTensor (perFrameScaled(B), one thread per
    (frame, lane): frame = thread / B, lane = thread mod B).  A graph that
    differs from a kernel-class schedule in one elementwise block."""
    s, d = p.off(src), p.off(dst)
    blk = Block(dispatch="perFrameScaled", n=lanes, frame_order="parallel")
    b = BlockBuilder(blk)
    tid = b.threadIndex(int_typed=True)
    f = b.div(tid, lanes, int_typed=True)
    lane = b.mod(tid, lanes, int_typed=True)
    idx = b.add(b.mul(lane, frames, int_typed=True), f, int_typed=True)
    v = b.memoryRead(idx, imm=(s, 0))
    b.stmt("memoryWrite", idx, b.tanh(b.mul(v, float(drive))), imm=(d, 0))
    p.blocks.append(blk)
    _block_op(p, len(p.blocks) - 1, frames=frames, label="lane_shaper", dispatch=f"perFrameScaled({lanes})",
              bytes=8.0 * lanes * frames, flops=20.0 * lanes * frames)
