"""Static tables on the GPU: the row schedule of a sampleRow read
(DGEN_HIP_K_ROW_SCHEDULE, built in parallel over segments and rows) against
a sequential restatement of Emit+RowSelection.swift:164-197, bit for bit,
for config 3's playhead, a control hop of 256, a wrapping playhead, and
playheads that overflow a segment's slots, a row's entries or are not
finite; the synth backward's run table (DGEN_HIP_K_RUN_TABLE) against a
restatement from the same segment rows and row lists; the xorshift32 noise table (built by bit-matrix jump-ahead) and the
playhead accumulator against the oracle's sequential streams.  Needs a GPU."""
import math

import numpy as np
import pytest

import oracle as O
from dgen_hip import runtime as R
from dgen_hip.program import Program

pytestmark = pytest.mark.gpu

SEG, SLOTS, ENTRIES = 64, 4, 16
RUN_SEGS, RUN_PARTS = 4, 6


def schedule_ref(play, rows, frames):
    """The sequential row schedule (one pass over segments and frames)."""
    nseg = (frames + SEG - 1) // SEG
    lerp = np.zeros((frames, 8), np.float32)
    seg_rows = np.full((nseg, SLOTS), -1.0, np.float32)
    row_list = np.full((rows, ENTRIES), -1.0, np.float32)
    status = 0.0
    nr = np.float32(rows)
    for s in range(nseg):
        srow = []
        for t in range(s * SEG, min(frames, (s + 1) * SEG)):
            w = np.fmod(np.float32(play[t]), nr)
            if w < 0:
                w = np.float32(w + nr)
            fl = np.float32(math.floor(w)) if np.isfinite(w) else np.float32(np.nan)
            if not (fl >= 0 and fl < nr):
                fl, w, status = np.float32(0), np.float32(0), max(status, 3.0)
            ce = np.float32(fl + np.float32(1))
            if ce >= nr:
                ce = np.float32(0)
            frac = np.float32(w - fl)
            slots = []
            for r in (int(fl), int(ce)):
                if r in srow:
                    slots.append(srow.index(r))
                elif len(srow) < SLOTS:
                    srow.append(r)
                    slots.append(len(srow) - 1)
                else:
                    status = max(status, 1.0)
                    slots.append(0)
            lerp[t] = (fl, ce, frac, np.float32(np.float32(1) - frac), slots[0], slots[1], 0, 0)
        for j, r in enumerate(srow):
            seg_rows[s, j] = r
            q = int(np.sum(row_list[r] >= 0))
            if q < ENTRIES:
                row_list[r, q] = s * SLOTS + j
            else:
                status = max(status, 2.0)
    return lerp, seg_rows, row_list, status


def run_table_ref(seg_rows, row_list, nseg):
    """Per run of RUN_SEGS segments: [0] = (rows, 0, 0, 0), then per control
    row its segments touch, in order of the row's first in-run entry,
    (row, before | outside << 8 | n << 16, entries lo, hi) with the run's n
    entries of the row packed 4 bits each as (segment - s0) * 4 + slot."""
    nruns = (nseg + RUN_SEGS - 1) // RUN_SEGS
    tab = np.zeros((nruns, RUN_SEGS * SLOTS + 1, 4), np.uint32)
    for run in range(nruns):
        s0, s1 = run * RUN_SEGS, min(run * RUN_SEGS + RUN_SEGS, nseg)
        out = []
        for q in range((s1 - s0) * SLOTS):
            sq, j = s0 + q // SLOTS, q % SLOTS
            if seg_rows[sq, j] < 0:
                continue
            r = int(seg_rows[sq, j])
            first, before, prev, outside, ents = -1, 0, -1, False, []
            for e in row_list[r]:
                if e < 0:
                    break
                en = int(e)
                rr = en // SLOTS // RUN_SEGS
                if rr == run:
                    first = en if first < 0 else first
                    ents.append(en - s0 * SLOTS)
                else:
                    outside = True
                    if first < 0 and rr != prev:
                        before += 1
                prev = rr
            if first == sq * SLOTS + j:
                packed = sum(v << (4 * i) for i, v in enumerate(ents))
                out.append((r, before | int(outside) << 8 | len(ents) << 16, packed & 0xFFFFFFFF, packed >> 32))
        tab[run, 0, 0] = len(out)
        for i, e in enumerate(out):
            tab[run, 1 + i] = e
    return tab


def run_schedule(play, rows, frames):
    nseg = (frames + SEG - 1) // SEG
    nruns = (nseg + RUN_SEGS - 1) // RUN_SEGS
    p = Program(max_frames=frames)
    pc = p.alloc("play", frames)
    lerp = p.alloc("lerp", frames * 8)
    segr = p.alloc("seg_rows", nseg * SLOTS)
    rowl = p.alloc("row_list", rows * ENTRIES)
    flag = p.alloc("flag", 1)
    ws = p.alloc("ws", nseg + rows)
    tab = p.alloc("run_table", nruns * (RUN_SEGS * SLOTS + 1) * 4)
    p.add(R.K_ROW_SCHEDULE, [pc, lerp, segr, rowl, flag, rows, frames, SEG, ws], label="row_schedule")
    p.add(R.K_RUN_TABLE, [segr, rowl, tab, nseg, rows], label="run_table")
    with R.HIPLazyRuntime(p, 0) as rt:
        rt.write("play", np.asarray(play, np.float32))
        rt.runNoCopy()
        return (rt.read("lerp").reshape(frames, 8), rt.read("seg_rows").reshape(nseg, SLOTS),
                rt.read("row_list").reshape(rows, ENTRIES), float(rt.read("flag")[0]),
                rt.read("run_table").view(np.uint32).reshape(nruns, RUN_SEGS * SLOTS + 1, 4))


CASES = {
    "config 3": (lambda: O.playhead(1000, 64000), 1000, 64000),
    "control hop 256": (lambda: O.playhead(64, 16384), 64, 16384),
    # negative positions (fmod + rows) and positions past the last row (wrap to 0)
    # (the jump between the two ramps falls on a segment boundary, frame 2496)
    "wrapping": (lambda: np.where(np.arange(5000) < 2496, -40 + np.float32(0.03) * np.arange(5000),
                                  250 + np.float32(0.03) * (np.arange(5000) - 2496)).astype(np.float32), 300, 5000),
    "slot overflow": (lambda: (np.arange(3000, dtype=np.float32) * np.float32(0.2)).astype(np.float32), 500, 3000),
    "entry overflow": (lambda: np.full(4000, 7.5, np.float32), 20, 4000),
    "non-finite": (lambda: np.where(np.arange(2000) == 777, np.nan, np.arange(2000) / 100.0).astype(np.float32),
                   40, 2000),
}


@pytest.mark.parametrize("name", list(CASES))
def test_row_schedule_matches_the_sequential_schedule(gpu, name):
    make, rows, frames = CASES[name]
    play = make()
    print(f"row schedule: {name} rows={rows} frames={frames}", flush=True)
    got = run_schedule(play, rows, frames)
    ref = schedule_ref(play, rows, frames)
    for g, r, what in zip(got[:3], ref[:3], ("lerp", "segment rows", "row lists")):
        np.testing.assert_array_equal(g, r, err_msg=what)
    assert got[3] == ref[3], (got[3], ref[3])
    expect = {"slot overflow": 1.0, "entry overflow": 2.0, "non-finite": 3.0}.get(name, 0.0)
    assert got[3] == expect
    # the run table from the GPU's segment rows and row lists (rows past a
    # run's count are not read)
    tab, tref = got[4], run_table_ref(got[1], got[2], got[1].shape[0])
    for run in range(tab.shape[0]):
        n = int(tref[run, 0, 0])
        np.testing.assert_array_equal(tab[run, :1 + n], tref[run, :1 + n], err_msg=f"run {run}")
    if expect == 0.0:
        # a valid schedule's rows meet at most RUN_PARTS runs
        before = tref[:, 1:, 1] & 255
        assert before.max() < RUN_PARTS


@pytest.mark.parametrize("frames", [1, 255, 256, 257, 64000, 100003])
def test_noise_and_playhead_tables_match_the_sequential_streams(gpu, frames):
    p = Program(max_frames=frames)
    nz = p.alloc("noise", frames)
    ph = p.alloc("play", frames)
    F = 1000
    fmaxi = np.float32(F - 1)
    step = fmaxi / np.float32(max(1, frames - 1))
    hi = np.float32(fmaxi - np.float32(1e-4))
    p.add(R.K_NOISE_TABLE, [nz, frames], flags=R.OP_STATIC, label="noise")
    p.add(R.K_ACCUM_TABLE, [ph, frames], [step, 0.0, fmaxi, 0.0, hi], flags=R.OP_STATIC, label="playhead")
    with R.HIPLazyRuntime(p, 0) as rt:
        noise, play = rt.read("noise"), rt.read("play")
    np.testing.assert_array_equal(noise, O.noise_stream(frames))
    np.testing.assert_array_equal(play, O.playhead(F, frames))
