"""Schedules for the benchmark workloads, as the HIP renderer lowers them.

Each builder returns a :class:`Program` whose ops follow the block order the
reference compiler produces for the same DGenLazy graph (forward blocks, then
the gradient blocks of ``loss.backward``, then the optimiser), with the
blocks pattern-matched to hand-written kernel classes.
"""
from __future__ import annotations

import numpy as np

from . import runtime as R
from .program import Program
from .workloads import (BiquadConfig, HarmonicConfig, MembraneConfig, OscBankConfig, StftConfig, SvfConfig,
                        SweptPhasorConfig)

SEG = 64          # frames per synth segment (checkpoint spacing)
SLOTS = 4         # control rows a segment may touch
ROW_ENTRIES = 16  # (segment, slot) entries per control row (kRowEntries)
RUN_SEGS = 4      # segments per synth-backward workgroup (kRunSegs)
RUN_PARTS = 6     # boundary partials a control row holds (kRunParts)
MAX_HARMONICS = 256  # the synth kernels' harmonic groups (four of 64)
MAX_CONTROLS = 512   # control columns K + 2 + NF
SPLITK_ROWS = 1024  # rows per split of the weight-gradient GEMMs
GEMM_TILE_M = 128  # output rows per GEMM workgroup tile (k_gemm.hip BM)
SPLITK_ROWS_HEADS = 256  # the heads' weight gradient has one 128-wide column tile: split finer to fill the chip
MSS_TILE = 4096     # output samples per spectral-loss workgroup
BQ_CHUNK = 512      # frames per biquad scan chunk (512 measured fastest of 128..1024)
SVF_CHUNK = 256     # frames per SVF scan chunk
STFT_TILE = 8192    # output samples per STFT forward workgroup
MEM_STEPS = 16      # membrane frames per time-blocked launch
MEM_TILE = 32       # membrane cells per workgroup tile side
MEM_WAVES = 16      # membrane waves per workgroup (4-row strips of a 64-row region)


GEMM_PRODUCTS = {"fp32": 0, "split-bf16": 1}  # DGEN_HIP_K_GEMM arg[20]


def _gemm_args(mode: int, args: list, b_planes: int = -1) -> list:
    """DGEN_HIP_K_GEMM arguments with the product mode at [20] and B's
    split-bf16 planes at [21] (column weights [18..19] default to none)."""
    a = list(args)
    if len(a) == 18:
        a += [-1, 0]
    if len(a) != 20:
        raise ValueError(f"gemm op with {len(a)} arguments")
    return a + [mode, b_planes if mode == 1 else -1]


def _split_planes(p: Program, name: str, src: int, K: int, N: int, ldk: int, ldn: int, k_pad: int = 0) -> int:
    """A DGEN_HIP_K_SPLIT_BF16 op of the [K][N] view (k, n) -> src[k*ldk + n*ldn]
    into a new planes cell (zero for K <= k < k_pad); returns the cell."""
    k8 = (max(K, k_pad) + 7) // 8
    cell = p.alloc(name, 3 * k8 * N * 4)
    p.add(R.K_SPLIT_BF16, [src, cell, K, N, ldk, ldn, k8], label=name, dispatch="perElement",
          bytes=K * N * 4.0 + 3 * k8 * N * 16.0, flops=6.0 * K * N)
    return cell


def _f32(x) -> float:
    return float(np.float32(x))


# ------------------------------------------------------------------ config 1
def oscbank_program(cfg: OscBankConfig) -> Program:
    """Signal.phasor(Tensor) bank -> sin -> *amps -> sum -> history one-pole."""
    p = Program(max_frames=cfg.frames)
    freqs = p.alloc("freqs", cfg.n_osc)
    amps = p.alloc("amps", cfg.n_osc)
    out = p.alloc("out", cfg.frames)
    tiles = (cfg.frames + 255) // 256
    ws = p.alloc("workspace", cfg.frames + 1 + 3 * tiles)
    # per output sample: n_osc x (divide-free phase 4 + sin ~20 + mul-add 2) + the one-pole 2
    p.add(R.K_OSC_BANK, [freqs, amps, out, cfg.n_osc, cfg.frames, ws], [cfg.sr, cfg.pole], label="osc_bank",
          dispatch=f"perFrame({cfg.frames}) + tile scan", bytes=4.0 * cfg.frames + 8.0 * cfg.n_osc,
          flops=float(cfg.frames) * (26.0 * cfg.n_osc + 2.0), bound="valu")
    p.output_cell = "out"
    return p


def stream_oscbank_program(cfg: OscBankConfig, stateful: bool = True, max_frames: int | None = None) -> Program:
    """The config-1 graph as a streaming process (dgen_process_v1 with
    preserved state): per call, frames [0, frame_count) of `out`; the
    oscillator phases (stateful) and the one-pole's y[n-1] carry over."""
    T = int(max_frames or cfg.frames)
    p = Program(max_frames=T)
    # the graph's memory first (what the reference keeps in the host's state
    # block), then the output channel's staging cell
    freqs = p.alloc("freqs", cfg.n_osc)
    amps = p.alloc("amps", cfg.n_osc)
    st = p.alloc("state", cfg.n_osc + 1)
    memory = p.size
    out = p.alloc("out", T)
    p.add(R.K_STREAM_OSC_BANK, [freqs, amps, out, cfg.n_osc, T, st, 1 if stateful else 0], [cfg.sr, cfg.pole],
          label="stream_osc_bank", dispatch="singleThreaded frame loop (one wave)", bytes=4.0 * T,
          flops=float(T) * (26.0 * cfg.n_osc + 2.0), bound="valu")
    p.output_cell = "out"
    p.meta.update(cfg=cfg, stateful=stateful, ports=([], [("out", 0, 1)]), memory=(0, memory))
    return p


# ------------------------------------------------------------------ config 3
def harmonic_program(cfg: HarmonicConfig, train: bool = True, optimizer: bool = True,
                     side_stream: bool = True, chain_timer: bool = False) -> Program:
    """Batched harmonic + noise synth with MLP decoder and MSS loss.

    ``train=False`` builds the forward render only (controls -> audio), used
    to render targets.  With ``train=True`` the schedule is forward, loss,
    backward to every parameter and (``optimizer``) one Adam step.  With
    ``side_stream`` the phase-carry chain (which depends only on f0) runs on a
    second stream, overlapping the control-network forward, and the weight
    and bias gradients of the backward overlap its data-gradient chain.
    ``chain_timer`` runs the phase chain's timed build, which fills the cell
    ``chain_timer`` ([G][B][8] uint64 records; see ``chain_timer.py``)."""
    SIDE = R.OP_SIDE if side_stream else 0
    JOIN = R.OP_JOIN if side_stream else 0
    FORK = R.OP_FORK if side_stream else 0
    B, T, F, K, NF, NC, M = cfg.B, cfg.T, cfg.F, cfg.K, cfg.NF, cfg.NC, cfg.M
    Hd, din, Lyr = cfg.hidden, cfg.din, cfg.layers
    if cfg.gemm_products not in GEMM_PRODUCTS:
        raise ValueError(f"gemm_products {cfg.gemm_products!r}: one of {sorted(GEMM_PRODUCTS)}")
    gm = GEMM_PRODUCTS[cfg.gemm_products]
    if K > MAX_HARMONICS:
        raise ValueError(f"K = {K} harmonics exceeds {MAX_HARMONICS}")
    if NC > MAX_CONTROLS:
        raise ValueError(f"K + 2 + NF = {NC} exceeds {MAX_CONTROLS}")
    LDC = cfg.ldc
    nseg = (T + SEG - 1) // SEG
    p = Program(max_frames=T)
    p.meta.update(cfg=cfg, nseg=nseg, train=train)

    # ---- data, parameters, optimiser state
    X = p.alloc("X", M * din)
    f0 = p.alloc("f0", F * B)
    uv = p.alloc("uv", F * B)
    npar = cfg.param_count()
    P = p.alloc("params", npar)
    woff, off = [], 0
    fan = din
    for _ in range(Lyr):
        woff.append((P + off, P + off + fan * Hd))
        off += fan * Hd + Hd
        fan = Hd
    Wh, bh = P + off, P + off + Hd * NC
    p.meta["param_offsets"] = [(w - P, b - P) for w, b in woff] + [(Wh - P, bh - P)]

    # ---- static tables
    play = p.alloc("playhead", T)
    lerp = p.alloc("lerp", T * 8)
    segrows = p.alloc("seg_rows", nseg * SLOTS)
    rowlist = p.alloc("row_list", F * ROW_ENTRIES)
    flag = p.alloc("row_flag", 1)
    noise = p.alloc("noise", T)
    fmaxi = np.float32(max(0, F - 1))
    step = fmaxi / np.float32(max(1, T - 1))
    hi = np.float32(max(np.float32(0.0), fmaxi - np.float32(1e-4)))
    p.add(R.K_ACCUM_TABLE, [play, T], [step, 0.0, fmaxi if F > 1 else 1.0, 0.0, hi], flags=R.OP_STATIC,
          label="playhead", dispatch="static singleThreaded")
    p.add(R.K_NOISE_TABLE, [noise, T], flags=R.OP_STATIC, label="noise", dispatch="static singleThreaded")
    rs_ws = p.alloc("row_schedule_ws", nseg + F)
    p.add(R.K_ROW_SCHEDULE, [play, lerp, segrows, rowlist, flag, F, T, SEG, rs_ws], flags=R.OP_STATIC,
          label="row_schedule", dispatch="static singleThreaded")
    # the synth backward's runs of RUN_SEGS segments: each run's control rows
    nruns = (nseg + RUN_SEGS - 1) // RUN_SEGS
    runtab = p.alloc("run_table", nruns * (RUN_SEGS * SLOTS + 1) * 4)
    p.add(R.K_RUN_TABLE, [segrows, rowlist, runtab, nseg, F], flags=R.OP_STATIC, label="run_table",
          dispatch="static perRun")

    # ---- activations
    Hs = [p.alloc(f"H{l + 1}", M * Hd) for l in range(Lyr)]
    Z = p.alloc("Z", M * LDC)
    ctrl = p.alloc("ctrl", M * LDC)
    ck = p.alloc("checkpoints", nseg * B * K)
    f0f = p.alloc("f0_frames", B * T)
    uvf = p.alloc("uv_frames", B * T)
    y = p.alloc("y", B * T)

    # ---- forward
    f4 = 4.0
    ctrl_b = M * NC * f4                      # one pass over the control rows
    lerp_b = T * 8 * f4
    ck_b = nseg * B * K * f4
    data_b = 2 * B * T * f4 + T * f4 + nseg * SLOTS * f4  # f0 and uv frames, noise, segment rows
    frames_b = lerp_b + F * B * f4 + B * T * f4
    p.add(R.K_LERP_FRAMES, [f0, lerp, f0f, B, F, T], flags=SIDE, label="f0_frames",
          dispatch=f"perFrameScaled({B})", bytes=frames_b, flops=3.0 * B * T)
    tm = p.alloc("chain_timer", 16 * B * ((K + 63) // 64)) if chain_timer else 0
    p.add(R.K_PHASOR_CARRY, [f0f, ck, B, K, T, tm, int(chain_timer)], [cfg.sr], flags=SIDE, label="phasor_carry",
          dispatch=f"fixedWithFrameLoop({B * K})", bytes=B * T * f4 + ck_b, flops=6.0 * B * K * T, bound="valu")
    p.add(R.K_LERP_FRAMES, [uv, lerp, uvf, B, F, T], label="uv_frames", dispatch=f"perFrameScaled({B})",
          bytes=frames_b, flops=3.0 * B * T)
    W1, b1 = woff[0]
    p.add(R.K_DENSE_SMALL, [X, W1, b1, Hs[0], M, din, Hd], label="mlp_in", dispatch="gemmSmall",
          bytes=(M * din + din * Hd + Hd + M * Hd) * f4, flops=2.0 * M * din * Hd)
    mfma = "mfma_x6" if gm == 1 else "mfma"
    gemm_hh = dict(flops=2.0 * M * Hd * Hd, bound=mfma)
    # split-bf16 products: the weights are split into bfloat16 planes once
    # per step (W for the forward layers, W^T for the data gradients), so no
    # GEMM tile splits them again
    fwd_pl, bwd_pl = [-1] * Lyr, [-1] * Lyr
    fwd_plh = bwd_plh = -1
    # the heads' data gradient runs over NC rounded up to 32 (dZ's padding
    # columns are zero, and so are the planes' rows past NC), so its tiles
    # take the pipelined full-tile kernel (whole k-steps of 32)
    kh = NC if gm == 0 else min(LDC, (NC + 31) // 32 * 32)
    if gm == 1:
        for l in range(1, Lyr):
            W, _b = woff[l]
            fwd_pl[l] = _split_planes(p, f"W{l + 1}_planes", W, Hd, Hd, Hd, 1)
        fwd_plh = _split_planes(p, "Wh_planes", Wh, Hd, NC, NC, 1)
    for l in range(1, Lyr):
        W, b = woff[l]
        p.add(R.K_GEMM, _gemm_args(gm, [Hs[l - 1], W, Hs[l], M, Hd, Hd, Hd, Hd, Hd, 0, 0, R.EPI_BIAS_TANH, b, -1, 0, 1,
                                        0, -1], fwd_pl[l]),
              label=f"mlp_l{l + 1}", dispatch="gemm", bytes=(2 * M * Hd + Hd * Hd + Hd) * f4, **gemm_hh)
    p.add(R.K_GEMM, _gemm_args(gm, [Hs[-1], Wh, Z, M, NC, Hd, Hd, NC, LDC, 0, 0, R.EPI_BIAS, bh, -1, 0, 1, 0, -1],
                               fwd_plh),
          label="mlp_heads",
          dispatch="gemm", bytes=(M * Hd + Hd * NC + NC + M * NC) * f4, flops=2.0 * M * Hd * NC, bound=mfma)
    p.add(R.K_HEADS_FWD, [Z, ctrl, M, K, NF, LDC], label="heads", dispatch=f"perFrameScaled({M})",
          bytes=2 * M * NC * f4, flops=M * (K * 12.0 + NF * 8.0))
    if gm == 1 and train:
        # the data gradients' W^T planes: after the control network, where
        # stream 0 waits for the phase chain, not before the forward GEMMs
        for l in range(1, Lyr):
            W, _b = woff[l]
            bwd_pl[l] = _split_planes(p, f"W{l + 1}T_planes", W, Hd, Hd, 1, Hd)
        bwd_plh = _split_planes(p, "WhT_planes", Wh, NC, Hd, 1, NC, k_pad=kh)
    aux = p.alloc("synth_tape", 3 * B * T) if train else -1
    synth_args = [ctrl, f0f, uvf, lerp, ck, y, B, K, NF, F, T, SEG, aux, noise, LDC, segrows]
    hs, ns = cfg.hscale, cfg.nscale
    # per (b, t): K harmonics x (phase 4 + sin 20 + lerp 3 + mask/div 3 + sum 1 + normaliser 4), NF taps x 5
    synth_flops = float(B) * T * (35.0 * K + 5.0 * NF)
    p.add(R.K_SYNTH_FWD, synth_args, [cfg.sr, hs, ns], flags=JOIN, label="synth_fwd",
          dispatch=f"perFrameScaled({B})", bytes=ctrl_b + lerp_b + ck_b + data_b + B * T * f4 * (4 if train else 1),
          flops=synth_flops, bound="valu")
    p.output_cell = "y"
    if not train:
        return p

    # ---- loss + backward
    target = p.alloc("target", B * T)
    lossf = p.alloc("loss_frames", T)
    dy = p.alloc("dy", B * T)
    sizes = list(cfg.fft_sizes)
    if len(sizes) > 8:
        raise ValueError("at most 8 FFT sizes")
    ns_ = np.float32(len(sizes))
    wl = np.float32(cfg.w_lin) / ns_
    wg = np.float32(cfg.w_log) / ns_
    maxf = np.float32(T)
    gl = wl / maxf / np.float32(B)
    gg = wg / maxf / np.float32(B)
    if any(N not in (64, 128, 256, 512, 1024, 2048) for N in sizes) or cfg.hop_div != 4:
        raise ValueError("spectral loss sizes must be powers of two in [64, 2048] with hop N/4")
    ntiles = (T + MSS_TILE - 1) // MSS_TILE
    mss_part = p.alloc("mss_tiles", B * ntiles * (MSS_TILE + 2047))
    wloss_cells, hann_cells, mss_flops = [], [], 0.0
    for N in sizes:
        hop = N // 4
        nwin = (T + hop - 1) // hop
        wloss_cells.append(p.alloc(f"win_loss_{N}", nwin * B * 2))
        tab = p.alloc(f"fft_tables_{N}", 3 * N - 2)
        p.add(R.K_FFT_TABLES, [tab, N, 0 if cfg.hann else 1], flags=R.OP_STATIC, label=f"fft_tables_{N}",
              dispatch="static")
        hann_cells.append(tab)
        # two real forward transforms + one real-output inverse (2.5 N log2 N each) + bin math
        mss_flops += nwin * B * (7.5 * N * np.log2(N) + 30.0 * N)
    larg = [y, target, mss_part, B, T, len(sizes)] + (sizes + [0] * 8)[:8] + (wloss_cells + [0] * 8)[:8] \
        + (hann_cells + [0] * 8)[:8] + [cfg.mss_mode & 7]
    p.add(R.K_SPECTRAL_LOSS, larg, [gl, gg], label="spectral_mss",
          dispatch=f"perFrameScaledThreadgroup1({B}) x {len(sizes)} sizes",
          bytes=(2 * B * T + B * ntiles * (MSS_TILE + 2047) + sum((T + N // 4 - 1) // (N // 4) for N in sizes) * B * 2)
          * f4, flops=mss_flops, bound="valu")
    garg = [dy, -1, B, T, len(sizes)] + (sizes + [0] * 8)[:8] + [mss_part] + [0] * 7 + (wloss_cells + [0] * 8)[:8] \
        + [y, target]
    w_mse = np.float32(cfg.w_mse)
    mse_b = 2 * B * T * f4 if w_mse else 0
    # d loss / d y (the tile partials gathered per sample, plus the MSE
    # term) is formed by the synth backward as it reads it, and stored to dy
    # the per-frame loss signal (only reported, nothing in the backward reads
    # it) is a launch of its own at the end of stream 0, which finishes
    # before the side stream: folded into the combine, its blocks were the
    # combine's tail (25 -> 9 us + a separate 9 us); between the combine and
    # the synth backward it cost the step ~9 us; on the side stream 75 us
    larg2 = [-1, lossf] + garg[2:]
    nwin_all = sum((T + N // 4 - 1) // (N // 4) for N in sizes)

    # the backward's workgroups own runs of RUN_SEGS segments and write the
    # rows within their run to d ctrl; a row shared between runs leaves one
    # partial per run ([B][F][RUN_PARTS][LDC]), added by the row reduce
    bpart = p.alloc("synth_boundary_partials", B * F * RUN_PARTS * LDC)
    dctrl = p.alloc("dctrl", M * LDC)
    bargs = list(synth_args)
    bargs[5] = dy
    bargs[12] = bpart
    bargs += [aux, runtab, dctrl, 1, mss_part, y, target]
    # rows per lane: shared by two runs at each run boundary
    shared = min(F, 2 * max(0, nruns - 1))
    bpart_b = B * 2 * shared * NC * f4
    p.add(R.K_SYNTH_BWD, bargs, [cfg.sr, hs, ns, w_mse], label="synth_bwd", dispatch=f"selfManagedThreads({B})",
          bytes=ctrl_b + lerp_b + ck_b + data_b + 4 * B * T * f4 + (M - B * shared) * NC * f4 + bpart_b
          + B * ntiles * (MSS_TILE + 2047) * f4 + mse_b,
          flops=synth_flops + float(B) * T * (6.0 * K + 4.0 * NC), bound="valu")
    # the row reduce also runs the head backward of every row (dZ from d ctrl and Z)
    dZ = p.alloc("dZ", M * LDC)
    p.add(R.K_SYNTH_BWD_REDUCE, [bpart, rowlist, dctrl, B, NC, F, T, SEG, LDC, Z, dZ, K, NF], label="synth_bwd_reduce",
          dispatch=f"perFrameScaled({M})", bytes=bpart_b + F * ROW_ENTRIES * f4 + 3 * M * NC * f4,
          flops=bpart_b / f4 + M * (K * 20.0 + NF * 14.0))

    G = p.alloc("grads", npar)
    split = max(1, (M + SPLITK_ROWS - 1) // SPLITK_ROWS)
    split_h = max(1, (M + SPLITK_ROWS_HEADS - 1) // SPLITK_ROWS_HEADS)
    ws_gemm = p.alloc("splitk_ws", max(split * Hd * Hd, split_h * Hd * NC))
    chunks = min(256, max(1, M // 32))
    ws_col = p.alloc("colsum_ws", chunks * (din + 1) * max(Hd, NC))
    # The weight and bias gradients of the heads and hidden layers run on the
    # side stream, each forked after the data GEMM that produced its input, so
    # they overlap the data-gradient chain (dX_heads -> dX_l3 -> dX_l2); they
    # use their own column-sum workspace, and Adam joins them.
    ws_col_side = p.alloc("colsum_ws_side", chunks * max(Hd, NC)) if side_stream else ws_col
    gW = [(G + (w - P), G + (b - P)) for (w, b) in woff]
    gWh, gbh = G + (Wh - P), G + (bh - P)
    # heads: dWh = H_L^T dZ ; dbh = colsum(dZ) ; dH_L = (dZ Wh^T) * (1 - H_L^2)
    p.add(R.K_GEMM, _gemm_args(gm, [Hs[-1], dZ, gWh, Hd, NC, M, Hd, LDC, NC, 1, 0, R.EPI_NONE, -1, -1, 0, split_h, ws_gemm, -1]),
          flags=SIDE | FORK, label="dW_heads", dispatch="gemmChunkPartials", bytes=(M * Hd + M * NC + Hd * NC) * f4,
          flops=2.0 * M * Hd * NC, bound=mfma)
    p.add(R.K_COLSUM, [dZ, gbh, M, NC, LDC, ws_col_side], flags=SIDE, label="db_heads",
          dispatch="chunkPartialsReduceToCell", bytes=(M * NC + NC) * f4, flops=float(M * NC))
    dH = [p.alloc(f"dZ{l + 1}", M * Hd) for l in range(Lyr)]
    # column sums of dH[l] per 128-row GEMM tile, written by the data GEMM
    # that produces dH[l]; the bias gradient reduces these tile rows.  For
    # the first layer the tile also writes the sums weighted by each input
    # column of X, so W1 and b1 (contiguous in the parameters) reduce
    # together from (din + 1) partial rows per tile.
    mt = (M + GEMM_TILE_M - 1) // GEMM_TILE_M
    if din > 4:
        raise ValueError(f"first-layer fan-in {din} > 4")
    dcol = [p.alloc(f"dZ{l + 1}_tile_colsums", mt * (din + 1 if l == 0 else 1) * Hd) for l in range(Lyr)]
    wcol = [[X, din] if l == 0 else [-1, 0] for l in range(Lyr)]
    p.add(R.K_GEMM, _gemm_args(gm, [dZ, Wh, dH[-1], M, Hd, kh, LDC, NC, Hd, 0, 1, R.EPI_TANH_GRAD, -1, Hs[-1], Hd, 1, 0,
                                    dcol[-1]] + wcol[-1], bwd_plh),
          label=f"dX_heads", dispatch="gemm", bytes=(M * NC + Hd * NC + 2 * M * Hd) * f4, flops=2.0 * M * Hd * NC,
          bound=mfma)
    for l in range(Lyr - 1, 0, -1):
        W, _b = woff[l]
        gw, gb = gW[l]
        # the bias gradient (a short reduce of tile partials) goes ahead of
        # the weight GEMM on the side stream, so the last one is not left
        # after the final weight GEMM
        p.add(R.K_COLSUM, [dcol[l], gb, mt, Hd, Hd, ws_col_side], flags=SIDE | FORK, label=f"db_l{l + 1}",
              dispatch="chunkPartialsReduceToCell", bytes=(mt * Hd + Hd) * f4, flops=float(mt * Hd))
        p.add(R.K_GEMM, _gemm_args(gm, [Hs[l - 1], dH[l], gw, Hd, Hd, M, Hd, Hd, Hd, 1, 0, R.EPI_NONE, -1, -1, 0, split, ws_gemm,
                                         -1]),
              flags=SIDE, label=f"dW_l{l + 1}", dispatch="gemmChunkPartials",
              bytes=(2 * M * Hd + Hd * Hd) * f4, **gemm_hh)
        p.add(R.K_GEMM, _gemm_args(gm, [dH[l], W, dH[l - 1], M, Hd, Hd, Hd, Hd, Hd, 0, 1, R.EPI_TANH_GRAD, -1, Hs[l - 1], Hd, 1,
                                         0, dcol[l - 1]] + wcol[l - 1], bwd_pl[l]),
              label=f"dX_l{l + 1}", dispatch="gemm", bytes=(3 * M * Hd + Hd * Hd) * f4, **gemm_hh)
    gw1, gb1 = gW[0]
    if gb1 != gw1 + din * Hd:
        raise ValueError("first-layer weight and bias gradients are not contiguous")
    p.add(R.K_COLSUM, [dcol[0], gw1, mt, (din + 1) * Hd, (din + 1) * Hd, ws_col], label="dWb_l1",
          dispatch="chunkPartialsReduceToCell", bytes=(mt + 1) * (din + 1) * Hd * f4,
          flops=float(mt * (din + 1) * Hd))
    p.add(R.K_SPECTRAL_GATHER, larg2, [wl, wg, maxf, w_mse], label="loss_frames",
          dispatch="perFrame", bytes=(nwin_all * B * 2 + T) * f4 + mse_b, flops=float(nwin_all * B * 2))
    if optimizer:
        m = p.alloc("adam_m", npar)
        v = p.alloc("adam_v", npar)
        tcell = p.alloc("adam_t", 1)
        p.add(R.K_ADAM, [P, G, m, v, npar, tcell], [cfg.lr, 0.9, 0.999, 1e-8], flags=JOIN, label="adam",
              dispatch=f"staticThreads({npar})", bytes=7.0 * npar * f4, flops=12.0 * npar)
    p.output_cell = "y"
    return p


def check_row_schedule(rt: R.HIPLazyRuntime) -> None:
    """The static row schedule reports overflow in a flag cell; fail loudly."""
    flag = float(rt.read("row_flag")[0])
    if flag != 0.0:
        raise R.HIPError(f"row schedule overflow (flag {flag}): a synth segment touches more than {SLOTS} "
                         f"control rows or a row more than {ROW_ENTRIES} segments")


class HarmonicSession:
    """Owns a training runtime (and a render runtime for the target) for one
    HarmonicConfig.  Inputs are staged once; every ``step()`` is one
    forward+backward(+Adam) pass with all data resident in HBM."""

    def __init__(self, cfg: HarmonicConfig, device: int = 0, optimizer: bool = True, target=None,
                 side_stream: bool = True, data=None, chain_timer: bool = False):
        self.cfg = cfg
        f0, uv, X = cfg.data() if data is None else data
        self.f0, self.uv, self.X = f0, uv, X
        self.params0 = cfg.weights()
        if target is None:
            target = self.render(cfg.weights(seed=cfg.target_seed), device)
        self.target = np.ascontiguousarray(target, np.float32).reshape(cfg.B, cfg.T)
        self.program = harmonic_program(cfg, train=True, optimizer=optimizer, side_stream=side_stream,
                                        chain_timer=chain_timer)
        self.rt = R.HIPLazyRuntime(self.program, device)
        check_row_schedule(self.rt)
        self.rt.write("X", X)
        self.rt.write("f0", f0)
        self.rt.write("uv", uv)
        self.rt.write("params", self.params0)
        self.rt.write("target", self.target)

    def render(self, params, device: int = 0) -> np.ndarray:
        prog = harmonic_program(self.cfg, train=False)
        with R.HIPLazyRuntime(prog, device) as rt:
            check_row_schedule(rt)
            rt.write("X", self.X)
            rt.write("f0", self.f0)
            rt.write("uv", self.uv)
            rt.write("params", params)
            rt.runNoCopy()
            return rt.read("y").reshape(self.cfg.B, self.cfg.T)

    def set_batch(self, f0, uv, X, target) -> None:
        """Stage the next batch (f0, uv [F][B], features X [B*F][din], target
        [B][T]; e.g. ``dataset.harmonic_batch`` of cached chunks) for the
        following steps, as the reference trainer updates its data tensors."""
        cfg = self.cfg
        for name, a, n in (("f0", f0, cfg.F * cfg.B), ("uv", uv, cfg.F * cfg.B), ("X", X, cfg.M * cfg.din),
                           ("target", target, cfg.B * cfg.T)):
            if np.asarray(a).size != n:
                raise ValueError(f"{name}: {np.asarray(a).size} values, the session takes {n}")
            self.rt.write(name, np.ascontiguousarray(a, np.float32))
        self.f0, self.uv, self.X = f0, uv, X
        self.target = np.ascontiguousarray(target, np.float32).reshape(cfg.B, cfg.T)

    def step(self) -> None:
        self.rt.runNoCopy()

    def loss(self) -> float:
        return float(self.rt.read("loss_frames").astype(np.float64).sum())

    def close(self):
        self.rt.close()


# ------------------------------------------------------------------ config 4
def _colsum_ws(rows: int, cols: int) -> int:
    return max(1, min(256, rows // 32)) * cols


def biquad_program(cfg: BiquadConfig, train: bool = True, optimizer: bool = True, modulated: bool = True,
                   chunk: int = BQ_CHUNK, fuse_adjoint: bool = True) -> Program:
    """Tensor biquad bank: x -> RBJ low-pass with cutoff base[k]*mod[n] and Q[k].

    ``train=False`` builds the forward render only (used for the fixed target
    bank, ``modulated=False``).  With ``train=True``: forward, loss
    sum (y - target)^2, BPTT to (base, Q), and (``optimizer``) one Adam step.
    Each recurrence runs as a chunked scan (chunk summaries, per-lane carry
    composition, replay) forward and, for the adjoint, backward.  With
    ``fuse_adjoint`` the forward replay also forms the adjoint's chunk
    summaries; without it a separate reverse pass over y and the target
    does."""
    B, T, L = cfg.B, cfg.T, int(chunk)
    if L <= 0:
        raise ValueError("chunk length must be positive")
    C = (T + L - 1) // L
    f4 = 4.0
    p = Program(max_frames=T)
    p.meta.update(cfg=cfg, chunk=L, chunks=C, train=train)
    x = p.alloc("x", T * B)
    mod = p.alloc("mod", T) if modulated else -1
    P = p.alloc("params", 2 * B)
    y = p.alloc("y", T * B)
    summ = p.alloc("summary", 12 * C * B)  # fp64
    init = p.alloc("init", 2 * C * B)
    # algorithmic cost per lane-frame: coefficients (|.|, cos, sin, 2 div, 9 mul/add) ~ 16 flops,
    # one Direct Form I step 9 flops
    n = float(T * B)
    mod_b = float(T) * f4 if modulated else 0.0
    sfx = "" if modulated else " (fixed cutoff)"
    p.add(R.K_BIQUAD_CHUNK, [x, mod, P, summ, B, T, L], label="bq_chunk", dispatch=f"chunk summaries {C}x{B}{sfx}",
          bytes=n * f4 + mod_b + 12.0 * C * B * f4, flops=n * (16 + 3 * 9))
    p.add(R.K_BIQUAD_CARRY, [summ, init, B, C, 0], label="bq_carry", dispatch=f"per-lane scan of {C} chunk maps",
          bytes=(12.0 + 2.0) * C * B * f4, flops=24.0 * C * B)
    if not train:
        p.add(R.K_BIQUAD_FWD, [x, mod, P, init, y, B, T, L, -1, -1], label="bq_fwd", dispatch=f"chunk replay{sfx}",
              bytes=2 * n * f4 + mod_b + 2.0 * C * B * f4, flops=n * (16 + 9))
        p.output_cell = "y"
        return p
    tgt = p.alloc("target", T * B)
    lossp = p.alloc("loss_partials", C * B)
    lane_loss = p.alloc("lane_loss", B)
    loss = p.alloc("loss", 1)
    asumm = p.alloc("adj_summary", 12 * C * B)  # fp64
    ainit = p.alloc("adj_init", 2 * C * B)
    gpart = p.alloc("grad_partials", 2 * C * B)
    G = p.alloc("grads", 2 * B)
    ws = p.alloc("colsum_ws", max(_colsum_ws(C, 2 * B), _colsum_ws(C, B), _colsum_ws(B, 1)))
    # fused: the replay also forms the adjoint chunk summaries (forward
    # prefix products), so no separate backward pass over y and the target
    p.add(R.K_BIQUAD_FWD, [x, mod, P, init, y, B, T, L, tgt, lossp] + ([asumm, 1] if fuse_adjoint else []),
          label="bq_fwd", dispatch="chunk replay + loss partials" + (" + adjoint summaries" if fuse_adjoint else ""),
          bytes=3 * n * f4 + mod_b + 3.0 * C * B * f4 + (12.0 * C * B * f4 if fuse_adjoint else 0.0),
          flops=n * (16 + 9 + 3 + (12 if fuse_adjoint else 0)))
    p.add(R.K_COLSUM, [lossp, lane_loss, C, B, B, ws], label="loss_lanes", dispatch="chunkPartialsReduceToCell",
          bytes=(C * B + B) * f4, flops=float(C * B))
    p.add(R.K_COLSUM, [lane_loss, loss, B, 1, 1, ws], label="loss_sum", dispatch="chunkPartialsReduceToCell",
          bytes=(B + 1) * f4, flops=float(B))
    if not fuse_adjoint:
        p.add(R.K_BIQUAD_ADJ_CHUNK, [mod, P, y, tgt, asumm, B, T, L], label="bq_adj_chunk",
              dispatch=f"reverse chunk summaries {C}x{B}", bytes=2 * n * f4 + mod_b + 12.0 * C * B * f4,
              flops=n * (16 + 3 * 6))
    p.add(R.K_BIQUAD_CARRY, [asumm, ainit, B, C, 1], label="bq_adj_carry", dispatch=f"reverse scan of {C} maps",
          bytes=(12.0 + 2.0) * C * B * f4, flops=24.0 * C * B)
    p.add(R.K_BIQUAD_BWD, [x, mod, P, y, tgt, ainit, gpart, B, T, L], label="bq_bwd",
          dispatch="reverse chunk replay + gradient partials", bytes=3 * n * f4 + mod_b + 4.0 * C * B * f4,
          flops=n * (16 + 6 + 30))
    p.add(R.K_COLSUM, [gpart, G, C, 2 * B, 2 * B, ws], label="grad_sum", dispatch="chunkPartialsReduceToCell",
          bytes=(2.0 * C * B + 2 * B) * f4, flops=2.0 * C * B)
    if optimizer:
        m = p.alloc("adam_m", 2 * B)
        v = p.alloc("adam_v", 2 * B)
        tcell = p.alloc("adam_t", 1)
        p.add(R.K_ADAM, [P, G, m, v, 2 * B, tcell], [cfg.lr, 0.9, 0.999, 1e-8], label="adam",
              dispatch=f"staticThreads({2 * B})", bytes=7.0 * 2 * B * f4, flops=12.0 * 2 * B)
    p.output_cell = "y"
    return p


def stream_biquad_program(cfg: BiquadConfig, max_frames: int | None = None, modulated: bool = True) -> Program:
    """The config-4 bank as a streaming process: per call, B input channels
    (and the modulation channel) in, B output channels out, the four history
    cells of every lane carried over (StatefulTensorParallelPolicy's per-lane
    frame loop)."""
    B, T = cfg.B, int(max_frames or cfg.T)
    p = Program(max_frames=T)
    # the graph's memory first (parameters, the lanes' history cells), then
    # the channels' staging cells
    P = p.alloc("params", 2 * B)
    st = p.alloc("state", 4 * B)
    memory = p.size
    x = p.alloc("x", T * B)
    mod = p.alloc("mod", T) if modulated else -1
    y = p.alloc("y", T * B)
    p.add(R.K_STREAM_BIQUAD, [x, mod, P, st, y, B, T], label="stream_biquad",
          dispatch=f"fixedWithFrameLoop({B})", bytes=8.0 * T * B, flops=float(T * B) * (16 + 9), bound="valu")
    p.output_cell = "y"
    ins = [("x", k, B) for k in range(B)] + ([("mod", 0, 1)] if modulated else [])
    p.meta.update(cfg=cfg, ports=(ins, [("y", k, B) for k in range(B)]), memory=(0, memory))
    return p


class BiquadSession:
    """Config-4 training runtime: the target bank is rendered once by a
    forward-only program with the fixed (tgt_fc, tgt_Q) coefficients, then
    every ``step()`` is forward + loss + BPTT (+ Adam) with all data in HBM."""

    def __init__(self, cfg: BiquadConfig, device: int = 0, optimizer: bool = True, chunk: int = BQ_CHUNK,
                 target=None, fuse_adjoint: bool = True):
        self.cfg = cfg
        self.x = cfg.inputs()
        self.mod = cfg.modulation()
        self.params0 = cfg.params()
        if target is None:
            target = self.render(cfg.target_params(), device, modulated=False, chunk=chunk)
        self.target = np.ascontiguousarray(target, np.float32).reshape(cfg.T, cfg.B)
        self.program = biquad_program(cfg, train=True, optimizer=optimizer, chunk=chunk, fuse_adjoint=fuse_adjoint)
        self.rt = R.HIPLazyRuntime(self.program, device)
        self.rt.write("x", self.x)
        self.rt.write("mod", self.mod)
        self.rt.write("params", self.params0)
        self.rt.write("target", self.target)

    def render(self, params, device: int = 0, modulated: bool = True, chunk: int = BQ_CHUNK) -> np.ndarray:
        prog = biquad_program(self.cfg, train=False, modulated=modulated, chunk=chunk)
        with R.HIPLazyRuntime(prog, device) as rt:
            rt.write("x", self.x)
            if modulated:
                rt.write("mod", self.mod)
            rt.write("params", params)
            rt.runNoCopy()
            return rt.read("y").reshape(self.cfg.T, self.cfg.B)

    def step(self) -> None:
        self.rt.runNoCopy()

    def loss(self) -> float:
        return float(self.rt.read("loss")[0])

    def close(self):
        self.rt.close()


# ------------------------------------------------------ ZDF SVF bank (BPTT)
def svf_program(cfg: SvfConfig, train: bool = True, optimizer: bool = True, saturating: bool | None = None,
                chunk: int = SVF_CHUNK, xbar: bool = False, fuse_adjoint: bool = True) -> Program:
    """ZDF SVF low-pass bank: x -> y with cutoff clip(base[k]*mod[n] + env[n])
    and res[k] (and, saturating, kSat[k]).

    Linear (kSat the constant 0): the forward is a chunked scan (fp64 chunk
    maps, per-lane carry composition, fp32 replay).  Saturating: one lane per
    thread over all frames.  ``train=False`` renders y only.  With
    ``train=True``: forward storing the cells entering every frame, loss
    sum (y - target)^2, BPTT to the parameters as a chunked reverse scan
    (``xbar``: also d loss / d x), and (``optimizer``) one Adam step.  With
    ``fuse_adjoint`` (linear bank) the forward replay also forms the
    adjoint's chunk summaries, else a separate reverse pass over y and the
    target does."""
    sat = cfg.saturating if saturating is None else bool(saturating)
    B, T, L = cfg.B, cfg.T, int(chunk)
    if L <= 0:
        raise ValueError("chunk length must be positive")
    P = 3 if sat else 2
    C = (T + L - 1) // L
    f4 = 4.0
    n = float(T * B)
    p = Program(max_frames=T)
    p.meta.update(cfg=cfg, chunk=L, chunks=C, train=train, saturating=sat, P=P)
    x = p.alloc("x", T * B)
    mod = p.alloc("mod", T)
    env = p.alloc("env", T)
    prm = p.alloc("params", P * B)
    y = p.alloc("y", T * B)
    sr = [cfg.sr]
    ctl_b = 2.0 * T * f4
    cells = p.alloc("cells", 2 * T * B) if train else -1
    tgt = p.alloc("target", T * B) if train else -1
    lossp = p.alloc("loss_partials", C * B) if train else -1
    asumm = p.alloc("adj_summary", 12 * C * B) if train else -1  # fp64
    # linear: the forward replay forms the adjoint chunk summaries too
    fused = train and fuse_adjoint and not sat
    # per lane-frame: coefficients (clip, div, tan, 1/Q, 4 mul/add) ~ 30 flops, one SVF frame 12
    if sat:
        tape = p.alloc("coef_tape", T * B)
        p.add(R.K_SVF_SEQ, [x, mod, env, prm, -1, y, cells, tgt, lossp, B, T, L, 0, tape], sr, label="svf_seq",
              dispatch=f"coefficient tape + fixedWithFrameLoop({B})",
              bytes=n * f4 * ((5 if train else 2) + 2) + ctl_b, flops=n * (30 + 18), bound="valu")
    else:
        summ = p.alloc("summary", 12 * C * B)  # fp64
        init = p.alloc("init", 2 * C * B)
        p.add(R.K_SVF_CHUNK, [x, mod, env, prm, summ, B, T, L], sr, label="svf_chunk",
              dispatch=f"chunk summaries {C}x{B}", bytes=n * f4 + ctl_b + 12.0 * C * B * f4,
              flops=n * (30 + 3 * 10))
        p.add(R.K_BIQUAD_CARRY, [summ, init, B, C, 0], label="svf_carry", dispatch=f"per-lane scan of {C} chunk maps",
              bytes=(12.0 + 2.0) * C * B * f4, flops=24.0 * C * B)
        p.add(R.K_SVF_FWD, [x, mod, env, prm, init, y, cells, tgt, lossp, B, T, L] + ([asumm, 1] if fused else []),
              sr, label="svf_fwd",
              dispatch="chunk replay" + (" + cells + loss partials" if train else "")
              + (" + adjoint summaries" if fused else ""),
              bytes=n * f4 * (5 if train else 2) + ctl_b + 2.0 * C * B * f4 + (12.0 * C * B * f4 if fused else 0.0),
              flops=n * (30 + 12 + (22 if fused else 0)))
    if not train:
        p.output_cell = "y"
        return p
    lane_loss = p.alloc("lane_loss", B)
    loss = p.alloc("loss", 1)
    ainit = p.alloc("adj_init", 2 * C * B)
    gpart = p.alloc("grad_partials", P * C * B)
    G = p.alloc("grads", P * B)
    xb = p.alloc("xbar", T * B) if xbar else -1
    ws = p.alloc("colsum_ws", max(_colsum_ws(C, P * B), _colsum_ws(C, B), _colsum_ws(B, 1)))
    p.add(R.K_COLSUM, [lossp, lane_loss, C, B, B, ws], label="loss_lanes", dispatch="chunkPartialsReduceToCell",
          bytes=(C * B + B) * f4, flops=float(C * B))
    p.add(R.K_COLSUM, [lane_loss, loss, B, 1, 1, ws], label="loss_sum", dispatch="chunkPartialsReduceToCell",
          bytes=(B + 1) * f4, flops=float(B))
    if not fused:
        p.add(R.K_SVF_ADJ_CHUNK, [mod, env, prm, y, tgt, cells if sat else -1, asumm, B, T, L, int(sat)], sr,
              label="svf_adj_chunk", dispatch=f"reverse chunk summaries {C}x{B}",
              bytes=n * f4 * (4 if sat else 2) + ctl_b + 12.0 * C * B * f4, flops=n * (30 + 3 * 12))
    p.add(R.K_BIQUAD_CARRY, [asumm, ainit, B, C, 1], label="svf_adj_carry", dispatch=f"reverse scan of {C} maps",
          bytes=(12.0 + 2.0) * C * B * f4, flops=24.0 * C * B)
    p.add(R.K_SVF_BWD, [x, mod, env, prm, y, tgt, cells, ainit, gpart, xb, B, T, L, int(sat)], sr, label="svf_bwd",
          dispatch="reverse chunk replay + gradient partials",
          bytes=n * f4 * (5 + (1 if xbar else 0)) + ctl_b + (2.0 + P) * C * B * f4, flops=n * (30 + 12 + 40))
    p.add(R.K_COLSUM, [gpart, G, C, P * B, P * B, ws], label="grad_sum", dispatch="chunkPartialsReduceToCell",
          bytes=(P * C * B + P * B) * f4, flops=float(P * C * B))
    if optimizer:
        m = p.alloc("adam_m", P * B)
        v = p.alloc("adam_v", P * B)
        tcell = p.alloc("adam_t", 1)
        p.add(R.K_ADAM, [prm, G, m, v, P * B, tcell], [cfg.lr, 0.9, 0.999, 1e-8], label="adam",
              dispatch=f"staticThreads({P * B})", bytes=7.0 * P * B * f4, flops=12.0 * P * B)
    p.output_cell = "y"
    return p


def stream_svf_program(cfg: SvfConfig, max_frames: int | None = None) -> Program:
    """The SVF bank as a streaming process: per call, B input channels plus
    the modulation and envelope channels in, B output channels out, each
    lane's two cells carried over (params [3][B]; kSat 0 is the linear
    filter).  Out stores map non-finite values to 0."""
    B, T = cfg.B, int(max_frames or cfg.T)
    p = Program(max_frames=T)
    # the graph's memory first (parameters, the lanes' two cells), then the
    # channels' staging cells
    prm = p.alloc("params", 3 * B)
    st = p.alloc("state", 2 * B)
    memory = p.size
    x = p.alloc("x", T * B)
    mod = p.alloc("mod", T)
    env = p.alloc("env", T)
    y = p.alloc("y", T * B)
    p.add(R.K_STREAM_SVF, [x, mod, env, prm, st, y, -1, -1, -1, B, T, SVF_CHUNK, 1, -1], [cfg.sr], label="stream_svf",
          dispatch=f"fixedWithFrameLoop({B})", bytes=8.0 * T * B, flops=float(T * B) * (30 + 18), bound="valu")
    p.output_cell = "y"
    ins = [("x", k, B) for k in range(B)] + [("mod", 0, 1), ("env", 0, 1)]
    p.meta.update(cfg=cfg, ports=(ins, [("y", k, B) for k in range(B)]), memory=(0, memory))
    return p


class SvfSession:
    """SVF-bank training runtime: the target bank is rendered once by a linear
    forward-only program with (tgt_fc, tgt_res), then every ``step()`` is
    forward + loss + BPTT (+ Adam) with all data in HBM."""

    def __init__(self, cfg: SvfConfig, device: int = 0, optimizer: bool = True, chunk: int = SVF_CHUNK,
                 target=None, xbar: bool = False, fuse_adjoint: bool = True):
        self.cfg = cfg
        self.x = cfg.inputs()
        self.mod = cfg.modulation()
        self.env = cfg.envelope()
        self.params0 = cfg.params()
        if target is None:
            target = self.render(cfg.target_params(), device, saturating=False, chunk=chunk)
        self.target = np.ascontiguousarray(target, np.float32).reshape(cfg.T, cfg.B)
        self.program = svf_program(cfg, train=True, optimizer=optimizer, chunk=chunk, xbar=xbar,
                                   fuse_adjoint=fuse_adjoint)
        self.rt = R.HIPLazyRuntime(self.program, device)
        for name, a in (("x", self.x), ("mod", self.mod), ("env", self.env), ("params", self.params0),
                        ("target", self.target)):
            self.rt.write(name, a)

    def render(self, params, device: int = 0, saturating: bool = False, chunk: int = SVF_CHUNK) -> np.ndarray:
        prog = svf_program(self.cfg, train=False, saturating=saturating, chunk=chunk)
        with R.HIPLazyRuntime(prog, device) as rt:
            for name, a in (("x", self.x), ("mod", self.mod), ("env", self.env), ("params", params)):
                rt.write(name, a)
            rt.runNoCopy()
            return rt.read("y").reshape(self.cfg.T, self.cfg.B)

    def step(self) -> None:
        self.rt.runNoCopy()

    def loss(self) -> float:
        return float(self.rt.read("loss")[0])

    def close(self):
        self.rt.close()


# ------------------------------------------------- temporal gradient (a21)
def swept_phasor_program(cfg: SweptPhasorConfig, optimizer: bool = True) -> Program:
    """The swept-phasor bank forward, loss and backward to the sweep rates:
    time = accum(1/sr) (a static table), the per-lane stateful phasor of
    base + slope * time with the mse loss, the phasor's temporal gradient (the
    reset-aware suffix scan, / sr) and d f / d slope = time summed over frames
    (Gradients.swift:209-261), then (``optimizer``) one Adam step."""
    E, T = cfg.E, cfg.T
    C = (T + 255) // 256
    f4 = 4.0
    p = Program(max_frames=T)
    p.meta.update(cfg=cfg)
    slope = p.alloc("slope", E)
    time = p.alloc("time", T)
    reset = p.alloc("reset", T)
    gup = p.alloc("upstream", T * E)
    lossp = p.alloc("loss_partials", E)
    loss = p.alloc("loss", 1)
    dfreq = p.alloc("dfreq", T * E)
    G = p.alloc("grads", E)
    ws_scan = p.alloc("scan_ws", 2 * C * E + C)
    chunks = min(256, max(1, T // 32))
    ws_col = p.alloc("colsum_ws", max(chunks * 2 * E, _colsum_ws(E, 1)))
    step = np.float32(np.float32(1.0) / np.float32(cfg.sr))
    p.add(R.K_ACCUM_TABLE, [time, T], [step, 0.0, 1.0, 0.0, 1.0], flags=R.OP_STATIC, label="time",
          dispatch="static singleThreaded")
    n = float(T * E)
    p.add(R.K_SWEPT_PHASOR, [slope, time, reset, -1, gup, lossp, E, T, int(cfg.smooth)], [cfg.sr, cfg.base, cfg.target],
          label="swept_phasor", dispatch=f"fixedWithFrameLoop({E})", bytes=n * f4 + T * 2 * f4, flops=n * 10.0,
          bound="valu")
    p.add(R.K_COLSUM, [lossp, loss, E, 1, 1, ws_col], label="loss_sum", dispatch="chunkPartialsReduceToCell",
          bytes=(E + 1) * f4, flops=float(E))
    p.add(R.K_TEMPORAL_GRAD_SCAN, [gup, reset, dfreq, E, T, ws_scan, 1], [cfg.sr], label="temporal_scan",
          dispatch=f"temporalGradScan({E}) chunked", bytes=2 * n * f4 + T * f4, flops=2.0 * n)
    p.add(R.K_DENSE_SMALL_WGRAD, [time, dfreq, G, T, 1, E, ws_col, -1], label="dslope",
          dispatch="chunkPartialsReduceToCell", bytes=(n + T + E) * f4, flops=2.0 * n)
    if optimizer:
        m = p.alloc("adam_m", E)
        v = p.alloc("adam_v", E)
        tcell = p.alloc("adam_t", 1)
        p.add(R.K_ADAM, [slope, G, m, v, E, tcell], [cfg.lr, 0.9, 0.999, 1e-8], label="adam",
              dispatch=f"staticThreads({E})", bytes=7.0 * E * f4, flops=12.0 * E)
    p.output_cell = "loss"
    return p


class SweptPhasorSession:
    """A swept-phasor bank runtime: slopes and the reset signal staged once,
    every ``step()`` is forward + loss + temporal-gradient backward (+ Adam)."""

    def __init__(self, cfg: SweptPhasorConfig, device: int = 0, optimizer: bool = True):
        self.cfg = cfg
        self.program = swept_phasor_program(cfg, optimizer=optimizer)
        self.rt = R.HIPLazyRuntime(self.program, device)
        self.rt.write("slope", cfg.slopes())
        self.rt.write("reset", cfg.reset())

    def step(self) -> None:
        self.rt.runNoCopy()

    def loss(self) -> float:
        return float(self.rt.read("loss")[0])

    def close(self):
        self.rt.close()


# ------------------------------------------------------------------ config 2
def stft_windows_per_block(N: int) -> int:
    """Windows summed by one gain-gradient workgroup (8 rounds of 4096/N)."""
    return 8 * (4096 // N)


def stft_program(cfg: StftConfig, train: bool = True, optimizer: bool = True) -> Program:
    """x.buffer(N, hop H) * hann -> FFT -> gains -> IFFT -> overlapAdd, loss
    sum (y - x)^2 / T against the raw input, gradient to the N/2+1 gains
    (``train``) and one Adam step (``optimizer``)."""
    S, T, N, H, nb = cfg.S, cfg.T, cfg.N, cfg.H, cfg.bins
    ntiles = (T + STFT_TILE - 1) // STFT_TILE
    nwin = (T + H - 1) // H
    nblk = (nwin + stft_windows_per_block(N) - 1) // stft_windows_per_block(N)
    f4 = 4.0
    p = Program(max_frames=T)
    p.meta.update(cfg=cfg, ntiles=ntiles, nblk=nblk, train=train)
    x = p.alloc("x", S * T)
    win = p.alloc("window", N)
    g = p.alloc("gains", nb)
    y = p.alloc("y", S * T)
    lognn = float(np.log2(N))
    fft_flops = 2.5 * N * lognn  # one real N-point transform (split-radix estimate)
    windows = float(S * nwin)
    halo = 1.0 + (N - H) / STFT_TILE  # windows recomputed at tile edges
    if not train:
        p.add(R.K_STFT_FWD, [x, win, g, y, -1, -1, S, T, N, H], label="stft_fwd",
              dispatch=f"tiles {ntiles}x{S}, windows {nwin}/signal", bytes=2.0 * S * T * f4,
              flops=windows * halo * 2 * fft_flops)
        p.output_cell = "y"
        return p
    dy = p.alloc("dy", S * T)
    lossp = p.alloc("loss_partials", S * ntiles)
    loss = p.alloc("loss", 1)
    gpart = p.alloc("grad_partials", S * nblk * nb)
    G = p.alloc("grads", nb)
    ws = p.alloc("colsum_ws", max(_colsum_ws(S * ntiles, 1), _colsum_ws(S * nblk, nb)))
    p.add(R.K_STFT_FWD, [x, win, g, y, dy, lossp, S, T, N, H], label="stft_fwd",
          dispatch=f"tiles {ntiles}x{S}, windows {nwin}/signal", bytes=3.0 * S * T * f4,
          flops=windows * halo * 2 * fft_flops)
    p.add(R.K_COLSUM, [lossp, loss, S * ntiles, 1, 1, ws], label="loss_sum", dispatch="chunkPartialsReduceToCell",
          bytes=(S * ntiles + 1) * f4, flops=float(S * ntiles))
    p.add(R.K_STFT_BWD, [x, win, dy, gpart, S, T, N, H], label="stft_bwd",
          dispatch=f"window runs {nblk}x{S}", bytes=2.0 * S * T * f4 + S * nblk * nb * f4,
          flops=windows * (2 * fft_flops + 4 * nb))
    p.add(R.K_COLSUM, [gpart, G, S * nblk, nb, nb, ws], label="grad_sum", dispatch="chunkPartialsReduceToCell",
          bytes=(S * nblk * nb + nb) * f4, flops=float(S * nblk * nb))
    if optimizer:
        m = p.alloc("adam_m", nb)
        v = p.alloc("adam_v", nb)
        tcell = p.alloc("adam_t", 1)
        p.add(R.K_ADAM, [g, G, m, v, nb, tcell], [cfg.lr, 0.9, 0.999, 1e-8], label="adam",
              dispatch=f"staticThreads({nb})", bytes=7.0 * nb * f4, flops=12.0 * nb)
    p.output_cell = "y"
    return p


class StftSession:
    """Config-2 training runtime: x, the window and the gains staged once;
    every ``step()`` is forward + loss + gain gradient (+ Adam) in HBM."""

    def __init__(self, cfg: StftConfig, device: int = 0, optimizer: bool = True, gains=None):
        self.cfg = cfg
        self.x = cfg.inputs()
        self.window = cfg.window()
        self.gains0 = cfg.gains() if gains is None else np.ascontiguousarray(gains, np.float32)
        self.program = stft_program(cfg, train=True, optimizer=optimizer)
        self.rt = R.HIPLazyRuntime(self.program, device)
        self.rt.write("x", self.x)
        self.rt.write("window", self.window)
        self.rt.write("gains", self.gains0)

    def step(self) -> None:
        self.rt.runNoCopy()

    def loss(self) -> float:
        return float(self.rt.read("loss")[0])

    def close(self):
        self.rt.close()


# ------------------------------------------------------------------ config 5
def membrane_program(cfg: MembraneConfig, train: bool = True, optimizer: bool = True,
                     steps: int = MEM_STEPS) -> Program:
    """Damped 2D wave equation on an R x C grid for T frames with a point
    pickup; with ``train`` the loss sum (out - target)^2, the discrete adjoint
    to (c2, d) and (``optimizer``) one Adam step.  Every forward state stays
    in HBM for the adjoint: (T + 2) fields of R x C floats."""
    rows, cols, T = cfg.R, cfg.C, cfg.T
    G = rows * cols
    py, px = cfg.pickup
    tiles = ((rows + MEM_TILE - 1) // MEM_TILE) * ((cols + MEM_TILE - 1) // MEM_TILE)
    f4 = 4.0
    p = Program(max_frames=T)
    p.meta.update(cfg=cfg, steps=steps, tiles=tiles, train=train)
    u0 = p.alloc("u0", G)
    P = p.alloc("params", 2)
    out = p.alloc("pickup", T)
    S = p.alloc("states", (T + 2) * G)
    cell_steps = float(G) * T
    # Compulsory HBM traffic of the store-every-state design: the forward
    # writes each state once (4 B per cell-step) for the adjoint, which reads
    # each once (4 B); the two fields a step reads and the adjoint fields
    # stay on chip inside a time-blocked launch.  ~10 flops per cell-step.
    p.add(R.K_MEMBRANE_FWD, [S, u0, P, out, rows, cols, T, py, px, steps], label="membrane_fwd",
          dispatch=f"{(T + steps - 1) // steps} time-blocked launches x {tiles} tiles",
          bytes=4.0 * cell_steps, flops=10.0 * cell_steps)
    if not train:
        p.output_cell = "pickup"
        return p
    tgt = p.alloc("target", T)
    lam = p.alloc("adjoint_fields", 4 * G)
    gpart = p.alloc("grad_partials", 4 * tiles * MEM_WAVES)  # fp64 (c2, d) per tile and wave
    lt = p.alloc("loss_terms", T)
    loss = p.alloc("loss", 1)
    Gc = p.alloc("grads", 2)
    ws = p.alloc("colsum_ws", _colsum_ws(T, 1))
    # per cell-step: the stored state read once (4 B); ~14 flops
    p.add(R.K_MEMBRANE_BWD, [S, P, out, tgt, lam, gpart, lt, rows, cols, T, py, px, steps, Gc], label="membrane_bwd",
          dispatch=f"{T // steps + 1} time-blocked adjoint launches x {tiles} tiles",
          bytes=4.0 * cell_steps, flops=14.0 * cell_steps)
    p.add(R.K_COLSUM, [lt, loss, T, 1, 1, ws], label="loss_sum", dispatch="chunkPartialsReduceToCell",
          bytes=(T + 1) * f4, flops=float(T))
    if optimizer:
        m = p.alloc("adam_m", 2)
        v = p.alloc("adam_v", 2)
        tcell = p.alloc("adam_t", 1)
        p.add(R.K_ADAM, [P, Gc, m, v, 2, tcell], [cfg.lr, 0.9, 0.999, 1e-8], label="adam",
              dispatch="staticThreads(2)", bytes=14.0 * f4, flops=24.0)
    p.output_cell = "pickup"
    return p


class MembraneSession:
    """Config-5 training runtime: the target pickup series is rendered once
    with (tgt_c2, tgt_d); every ``step()`` is forward + loss + adjoint
    (+ Adam) with all states in HBM."""

    def __init__(self, cfg: MembraneConfig, device: int = 0, optimizer: bool = True, steps: int = MEM_STEPS,
                 target=None):
        self.cfg = cfg
        self.u0 = cfg.bump()
        self.params0 = cfg.params()
        if target is None:
            target = self.render(cfg.target_params(), device, steps)
        self.target = np.ascontiguousarray(target, np.float32).reshape(cfg.T)
        self.program = membrane_program(cfg, train=True, optimizer=optimizer, steps=steps)
        self.rt = R.HIPLazyRuntime(self.program, device)
        self.rt.write("u0", self.u0)
        self.rt.write("params", self.params0)
        self.rt.write("target", self.target)

    def render(self, params, device: int = 0, steps: int = MEM_STEPS) -> np.ndarray:
        with R.HIPLazyRuntime(membrane_program(self.cfg, train=False, steps=steps), device) as rt:
            rt.write("u0", self.u0)
            rt.write("params", params)
            rt.runNoCopy()
            return rt.read("pickup")

    def step(self) -> None:
        self.rt.runNoCopy()

    def loss(self) -> float:
        return float(self.rt.read("loss")[0])

    def close(self):
        self.rt.close()
