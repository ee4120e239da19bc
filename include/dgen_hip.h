/*
 * dgen_hip.h -- C ABI of libdgen_hip.so, the MI355X (gfx950) execution backend
 * for DGen schedules.
 *
 * The library plays the two roles the reference splits between a Renderer
 * and a LazyRuntime:
 *   - it accepts a *schedule*: an ordered list of kernel-class launches over
 *     cells of one flat float arena (the reference's `memory`, addressed by
 *     cell offsets), i.e. what a renderer emits as [CompiledKernel]
 *     (reference: Sources/DGen/Renderer/Renderer.swift:134-143, 203-226);
 *   - it owns the device arena, a pinned host mirror, the HIP streams and the
 *     per-kernel timing, mirroring the LazyRuntime protocol
 *     (Sources/DGenLazy/Realize.swift:12-19) and MetalCompiledKernel
 *     (Sources/DGen/MetalRuntime.swift:5-893).
 *
 * Conventions (shared by every entry point):
 *   - Every function returns 0 on success or a negative DGEN_HIP_E_* code.
 *     Nothing aborts across the ABI; the message of the last failure on the
 *     calling thread is returned by dgen_hip_last_error().
 *   - Offsets and lengths are in floats (4-byte cells) of the arena.
 *   - One context per thread; calls on one context must be serialised
 *     (the reference is single-threaded per graph, LazyGraph.swift:255).
 *   - No torch or HIP types appear in this header.
 */
#ifndef DGEN_HIP_H
#define DGEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DGEN_HIP_ABI_VERSION 2

/* ---- status codes ------------------------------------------------------ */
#define DGEN_HIP_OK 0
#define DGEN_HIP_E_INVALID (-1)   /* bad argument / shape / offset        */
#define DGEN_HIP_E_DEVICE (-2)    /* HIP runtime error                    */
#define DGEN_HIP_E_STATE (-3)     /* call out of order (e.g. run before configure) */
#define DGEN_HIP_E_RANGE (-4)     /* frame count not runnable, cell out of arena */
#define DGEN_HIP_E_NOMEM (-5)     /* device or pinned allocation failed   */

typedef struct dgen_hip_ctx dgen_hip_ctx;

/* Loss-mode bits of DGEN_HIP_K_SPECTRAL_LOSS (spectralLossFFT's options,
 * HigherOps.swift:49-65): the magnitude term's and the log-magnitude term's
 * lossMode .l2 (else .l1), and useSmoothLogMagnitude for the log term
 * (0.5 log(|X|^2 + eps^2)).  useHannWindow: false is the window of the FFT
 * tables (DGEN_HIP_K_FFT_TABLES arg[2]). */
#define DGEN_HIP_MSS_L2_LIN 1
#define DGEN_HIP_MSS_L2_LOG 2
#define DGEN_HIP_MSS_SMOOTH_LOG 4

/* ---- kernel classes ----------------------------------------------------
 * Argument meaning per class is documented at each class below.
 * "cell" = arena offset in floats; "n" = element count.                   */
enum dgen_hip_kernel {
  /* Accumulator table (static block): out[t] = min(max(accum_t, lo), hi),
   * accum_t the pre-increment output of u_accum(step, reset 0, min, max)
   * evaluated sequentially in fp32 (Definitions.swift:215-246).
   * arg: [0]=out cell [1]=frames   farg: [0]=step [1]=min [2]=max [3]=lo [4]=hi */
  DGEN_HIP_K_ACCUM_TABLE = 1,

  /* First MLP layer for a small fan-in: H = tanh(X W + b).
   * arg: [0]=X [1]=W [2]=b [3]=H (cells) [4]=rows [5]=fan_in [6]=width */
  DGEN_HIP_K_DENSE_SMALL = 2,

  /* MFMA GEMM  C[M][N] = op(A) op(B) with fused epilogue, fp32 results.
   * arg: [0]=A [1]=B [2]=C [3]=M [4]=N [5]=K [6]=lda [7]=ldb [8]=ldc
   *      [9]=a_layout (0: A stored [M][K], 1: A stored [K][M])
   *      [10]=b_layout (0: B stored [K][N], 1: B stored [N][K])
   *      [11]=epilogue (DGEN_HIP_EPI_*) [12]=bias cell (-1 none)
   *      [13]=aux cell (tanh output for EPI_TANH_GRAD, -1 none) [14]=ld aux
   *      [15]=split_k (1 = none; >1: partial sums in [16]) [16]=workspace cell
   *      [17]=column-partials cell or -1: with EPI_TANH_GRAD and no split,
   *           tile t (t < ceil(M/128)) covers output rows [128t, 128t+128)
   *           and writes nw+1 rows of N partials at row t*(nw+1): for
   *           q < nw the sums over its rows r of X[r][q]*C[r][n], then the
   *           plain column sums, so the weight and bias gradients of a
   *           layer fed by X are a reduction over ceil(M/128) rows instead
   *           of M (DGEN_HIP_K_COLSUM on the cell)
   *      [18]=X cell ([M][nw], read when nw > 0) [19]=nw (0..4)
   *      [20]=products: 0 fp32 matrix cores (v_mfma_f32_32x32x2_f32),
   *           1 split bf16: each operand value split into three bfloat16
   *           parts and the six partial products of significance down to
   *           2^-16 accumulated in fp32 (v_mfma_f32_32x32x16_bf16), as
   *           accurate as fp32 products
   *      [21]=with products 1 only: B planes cell or -1 (op(B) already
   *           split, [K][N] view, DGEN_HIP_K_SPLIT_BF16; B itself and its
   *           stride are then not read); not read with products 0 */
  DGEN_HIP_K_GEMM = 3,

  /* Head activations of HarmonicDecoderModel (Model.swift:100-114):
   * amps = softplus/sum, gain/noise gain = softplus, taps = tanh/sum|.|.
   * arg: [0]=Z [1]=ctrl [2]=rows [3]=K (<= 256) [4]=NF (<= 256)
   *      [5]=row stride of Z and ctrl (>= K + 2 + NF) */
  DGEN_HIP_K_HEADS_FWD = 4,

  /* Sequential tensor-phasor carry pass (Emit+State.swift:322-369) for
   * lanes (b,k), freq = (k+1) * f0 frames[b][t]; stores the phase at the
   * start of every 64-frame segment.
   * arg: [0]=f0 frames cell ([B][T], from DGEN_HIP_K_LERP_FRAMES)
   *      [1]=checkpoints cell ([nseg][B][K]) [2]=B [3]=K (<= 256) [4]=T
   *      [5]=timer cell, read only if [6] == 1 [6]=1: the timed build,
   *      which writes per workgroup (g, b) at [(g*B + b)*8] eight uint64:
   *      the chain wave's and the first producer wave's summed barrier
   *      waits (shader-clock cycles), the chain's first and last cycle
   *      stamps, the matching 100 MHz real-time stamps, the interval count
   *      and 0 (0 leaves it out: the timer has no counterpart in the
   *      reference; it measures the chain)
   * farg: [0]=sample rate */
  DGEN_HIP_K_PHASOR_CARRY = 5,

  /* Batched harmonic + FIR-noise synth forward
   * (Examples/HarmonicE2E/Synth.swift:47-102).
   * arg: [0]=ctrl ([B*F][ldc]) [1]=f0 frames ([B][T]) [2]=uv frames ([B][T])
   *      [3]=lerp table ([T][8]) [4]=checkpoints [5]=y ([B][T]) [6]=B
   *      [7]=K (<= 256) [8]=NF (K + 2 + NF <= 512) [9]=F [10]=T
   *      [11]=segment length (64) [12]=per-frame tape ([3][B][T]: harmonic
   *      sum, normaliser, FIR output) or -1 [13]=noise ([T]) [14]=ldc
   *      [15]=segment rows ([nseg][4])
   * farg: [0]=sample rate [1]=harmonic scale [2]=noise scale */
  DGEN_HIP_K_SYNTH_FWD = 6,

  /* Multi-scale batched spectral loss and its gradient, every FFT size in
   * one launch (Emit+SpectralLoss.swift:719-1235).  Sizes are powers of two
   * in [64, 2048] with hop N/4.  Each workgroup owns a 4096-sample tile of
   * one lane; the tile's dx (samples a-2047 .. a+4095) goes to the tile
   * partials, the per-window (lin, log) sums to the window-loss cells.
   * arg: [0]=x ([B][T]) [1]=target ([B][T]) [2]=tile partials
   *      ([B][ceil(T/4096)][6143]) [3]=B [4]=T [5]=n_sizes [6..13]=N_s
   *      [14..21]=window-loss cells ([ceil(T/hop)][B][2])
   *      [22..29]=FFT tables (DGEN_HIP_K_FFT_TABLES output, 3N-2 floats: the
   *      window and the transforms' twiddles)
   *      [30]=loss mode: DGEN_HIP_MSS_* bits (0: the trainer's L1 terms on
   *      magnitude and log(magnitude + 1e-8))
   * farg: [0]=lin upstream grad per window (w_lin/nsizes/maxFrames/B)
   *       [1]=log upstream grad per window */
  DGEN_HIP_K_SPECTRAL_LOSS = 7,

  /* dx from the spectral-loss tile partials (owning tile + next tile's
   * halo) and the per-frame loss signal (batch mean, / maxFrameCount).
   * arg: [0]=dx ([B][T]) or -1 [1]=loss frames ([T]) or -1 (not both -1)
   *      [2]=B [3]=T
   *      [4]=n_sizes [5..12]=N_s [13]=tile partials [21..28]=window-loss cells
   *      [29]=x [30]=target ([B][T]; read only when farg[3] != 0)
   * farg: [0]=lin weight per size [1]=log weight per size [2]=maxFrameCount
   *       [3]=weight of the time-domain term w sum_b (x - target)^2 / B per
   *       frame (the trainer's mseLossWeight, Trainer.swift:547-551; its
   *       gradient 2 w (x - target) / B joins dx) or 0 */
  DGEN_HIP_K_SPECTRAL_GATHER = 8,

  /* Synth backward.  A workgroup owns a run of 4 consecutive segments of a
   * lane and sums its segments' row-slot gradients per control row in LDS:
   * rows whose listed (segment, slot) entries all lie in the run are
   * written to d ctrl; a row shared with other runs leaves one partial per
   * run, at the run's index among the row's runs.
   * arg: as DGEN_HIP_K_SYNTH_FWD with [5]=dy ([B][T]) [12]=boundary partials
   *      cell ([B][F][6][ldc]) [16]=the forward's per-frame tape [17]=run
   *      table (DGEN_HIP_K_RUN_TABLE) [18]=dctrl ([B*F][ldc])
   *      [19]=1 to form dy here, else 0 (dy read as given)
   *      [20]=spectral-loss tile partials ([B][ntiles][tile + halo] as
   *      DGEN_HIP_K_SPECTRAL_LOSS leaves them) [21]=prediction x ([B][T])
   *      [22]=target ([B][T]; read only when farg[3] != 0)
   * farg: as DGEN_HIP_K_SYNTH_FWD with [3]=weight of the time-domain term
   *       (its gradient 2 w (x - target) / B joins dy) or 0.
   * With [19]=1 each sample's d loss / d y (owning tile + next tile's halo,
   * plus the time-domain term) is summed as the segment reads it and also
   * stored to dy, so no DGEN_HIP_K_SPECTRAL_GATHER launch is needed. */
  DGEN_HIP_K_SYNTH_BWD = 9,

  /* d ctrl of the rows shared between synth-backward runs: their partials
   * added in run order (deterministic); a row no segment touches is zero.
   * Rows within one run are left as the synth backward wrote them.
   * arg: [0]=boundary partials [1]=row list [2]=dctrl [3]=B [4]=NC [5]=F
   *      [6]=T [7]=seg [8]=row stride [9]=Z cell or -1: with Z, the head
   *      backward of every row too (as DGEN_HIP_K_HEADS_BWD), into [10]=dZ,
   *      [11]=K [12]=NF (K + 2 + NF = NC) */
  DGEN_HIP_K_SYNTH_BWD_REDUCE = 10,

  /* Head backward: dZ from d ctrl and Z.  arg: [0]=Z [1]=dctrl [2]=dZ
   * [3]=rows [4]=K (<= 256) [5]=NF (<= 256) [6]=row stride (>= K + 2 + NF;
   * dZ's padding columns are written as zero) */
  DGEN_HIP_K_HEADS_BWD = 11,

  /* Column sums (bias gradients): out[n] = sum_m A[m][n], deterministic
   * two-stage order.  arg: [0]=A [1]=out [2]=M [3]=N [4]=lda [5]=workspace
   * cell (min(256, M/32) * N floats) */
  DGEN_HIP_K_COLSUM = 12,

  /* First-layer weight gradient for a small fan-in (<= 4): dW[i][j] =
   * sum_m X[m][i] dZ[m][j], and with [7] >= 0 the bias gradient
   * db[j] = sum_m dZ[m][j] from the same pass.  arg: [0]=X [1]=dZ [2]=dW
   * [3]=rows [4]=fan_in [5]=width [6]=workspace cell
   * (min(256, rows/32) * (fan_in+1) * width floats) [7]=db cell or -1 */
  DGEN_HIP_K_DENSE_SMALL_WGRAD = 13,

  /* Adam.step over a flat parameter blob (Optimizers.swift:164-204).
   * arg: [0]=params [1]=grads [2]=m [3]=v [4]=n [5]=step-counter cell
   * farg: [0]=lr [1]=beta1 [2]=beta2 [3]=eps */
  DGEN_HIP_K_ADAM = 14,

  /* Deterministic phasor bank -> sum -> one-pole (config 1).
   * arg: [0]=freqs [1]=amps [2]=out [3]=n_osc [4]=frames [5]=workspace cell
   * farg: [0]=sample rate [1]=pole */
  DGEN_HIP_K_OSC_BANK = 15,

  /* xorshift32 noise stream of a zeroed cell (CRenderer.swift:685-693), a
   * static table.  arg: [0]=out cell [1]=frames */
  DGEN_HIP_K_NOISE_TABLE = 16,

  /* Row schedule of a sampleRow read (Emit+RowSelection.swift:164-197) from a
   * playhead table, a static table set.  arg: [0]=playhead [1]=lerp ([T][8]:
   * lo, hi, frac, 1-frac, slot(lo), slot(hi), 0, 0) [2]=segment rows
   * ([nseg][4], 16-byte aligned) [3]=row entries ([F][16]) [4]=status flag
   * cell [5]=F [6]=T [7]=segment length [8]=workspace (nseg + F floats).
   * The flag is 0 when every segment touches <= 4 rows, every row has <= 16
   * (segment, slot) entries and the playhead is finite; else the largest of
   * 1, 2, 3 for those three conditions. */
  DGEN_HIP_K_ROW_SCHEDULE = 17,

  /* Radix-2 spectral-loss tables for one FFT size (HigherOps.swift:69-99):
   * window[N] | twre[N-1] | twim[N-1].  arg: [0]=out cell [1]=N [2]=window:
   * 0 the symmetric Hann, 1 all ones (useHannWindow: false) */
  DGEN_HIP_K_FFT_TABLES = 18,

  /* Frame-rate sampleRow read of a [F][B] data table through a lerp table
   * (Emit+RowSelection.swift:164-197): out[b][t] = (1-frac) src[lo][b] +
   * frac src[hi][b].  arg: [0]=src [1]=lerp ([T][8]) [2]=out ([B][T]) [3]=B
   * [4]=F [5]=T */
  DGEN_HIP_K_LERP_FRAMES = 19,

  /* ---- tensor biquad bank (HigherOps.swift:401-570, RBJ low-pass, mode 0,
   * gain 1, coefficients recomputed every frame from cutoff base[k]*mod[n]
   * and Q[k]).  x, y, target: [T][B]; params: [2][B] = base | Q; mod: [T] or
   * -1 (unmodulated).  Time is cut into C = ceil(T/L) chunks of L frames.
   *
   * Forward part 1: per (lane, chunk) the zero-state response and the
   * responses to the unit initial states, summary [C][6][B] in fp64 (12*C*B
   * floats, even cell offset).
   * arg: [0]=x [1]=mod [2]=params [3]=summary [4]=B [5]=T [6]=L */
  DGEN_HIP_K_BIQUAD_CHUNK = 20,

  /* Compose the fp64 chunk summaries per lane (ascending chunks, or
   * descending when reverse = 1, for the adjoint): init [C][2][B] (fp32) =
   * the state entering each chunk.  Any two-cell affine chunk maps in this
   * layout compose here (the SVF bank's too).
   * arg: [0]=summary [1]=init [2]=B [3]=C [4]=reverse */
  DGEN_HIP_K_BIQUAD_CARRY = 21,

  /* Forward part 2: each chunk re-run from its initial state; writes y and,
   * when a target is given, per-chunk partial sums of (y - target)^2.
   * arg: [0]=x [1]=mod [2]=params [3]=init [4]=y [5]=B [6]=T [7]=L
   *      [8]=target or -1 [9]=loss partials [C][B] (with a target) or -1
   *      [10]=adjoint summary cell when [11]=1 (with a target): the chunk
   *      summaries DGEN_HIP_K_BIQUAD_ADJ_CHUNK would write, accumulated
   *      forwards during the replay (that op is then not needed) */
  DGEN_HIP_K_BIQUAD_FWD = 22,

  /* BPTT part 1 (BPTTEmission.swift:133-160): per (lane, chunk), the reverse
   * adjoint recurrence's zero-carry result and its responses to the unit
   * carries, summary [C][6][B] fp64 (then DGEN_HIP_K_BIQUAD_CARRY, reverse 1).
   * arg: [0]=mod [1]=params [2]=y [3]=target [4]=summary [5]=B [6]=T [7]=L */
  DGEN_HIP_K_BIQUAD_ADJ_CHUNK = 23,

  /* BPTT part 2: each chunk's adjoint from its carry, chained through the
   * coefficients to per-chunk gradient partials [C][2][B] (d/d base,
   * d/d Q), summed over chunks by DGEN_HIP_K_COLSUM.
   * arg: [0]=x [1]=mod [2]=params [3]=y [4]=target [5]=adjoint init
   *      [6]=grad partials [7]=B [8]=T [9]=L */
  DGEN_HIP_K_BIQUAD_BWD = 24,

  /* ---- hop-gated STFT round trip (bufferView -> * window -> tensorFFT ->
   * per-bin gains -> tensorIFFT -> overlapAdd; HigherOps.swift:738-813,
   * HigherOps+FFT.swift:16-123, Emit+FFT.swift:6-62).  x, y, dy: [S][T];
   * window: [N] (N a power of two in [64, 2048]); gains: [N/2+1] applied to
   * bins k and N-k; hop H in [1, N].
   *
   * Forward: y, dL/dy = 2 (y - x)/T and per-8192-sample-tile loss partials
   * sum (y - x)^2 / T.  arg: [0]=x [1]=window [2]=gains [3]=y or -1
   * [4]=dy or -1 [5]=loss partials ([S][ceil(T/8192)]) or -1 [6]=S [7]=T
   * [8]=N [9]=H */
  DGEN_HIP_K_STFT_FWD = 25,

  /* Gain gradient partials: row (s, b) sums (c_k/N) Re(X_k conj(E_k)) over
   * a run of 8*4096/N windows of signal s (X: window spectrum, E: spectrum
   * of dy over the window's outputs, c_k = 1 at k = 0, N/2, else 2); the
   * rows are reduced by DGEN_HIP_K_COLSUM.  arg: [0]=x [1]=window [2]=dy
   * [3]=grad partials ([S][nblk][N/2+1], nblk = ceil(ceil(T/H) / (8*4096/N)))
   * [4]=S [5]=T [6]=N [7]=H */
  DGEN_HIP_K_STFT_BWD = 26,

  /* ---- 2D membrane (Examples/BendingMetal/main.swift:96-169 idiom):
   * u_{n+1} = 2u_n - u_{n-1} + c2 L(u_n) - d (u_n - u_{n-1}), L the 3x3
   * zero-padded Laplacian, u_{-1} = u_0; pickup out[n] = u_{n+1}[py][px].
   * states: [(T+2)][R][C] with S[0] = u_{-1}, S[1] = u_0, S[n+1] = u_n;
   * params: (c2, d).  Time-blocked: one launch per `steps` (<= 16) frames.
   *
   * Forward: copies u0 into S[0], S[1], then fills S and the pickup.
   * arg: [0]=states [1]=u0 ([R][C]) [2]=params [3]=pickup ([T]) [4]=R [5]=C
   *      [6]=T [7]=py [8]=px [9]=steps per launch */
  DGEN_HIP_K_MEMBRANE_FWD = 27,

  /* Discrete adjoint of the forward against a target pickup series: the
   * gradient (d/d c2, d/d d), accumulated in fp64 per 32x32 tile and wave
   * ([ceil(R/32)*ceil(C/32)][16][2] doubles, even cell offset; zeroed by
   * the call) and summed in a fixed order, and the loss terms
   * (out - tgt)^2 ([T]).
   * arg: [0]=states [1]=params [2]=pickup [3]=target ([T]) [4]=adjoint
   *      boundary fields ([4][R][C]) [5]=grad partials [6]=loss terms
   *      [7]=R [8]=C [9]=T [10]=py [11]=px [12]=steps per launch [13]=grads */
  DGEN_HIP_K_MEMBRANE_BWD = 28,

  /* ---- streaming classes (dgen_hip_process_v1 / dgen_hip_run with
   * preserved state, Realize.swift:553-563).  A run of frame_count frames
   * processes frames [0, frame_count) of the op's cells (any frame_count up
   * to the op's frames) and carries the graph's state cells to the next run;
   * a DGEN_HIP_PROCESS_RESET call starts from zero state.  Any split of a
   * signal into runs gives the same samples.
   *
   * Oscillator bank -> sum -> history one-pole (config 1), frame-sequential
   * like the C backend: arg: [0]=freqs [1]=amps [2]=out [3]=n_osc (<= 64)
   * [4]=frames [5]=state (n_osc phases, then y[n-1]) [6]=stateful (0:
   * Signal.phasor(Tensor), the deterministic phasor of the frame index within
   * the run, Emit+State.swift:370-387; 1: stateful u_phasor accumulators,
   * Definitions.swift:96-102)   farg: [0]=sample rate [1]=pole */
  DGEN_HIP_K_STREAM_OSC_BANK = 29,

  /* Tensor biquad bank, one lane per thread, Direct Form I history in the
   * state cell ([4][B]: x[n-1], x[n-2], y[n-1], y[n-2]); coefficients as
   * DGEN_HIP_K_BIQUAD_*.  arg: [0]=x ([frames][B]) [1]=mod ([frames]) or -1
   * [2]=params ([2][B] base | Q) [3]=state [4]=y ([frames][B]) [5]=B
   * [6]=frames */
  DGEN_HIP_K_STREAM_BIQUAD = 30,

  /* ---- temporal gradient of stateful accumulators (phasor, accum):
   * temporalIncrementGradient, Gradients.swift:209-261, and its three-phase
   * emission, Emit+TemporalGradient.swift:15-105.  The reset-aware exclusive
   * suffix scan of the output gradient, per element, from the last frame
   * down: active = reset[n] > 0 ? 0 : carry; out[n] = active (/ sample rate
   * for a phasor); carry = g[n] + active.  Chunked in time (the carries
   * between 256-frame chunks are reassociated).
   * arg: [0]=g ([T][E]) [1]=reset ([T]) or -1 [2]=out ([T][E]) [3]=E [4]=T
   *      [5]=workspace (2*C*E + C floats, C = ceil(T/256)) [6]=divide by the
   *      sample rate (0/1)   farg: [0]=sample rate */
  DGEN_HIP_K_TEMPORAL_GRAD_SCAN = 31,

  /* Swept-phasor bank forward and loss (TemporalGradientTests.swift:24-60),
   * one lane per thread: f[n] = base + slope[e] * time[n], the stateful
   * phasor of f with reset, mse of the phase (or, smooth, of sin(2 pi
   * phase)) against target: loss partials per lane and the upstream gradient.
   * arg: [0]=slope ([E]) [1]=time ([T]) [2]=reset ([T]) or -1 [3]=phase
   *      ([T][E]) or -1 [4]=upstream ([T][E]) [5]=loss partials ([E]) [6]=E
   *      [7]=T [8]=smooth (0/1)
   * farg: [0]=sample rate [1]=base frequency [2]=target */
  DGEN_HIP_K_SWEPT_PHASOR = 32,

  /* ---- ZDF state-variable filter bank (low-pass): the two-cell
   * Cytomic/TPT SVF of SVFBPTTScratchTests.swift:21-34 per lane, cutoff
   * fc = clip(base[k] * mod[n] + env[n], 20, 20000) (mod, env optional
   * [T] signals), g = tan((pi fc) / sr), kDamp = 1 / res[k], saturation
   * s = ic / (1 + |kSat[k] ic|).  x, y, target: [T][B]; cells: [2][T][B]
   * (ic1 | ic2 entering every frame); params [P][B] = base | res (P = 2,
   * kSat the constant 0) or base | res | kSat (P = 3).  Every class takes
   * farg[0] = sample rate (the run's host rate when one is set).
   *
   * Linear forward part 1: per (lane, chunk of L frames) the chunk's
   * zero-state result and unit-state responses as fp64 affine maps,
   * summary [C][6][B] (C = ceil(T/L)); then DGEN_HIP_K_BIQUAD_CARRY.
   * arg: [0]=x [1]=mod or -1 [2]=env or -1 [3]=params (P = 2) [4]=summary
   *      [5]=B [6]=T [7]=L */
  DGEN_HIP_K_SVF_CHUNK = 33,

  /* Linear forward part 2: each chunk re-run from its state: y, the cells
   * (or -1), per-chunk loss partials sum (y - target)^2 (with a target).
   * arg: [0]=x [1]=mod [2]=env [3]=params (P = 2) [4]=init ([C][2][B])
   *      [5]=y [6]=cells or -1 [7]=target or -1 [8]=loss partials ([C][B])
   *      or -1 [9]=B [10]=T [11]=L
   *      [12]=adjoint summary cell when [13]=1 (with a target): the chunk
   *      summaries DGEN_HIP_K_SVF_ADJ_CHUNK would write for the linear bank,
   *      accumulated forwards during the replay (that op is then not needed) */
  DGEN_HIP_K_SVF_FWD = 34,

  /* Saturating forward (P = 3), one lane per thread over all frames (the
   * reference's per-lane frame loop); loss partials per L-frame chunk.
   * arg: [0]=x [1]=mod [2]=env [3]=params [4]=state ([2][B]) or -1 [5]=y
   *      [6]=cells or -1 [7]=target or -1 [8]=loss partials or -1 [9]=B
   *      [10]=T [11]=L [12]=sanitize (non-finite out stores -> 0)
   *      [13]=coefficient tape ([T][B]: g, filled by the call before the
   *      sequential loop reads it) or -1 (evaluated in the loop)
   * With a target, cells and a tape, B a multiple of 64 and T and L of 32,
   * the loop runs on 32-frame LDS tiles (the same results). */
  DGEN_HIP_K_SVF_SEQ = 35,

  /* BPTT part 1: per (lane, chunk), reverse, the cells' adjoint from a zero
   * carry under the loss 2 (y - target) and its unit-carry responses
   * (fp64, summary [C][6][B]; then DGEN_HIP_K_BIQUAD_CARRY, reverse 1).
   * arg: [0]=mod [1]=env [2]=params [3]=y [4]=target [5]=cells (required
   *      when saturating) or -1 [6]=summary [7]=B [8]=T [9]=L
   *      [10]=saturating (0/1) */
  DGEN_HIP_K_SVF_ADJ_CHUNK = 36,

  /* BPTT part 2: each chunk's adjoint from its carry, chained through the
   * coefficient nodes to gradient partials [C][P][B] (d/d base, d/d res,
   * d/d kSat) for DGEN_HIP_K_COLSUM, and (optional) d loss / d x.
   * arg: [0]=x [1]=mod [2]=env [3]=params [4]=y [5]=target [6]=cells
   *      [7]=adjoint init ([C][2][B]) [8]=grad partials [9]=xbar ([T][B])
   *      or -1 [10]=B [11]=T [12]=L [13]=saturating (0/1) */
  DGEN_HIP_K_SVF_BWD = 37,

  /* Streaming SVF bank: DGEN_HIP_K_SVF_SEQ's arguments with a state cell,
   * no cells and no loss; a run processes frames [0, frame_count) and
   * carries ic1, ic2 to the next (zero after a reset). */
  DGEN_HIP_K_STREAM_SVF = 38,

  /* Split of an fp32 matrix into three bfloat16 planes for the split-bf16
   * GEMM (DGEN_HIP_K_GEMM arg[21]): value (k, n) at src[k*ld_k + n*ld_n]
   * goes to plane p (p = 0..2: x = h + m + l, h = bf16(x), m = bf16(x - h),
   * l = bf16(x - h - m)) as bf16 element k%8 of 16-byte entry
   * (p*K8 + k/8)*N + n, K8 = ceil(K/8), zero for k >= K.  Done once for an
   * operand that many GEMM tiles share (the weights, per step).
   * arg: [0]=src [1]=planes cell (3*K8*N*4 floats, 16-byte aligned) [2]=K
   *      [3]=N [4]=ld_k [5]=ld_n [6]=K8 or 0 (ceil(K/8)): more groups pad
   *      the planes with zeros, for a GEMM whose K runs past the source's */
  DGEN_HIP_K_SPLIT_BF16 = 39,

  /* One generic UOp block (dgen_hip_set_blocks): the kernel the renderer
   * generated for it, launched with its dispatch mode's grid
   * (DispatchMode.threadCount, Renderer.swift:71-86) for the run's frame
   * count.  Runs any frame_count up to arg[7].
   * arg: [0]=block index [1]=tape cell ([slots][frames], `t`) or -1
   *      [2]=tape slots [3]=outputs cell ([channels][frames]) or -1
   *      [4]=output channels [5]=inputs cell ([channels][frames]) or -1
   *      [6]=input channels [7]=frames the tape/outputs/inputs cells hold
   * farg: [0]=the graph's sample rate (the hostSampleRate UOp; a run's host
   *       rate replaces it) */
  DGEN_HIP_K_UOP_BLOCK = 40,

  /* Row table of the synth backward's runs of 4 segments, a static table:
   * per run, {rows, 0, 0, 0} then per control row its segments touch
   * {row, before | outside << 8 | n << 16, entries lo, hi} (where the run's
   * sum of the row goes, and the run's n (segment, slot) entries of the row
   * in list order, 4 bits each).
   * arg: [0]=segment rows ([nseg][4]) [1]=row list ([F][16], both from
   *      DGEN_HIP_K_ROW_SCHEDULE) [2]=table (ceil(nseg/4) x 17 x 4 floats,
   *      16-byte aligned) [3]=nseg [4]=F */
  DGEN_HIP_K_RUN_TABLE = 41,
};

/* GEMM epilogues */
enum dgen_hip_epilogue {
  DGEN_HIP_EPI_NONE = 0,       /* C = acc                                   */
  DGEN_HIP_EPI_BIAS = 1,       /* C = acc + bias[n]                         */
  DGEN_HIP_EPI_BIAS_TANH = 2,  /* C = tanh(acc + bias[n])                   */
  DGEN_HIP_EPI_TANH_GRAD = 3,  /* C = acc * (1 - aux[m][n]^2)               */
};

/* op flags */
#define DGEN_HIP_OP_STATIC 1u /* run once, at configure (static temporality) */
#define DGEN_HIP_OP_SIDE 2u   /* launch on the side stream (overlaps stream 0) */
#define DGEN_HIP_OP_JOIN 4u   /* stream 0 waits for the side stream first    */
/* with SIDE: the side stream first waits for the stream-0 work enqueued
 * before this op (a fork point); without it, side ops wait only for the
 * start of the run */
#define DGEN_HIP_OP_FORK 8u

#define DGEN_HIP_OP_NARG 32
#define DGEN_HIP_OP_NFARG 8

typedef struct dgen_hip_op {
  uint32_t kernel; /* enum dgen_hip_kernel */
  uint32_t flags;  /* DGEN_HIP_OP_* */
  int64_t arg[DGEN_HIP_OP_NARG];
  float farg[DGEN_HIP_OP_NFARG];
} dgen_hip_op;

/* ---- generic UOp blocks ------------------------------------------------
 * The compiler's fused blocks as it hands them to a renderer: BlockUOps
 * (Renderer.swift:3-24) = UOps (UOps.swift:17-138) + frame order + temporality
 * + dispatch mode.  dgen_hip_set_blocks renders them to HIP C++ the way the
 * Metal renderer renders MSL (prepareSchedule's range guard, frame loop and
 * hop check, MetalRenderer.swift:787-938; per-UOp emission :1316-1720),
 * compiles them with hiprtc for the context's device and loads them; each
 * DGEN_HIP_K_UOP_BLOCK op of the schedule launches one.  This is the path for
 * blocks no kernel class pattern-matches. */

/* An operand (the reference's Lazy, UOps.swift:1-7). */
enum dgen_hip_lazy_kind {
  DGEN_HIP_LAZY_EMPTY = 0,
  DGEN_HIP_LAZY_CONST = 1,      /* .constant: value */
  DGEN_HIP_LAZY_VAR = 2,        /* .variable: a kernel-local value, id = VarID */
  DGEN_HIP_LAZY_GLOBAL = 3,     /* .global / a variable in ctx.globals: id = its tape slot (getGlobalId) */
  DGEN_HIP_LAZY_FRAME_COUNT = 4 /* the variable -1: the run's frame count */
};
typedef struct dgen_hip_lazy {
  int32_t kind; /* enum dgen_hip_lazy_kind */
  int32_t id;
  float value;
  int32_t reserved;
} dgen_hip_lazy;

/* UOp operations, in the reference's order (Op, UOps.swift:17-138).  Cells,
 * channels, counts and steps go in imm[0] (threadgroupArrayDecl: imm[0] the
 * scratch id, imm[1] its size). */
enum dgen_hip_uop_op {
  DGEN_HIP_UOP_NOP = 0,          /* view ops and markers: no code */
  DGEN_HIP_UOP_LOAD = 1,         /* value = memory[imm0] */
  DGEN_HIP_UOP_STORE,            /* memory[imm0] = a */
  DGEN_HIP_UOP_DELAY1,           /* value = memory[imm0]; memory[imm0] = a */
  DGEN_HIP_UOP_MUTATE,           /* a = b */
  DGEN_HIP_UOP_ADD, DGEN_HIP_UOP_SUB, DGEN_HIP_UOP_MUL, DGEN_HIP_UOP_DIV,
  DGEN_HIP_UOP_ABS, DGEN_HIP_UOP_SIGN, DGEN_HIP_UOP_SIN, DGEN_HIP_UOP_COS,
  DGEN_HIP_UOP_AND, DGEN_HIP_UOP_OR, DGEN_HIP_UOP_XOR,
  DGEN_HIP_UOP_TAN, DGEN_HIP_UOP_ATAN, DGEN_HIP_UOP_TANH, DGEN_HIP_UOP_EXP, DGEN_HIP_UOP_LOG,
  DGEN_HIP_UOP_LOG10, DGEN_HIP_UOP_SQRT, DGEN_HIP_UOP_POW, DGEN_HIP_UOP_ATAN2, DGEN_HIP_UOP_MOD,
  DGEN_HIP_UOP_GT, DGEN_HIP_UOP_GTE, DGEN_HIP_UOP_LTE, DGEN_HIP_UOP_LT, DGEN_HIP_UOP_EQ,
  DGEN_HIP_UOP_MIN, DGEN_HIP_UOP_MAX, DGEN_HIP_UOP_FLOOR, DGEN_HIP_UOP_CEIL, DGEN_HIP_UOP_ROUND,
  DGEN_HIP_UOP_NOISE,            /* xorshift32 on memory[imm0]'s bits, value in [0, 1) */
  DGEN_HIP_UOP_MEMORY_READ,      /* value = memory[imm0 + a] */
  DGEN_HIP_UOP_MEMORY_WRITE,     /* memory[imm0 + a] = b */
  DGEN_HIP_UOP_MEMORY_ACCUMULATE,/* atomic memory[imm0 + a] += b */
  DGEN_HIP_UOP_SIMD_BROADCAST_LOAD, /* as MEMORY_READ */
  DGEN_HIP_UOP_BROADCAST_SCALAR, /* value = a */
  DGEN_HIP_UOP_BEGIN_IF,         /* if (a) { */
  DGEN_HIP_UOP_GSWITCH,          /* value = a > 0 ? b : c */
  DGEN_HIP_UOP_SELECTOR,         /* value = options[ceil(a) - 1] (list), 0 outside */
  DGEN_HIP_UOP_END_IF,
  DGEN_HIP_UOP_DEFINE_GLOBAL,    /* a = the global (GLOBAL operand) this block defines */
  DGEN_HIP_UOP_LOAD_GLOBAL,      /* no code: globals are read through their operands */
  DGEN_HIP_UOP_BEGIN_LOOP,       /* for (i = 0; i < a; i += imm0 (1 if 0)), negative step reverses */
  DGEN_HIP_UOP_BEGIN_FOR_LOOP,   /* for (a = 0; a < b; a++), a a VAR operand */
  DGEN_HIP_UOP_BEGIN_REVERSE_LOOP, /* for (i = a - 1; i >= 0; i--) */
  DGEN_HIP_UOP_END_LOOP,
  DGEN_HIP_UOP_BEGIN_RANGE,      /* if (id >= a && id < b) { */
  DGEN_HIP_UOP_END_RANGE,
  DGEN_HIP_UOP_BEGIN_PARALLEL_RANGE, /* for (value = 0; value < imm0; value++) */
  DGEN_HIP_UOP_END_PARALLEL_RANGE,
  DGEN_HIP_UOP_SET_THREAD_COUNT_SCALE, /* no code (the dispatch mode carries it) */
  DGEN_HIP_UOP_SET_FRAME_INDEX,  /* the frame index of later outputs and tape accesses = a */
  DGEN_HIP_UOP_OUTPUT,           /* outputs[imm0][frame] = a (non-finite -> 0) */
  DGEN_HIP_UOP_INPUT,            /* value = inputs[imm0][frame] */
  DGEN_HIP_UOP_FRAME_COUNT,      /* value = frameCount (no code with an EMPTY value) */
  DGEN_HIP_UOP_HOST_SAMPLE_RATE, /* value = the run's host sample rate */
  DGEN_HIP_UOP_FRAME_INDEX,      /* value = the frame (thread in parallel blocks, loop index in sequential) */
  DGEN_HIP_UOP_THREAD_INDEX,     /* value = the thread index */
  DGEN_HIP_UOP_LOAD_TAPE,        /* value = tape a at frame b, 0 outside [0, frameCount) */
  DGEN_HIP_UOP_CAST,             /* value = (imm0 ? int : float) a */
  DGEN_HIP_UOP_IDENTITY,         /* value = a */
  DGEN_HIP_UOP_DECLARE_VAR,      /* value = a */
  DGEN_HIP_UOP_BEGIN_HOP_CHECK,  /* if (a == 0) { */
  DGEN_HIP_UOP_END_HOP_CHECK,
  DGEN_HIP_UOP_THREADGROUP_ARRAY_DECL, /* __shared__ float scratch_imm0[imm1] */
  DGEN_HIP_UOP_THREADGROUP_READ, /* value = scratch_imm0[a] */
  DGEN_HIP_UOP_THREADGROUP_WRITE,/* scratch_imm0[a] = b */
  DGEN_HIP_UOP_THREADGROUP_BARRIER
};

typedef struct dgen_hip_uop {
  int32_t op;        /* enum dgen_hip_uop_op */
  int32_t int_typed; /* UOp.scalarType == .int: the value is declared int */
  dgen_hip_lazy value;
  dgen_hip_lazy a, b, c;
  int64_t imm[2];
  const dgen_hip_lazy* list; /* SELECTOR options */
  uint32_t n_list;
  uint32_t reserved;
} dgen_hip_uop;

/* DispatchMode (Renderer.swift:26-67), without the GEMM modes. */
enum dgen_hip_dispatch {
  DGEN_HIP_DISPATCH_SINGLE_THREADED = 0,     /* 1 thread, frame loop */
  DGEN_HIP_DISPATCH_PER_FRAME = 1,           /* frameCount threads */
  DGEN_HIP_DISPATCH_PER_FRAME_SCALED = 2,    /* frameCount * n threads */
  DGEN_HIP_DISPATCH_FIXED_WITH_FRAME_LOOP = 3, /* n threads, each loops over the frames */
  DGEN_HIP_DISPATCH_STATIC_THREADS = 4,      /* n threads, no frame loop */
  DGEN_HIP_DISPATCH_SELF_MANAGED = 5,        /* 1 thread, the block's own loops */
  DGEN_HIP_DISPATCH_SELF_MANAGED_THREADS = 6,/* n threads, the block's own loops */
  DGEN_HIP_DISPATCH_PER_FRAME_TG1 = 7,       /* frameCount threads, groups of 1 */
  DGEN_HIP_DISPATCH_PER_FRAME_SCALED_TG1 = 8 /* frameCount * n threads, groups of 1 */
};
enum { DGEN_HIP_FRAME_SEQUENTIAL = 0, DGEN_HIP_FRAME_PARALLEL = 1 };
enum { DGEN_HIP_TEMPORAL_FRAME = 0, DGEN_HIP_TEMPORAL_HOP = 1, DGEN_HIP_TEMPORAL_STATIC = 2 };

typedef struct dgen_hip_block {
  int32_t dispatch;    /* enum dgen_hip_dispatch */
  int32_t dispatch_n;  /* n of the scaled / fixed / static / self-managed-threads modes */
  int32_t frame_order; /* DGEN_HIP_FRAME_* */
  int32_t temporality; /* DGEN_HIP_TEMPORAL_* */
  int32_t hop_size;
  int32_t reserved;
  dgen_hip_lazy hop_counter; /* hop-based: the counter value (runs where it is 0) */
  const dgen_hip_uop* ops;
  uint32_t n_ops;
  uint32_t reserved2;
} dgen_hip_block;

typedef struct dgen_hip_kernel_time {
  uint32_t index;  /* position in the schedule */
  uint32_t kernel; /* enum dgen_hip_kernel */
  float gpu_ms;    /* hipEvent time of the op's launches */
} dgen_hip_kernel_time;

/* ---- runtime ----------------------------------------------------------- */

/* ABI version (DGEN_HIP_ABI_VERSION) and the device count. No device init
 * beyond hipGetDeviceCount. */
int dgen_hip_abi_version(void);
int dgen_hip_device_count(int* out);

/* Create a context on `device`: streams and events; no arena yet.
 * Mirrors MetalCompiledKernel.init (MetalRuntime.swift:30-206). */
int dgen_hip_create(int device, dgen_hip_ctx** out);
/* Release everything the context owns (MetalRuntime.swift:572-588). */
int dgen_hip_destroy(dgen_hip_ctx* ctx);
/* Message of the last failing call on this thread ("" if none). */
const char* dgen_hip_last_error(void);

/* Allocate the device arena (memory_floats floats, zeroed) and its pinned
 * host mirror, copy the schedule (the caller keeps ownership of `ops`),
 * validate every op's cells against the arena, and run the STATIC ops.
 * Mirrors initializeBuffers + kernel creation (MetalRuntime.swift:221-254).
 * max_frames bounds dgen_hip_run's frame_count (maxFrameCount). */
int dgen_hip_configure(dgen_hip_ctx* ctx, const dgen_hip_op* ops, uint32_t n_ops, uint64_t memory_floats,
                       uint32_t max_frames);

/* Render, compile (hiprtc, gfx950) and load the context's generic UOp
 * blocks; DGEN_HIP_K_UOP_BLOCK op arg[0] indexes them.  Replaces the blocks
 * set before.  Call before dgen_hip_configure (configure checks the ops that
 * name a block).  A block that does not render or compile fails with
 * DGEN_HIP_E_INVALID and the compiler's log in dgen_hip_last_error().
 * Compiled code objects are cached per process by source text. */
int dgen_hip_set_blocks(dgen_hip_ctx* ctx, const dgen_hip_block* blocks, uint32_t n_blocks);
/* The HIP C++ source dgen_hip_set_blocks would compile for these blocks,
 * without a context or a device: writes up to cap bytes (NUL-terminated) to
 * buf and the full length to *len.  With compile != 0 it also compiles the
 * source with hiprtc (no device needed) and fails with the log on errors. */
int dgen_hip_render_blocks(const dgen_hip_block* blocks, uint32_t n_blocks, int compile, char* buf, size_t cap,
                           size_t* len);

/* Host mirror of the arena (LazyRuntime.memoryPointer, Realize.swift:16).
 * Valid until the next configure/destroy. */
float* dgen_hip_host_memory(dgen_hip_ctx* ctx);
/* Copy [off, off+n) host mirror -> device now (injectTensorData,
 * Realize.swift:257-282). */
int dgen_hip_upload(dgen_hip_ctx* ctx, uint64_t off, uint64_t n);
/* Copy [off, off+n) device -> host mirror now (readOutputs / readGradients,
 * Realize.swift:298-306, Backward.swift:132-165). */
int dgen_hip_download(dgen_hip_ctx* ctx, uint64_t off, uint64_t n);
/* Zero [off, off+n) on the device (n = 0: the whole arena); mirrors
 * zeroAllBuffers (MetalRuntime.swift:265-281). */
int dgen_hip_zero(dgen_hip_ctx* ctx, uint64_t off, uint64_t n);

/* Enqueue every non-static op in schedule order and wait for completion
 * (runNoCopy -> run, MetalRuntime.swift:283-342,676-698: synchronous on
 * return); then the output cells (dgen_hip_set_outputs) are copied to the
 * host mirror.
 * frame_count must lie in [1, max_frames].  Each op is rendered for a frame
 * count (its frame argument): the oscillator bank runs the first frame_count
 * frames of it (the reference's kernels loop over [0, frameCount) of cells
 * sized for maxFrameCount), every other frame-indexed class only the exact
 * count it was rendered for (its static tables, tiles and loss normalisation
 * are laid out for that count).  Any other frame_count fails with
 * DGEN_HIP_E_RANGE before anything is enqueued. */
int dgen_hip_run(dgen_hip_ctx* ctx, uint32_t frame_count);
/* As dgen_hip_run but returns without waiting: dgen_hip_sync waits for the
 * run and then copies the declared output cells to the host mirror, so
 * dgen_hip_host_outputs is current after the sync (not before it). */
int dgen_hip_run_async(dgen_hip_ctx* ctx, uint32_t frame_count);
int dgen_hip_sync(dgen_hip_ctx* ctx);

/* Declare the output cells [off, off+n) of the schedule: every dgen_hip_run
 * (and the dgen_hip_sync after a dgen_hip_run_async) copies them to the host
 * mirror after the run, and dgen_hip_host_outputs
 * returns where they are (LazyRuntime.outputsPointer, Realize.swift:17;
 * MetalCompiledKernel's host-visible outputs buffer, MetalRuntime.swift:
 * 232-254).  n = 0 declares none.  Reset by dgen_hip_configure. */
int dgen_hip_set_outputs(dgen_hip_ctx* ctx, uint64_t off, uint64_t n);
/* Host pointer of the declared output cells (NULL if none); *n_out (if not
 * NULL) receives their float count.  Valid until the next configure/destroy. */
float* dgen_hip_host_outputs(dgen_hip_ctx* ctx, uint64_t* n_out);

/* Host sample rate of later runs, in Hz: the divisor of every phase
 * increment (u_phasor divides by hostSampleRate, Definitions.swift:96-102;
 * the C backend reads it from DGenProcessContextV1.sample_rate,
 * CRenderer.swift:357-359, defaulting to the graph's rate,
 * Realize.swift:246-252).  Rates the graph itself fixes (the synth's
 * Nyquist mask, Synth.swift:158-167) keep the rendered value.  0 restores
 * the rate each op was rendered with; otherwise [1, 1e7].  Drops a captured
 * graph. */
int dgen_hip_set_sample_rate(dgen_hip_ctx* ctx, float sample_rate);

/* ---- streaming process calls (dgen_process_v1, dgen_runtime.h:252-291) -- */
typedef struct dgen_hip_process_context_v1 {
  uint32_t abi_version; /* DGEN_HIP_ABI_VERSION */
  uint32_t struct_size; /* sizeof(dgen_hip_process_context_v1) */
  float sample_rate;    /* host sample rate of this call (DGenProcessContextV1.sample_rate); 0: rendered */
  uint32_t flags;       /* DGEN_HIP_PROCESS_* */
} dgen_hip_process_context_v1;
#define DGEN_HIP_PROCESS_RESET 1u /* streaming classes start this call from zero state */

/* Declare the channels of dgen_hip_process_v1: input channel c's frame i is
 * written to cell in_cells[c] + i * in_strides[c], output channel c's frame i
 * read from out_cells[c] + i * out_strides[c] (a [frames][lanes] cell is one
 * channel per lane with stride lanes).  Every channel must fit max_frames
 * frames in the arena, and no two input channels may share a cell
 * (DGEN_HIP_E_INVALID).  Cells between the input ports that are not ports
 * (e.g. state a streaming class carries) keep their device values across a
 * process call.  Reset by dgen_hip_configure. */
int dgen_hip_set_process_ports(dgen_hip_ctx* ctx, uint32_t n_in, const uint64_t* in_cells, const uint32_t* in_strides,
                               uint32_t n_out, const uint64_t* out_cells, const uint32_t* out_strides);

/* One block of a streaming schedule (the reference's dgen_process_v1(inputs,
 * outputs, frame_count, state, context, host)): the input channels'
 * frame_count samples (host arrays) go to their cells, the per-run ops run
 * on frame_count frames, carrying their state cells from the previous call
 * (the context's state is the arena), and the output channels' samples come
 * back to the host arrays.  Synchronous.  context may be NULL (rendered
 * sample rate, no reset).  Ops are enqueued one by one (no graph replay). */
int dgen_hip_process_v1(dgen_hip_ctx* ctx, const float* const* inputs, float* const* outputs, uint32_t frame_count,
                        const dgen_hip_process_context_v1* context);

/* Bind the schedule the reference-named exports dgen_process_v1 /
 * dgen_set_param_value_v1 (dgen_process_v1.h) run: a configured context with
 * its process ports set, and the arena range [memory_off, memory_off +
 * memory_floats) that is the graph's memory -- the cells the reference keeps
 * in the host's state block (Runtime.swift:728-740): parameters, tensors and
 * every state cell a streaming class carries between calls.  The reference
 * loads one compiled graph per process-function library; here one context
 * is bound per process at a time.  ctx NULL unbinds.  The context must
 * outlive its binding (dgen_hip_destroy of the bound context unbinds it).
 * No counterpart in the reference beyond the library load it replaces. */
int dgen_hip_process_bind(dgen_hip_ctx* ctx, uint64_t memory_off, uint64_t memory_floats);
/* Floats of the state block dgen_process_v1 reads and writes:
 * max(memory_floats, 1024) of the bound schedule (the reference's
 * getMemorySize(), Runtime.swift:228-237, 728-730), 0 when nothing is bound. */
uint64_t dgen_hip_process_memory_size(void);

/* Graph replay of runs (enable != 0): the per-run schedule for a frame count
 * is captured once from both streams into a HIP graph and every later
 * dgen_hip_run / dgen_hip_run_async / dgen_hip_time_runs with that frame
 * count replays it with one launch, instead of enqueuing each kernel from
 * the host.  Kernel arguments are fixed at capture; dgen_hip_configure and
 * a change of frame count capture afresh.  dgen_hip_profile and
 * dgen_hip_time_op always launch op by op.  Waits for outstanding work.
 * The reference re-encodes its command buffers on every run
 * (MetalRuntime.swift:676-698, runNoCopy -> run); this is the MI355X launch
 * path for schedules of many short kernels (config 5: ~600 per step). */
int dgen_hip_set_graphs(dgen_hip_ctx* ctx, int enable);

/* Run once with a hipEvent pair around every op; fills up to `cap` entries
 * and sets *n_out.  Mirrors profileKernels (MetalRuntime.swift:397-425). */
int dgen_hip_profile(dgen_hip_ctx* ctx, uint32_t frame_count, dgen_hip_kernel_time* out, size_t cap,
                     size_t* n_out);

/* Time `iters` back-to-back runs (after `warmup` untimed runs) with one
 * hipEvent pair on stream 0; *ms_out = total milliseconds. */
int dgen_hip_time_runs(dgen_hip_ctx* ctx, uint32_t frame_count, int warmup, int iters, double* ms_out);

/* Run schedule op `op_index` alone, once, on the arena's current contents,
 * and wait: for measuring one op in isolation (its HBM traffic under a
 * counter profiler).  The reference has no counterpart; its profileKernels
 * (MetalRuntime.swift:397-425) times kernels inside a full run. */
int dgen_hip_run_op(dgen_hip_ctx* ctx, uint32_t frame_count, uint32_t op_index);

/* Average duration of the launches of schedule op `op_index` over `iters`
 * runs, timed with hipEvents recorded on the stream that op launches on. */
int dgen_hip_time_op(dgen_hip_ctx* ctx, uint32_t frame_count, uint32_t op_index, int iters, double* ms_out);

/* Average duration of schedule op `op_index` run alone: one untimed run,
 * then `iters` runs back to back on stream 0 between one hipEvent pair, on
 * the arena's current contents, nothing else in flight.  (dgen_hip_time_op
 * times the op inside whole runs, where a side-stream op shares the chip
 * with the stream-0 work it overlaps.)  No counterpart in the reference. */
int dgen_hip_time_op_alone(dgen_hip_ctx* ctx, uint32_t frame_count, uint32_t op_index, int iters, double* ms_out);

/* ---- bank forward without allocation --------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, real-time render loops, hosts that
 * forbid hipMalloc): the tensor biquad bank forward of the schedule classes
 * DGEN_HIP_K_BIQUAD_CHUNK -> _CARRY -> _FWD (RBJ low-pass, cutoff
 * base[k] * mod[n], Q[k], zero initial state) on caller-owned device buffers,
 * with the chunk summaries in a fixed scratch array the library holds on each
 * device (16 MiB: lanes x ceil(T/chunk) <= 299593; larger banks fail with
 * DGEN_HIP_E_RANGE).  No device memory is allocated or freed.
 *   x [T][B], y [T][B] (frame-major), params [2][B] = base | Q, mod [T] or
 *   NULL (unmodulated); chunk = frames per scan chunk (0: 256); stream: a
 *   hipStream_t, or NULL for the null stream.
 * The work is enqueued on `stream` and the call returns without waiting.
 * Every call on a device shares that device's scratch, so calls that can
 * overlap on one device (other streams, other host threads) race: order them
 * on one stream.  The caller's current device is restored on return. */
int dgen_hip_biquad_forward_noalloc(int device, const float* x, const float* mod, const float* params, float* y,
                                    uint32_t B, uint32_t T, uint32_t chunk, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DGEN_HIP_H */
