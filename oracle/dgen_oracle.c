/*
 * dgen_oracle.c -- CPU restatement of the DGen reference C-backend semantics
 * for the five workloads served by the HIP backend.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (libdgen_hip.so) never links, calls or falls back to it.
 *
 * One source, two builds:
 *   -DREAL=float  -DSFX=_f32   emission-faithful fp32 (IEEE, no contraction):
 *                              the forward parity reference and the CPU baseline
 *   -DREAL=double -DSFX=_f64   the same program in fp64, for central finite
 *                              differences of sum_frames(loss)
 * Constants that the reference computes in Float (steps, windows, twiddles,
 * 2*pi, noise samples) are rounded to fp32 in BOTH builds, so the f64 build is
 * the exact-arithmetic version of the same fp32 program.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the universalsequences/dgen-audio repository root).
 *
 * Pinning (see tests/test_oracle_*.py):
 *   deterministic phasor  closed form + CBackendTests.swift:46-76 known answers
 *   one-pole              impulse response 0.9^n (closed form)
 *   stateful phasor       fp64 closed-form phase sum, pre-increment output
 *   xorshift32 noise      bit-exact brute force of the published recurrence
 *   sampleRow             closed-form linear interpolation with wrap
 *   radix-2 FFT           brute-force DFT, impulse/DC/cosine, Parseval
 *   spectral loss         identical signals -> 0, brute-force DFT magnitudes
 *   MLP / heads           numpy restatement + finite differences
 *   ZDF SVF               TPT low-pass response (|H| on a steady sinusoid,
 *                         scipy lfilter of the bilinear transfer function),
 *                         odd symmetry and the exact 2x scaling invariant of
 *                         the saturation
 *   all analytic grads    central finite differences of the f64 build
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifndef REAL
#define REAL float
#define SFX _f32
#endif

#define CAT2(a, b) a##b
#define CAT(a, b) CAT2(a, b)
#define FN(name) CAT(name, SFX)

#define IS_F32 (sizeof(REAL) == 4)
#define R_SIN(x) (IS_F32 ? (REAL)sinf((float)(x)) : (REAL)sin((double)(x)))
#define R_COS(x) (IS_F32 ? (REAL)cosf((float)(x)) : (REAL)cos((double)(x)))
#define R_SQRT(x) (IS_F32 ? (REAL)sqrtf((float)(x)) : (REAL)sqrt((double)(x)))
#define R_LOG(x) (IS_F32 ? (REAL)logf((float)(x)) : (REAL)log((double)(x)))
#define R_EXP(x) (IS_F32 ? (REAL)expf((float)(x)) : (REAL)exp((double)(x)))
#define R_TANH(x) (IS_F32 ? (REAL)tanhf((float)(x)) : (REAL)tanh((double)(x)))
#define R_FLOOR(x) (IS_F32 ? (REAL)floorf((float)(x)) : (REAL)floor((double)(x)))
#define R_FMOD(x, y) (IS_F32 ? (REAL)fmodf((float)(x), (float)(y)) : (REAL)fmod((double)(x), (double)(y)))
#define R_ABS(x) (IS_F32 ? (REAL)fabsf((float)(x)) : (REAL)fabs((double)(x)))
#define R_TAN(x) (IS_F32 ? (REAL)tanf((float)(x)) : (REAL)tan((double)(x)))

static inline REAL r_sign(REAL x) { return x > 0 ? (REAL)1 : (x < 0 ? (REAL)-1 : (REAL)0); }
static inline REAL r_max(REAL a, REAL b) { return a >= b ? a : b; }
static inline REAL r_min(REAL a, REAL b) { return a <= b ? a : b; }

/* 2*Float.pi as Swift computes it in Float. */
#define TWO_PI_F32 ((REAL)(2.0f * 3.14159265358979323846f))

/* ------------------------------------------------------------------------ */
/* Shared helpers (compiled once per build; names carry the suffix).        */
/* ------------------------------------------------------------------------ */

/* Non-finite output containment: toolchain/include/dgen_runtime.h:58-85,
 * Sources/DGen/Renderer/CRenderer.swift:1021-1039 (every `out` store). */
static inline REAL sanitize(REAL v) { return isfinite(v) ? v : (REAL)0; }

/* u_accum: Sources/DGen/Definitions.swift:215-246.  Returns the
 * pre-increment value and updates *state. */
static inline REAL accum_step(REAL* state, REAL incr, REAL reset, REAL mn, REAL mx) {
  REAL acc = *state;
  REAL span = mx - mn;
  REAL next = reset > 0 ? mn : acc + incr;
  REAL k = R_FLOOR((next - mn) / span);
  REAL w = next - k * span;
  if (w >= mx) w = w - span;
  if (reset > 0) w = mn;
  *state = w;
  return acc;
}

/* Tensor stateful phasor: Sources/DGen/Emit+State.swift:322-369
 * (incr = freq / sampleRate; floor-wrap; >=1 correction; pre-increment out).
 * Always fp32: the phase depends on no parameter (f0 is data). */
static inline float phasor_step(float* state, float freq, float sr) {
  float prev = *state;
  float incr = freq / sr;
  float next = prev + incr;
  float w = next - floorf(next);
  if (w >= 1.0f) w = w - 1.0f;
  *state = w;
  return prev;
}

/* xorshift32 noise: Sources/DGen/Renderer/CRenderer.swift:685-693.  The state
 * lives in a zeroed float cell; 0 is replaced by 1 before the update. */
static inline float noise_step(uint32_t* s) {
  uint32_t x = *s;
  if (x == 0u) x = 1u;
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  *s = x;
  return (float)x / 4294967296.0f;
}

/* sampleInline row lookup: Sources/DGen/Emit+RowSelection.swift:164-197.
 * The row index and weights depend on no parameter: fp32 in both builds. */
typedef struct {
  int lo, hi;
  float frac, omf;
} RowLerp;
static inline RowLerp row_lerp(float index, int rows) {
  RowLerp r;
  float nr = (float)rows;
  float w = fmodf(index, nr);
  if (w < 0) w = w + nr;
  float fl = floorf(w);
  float ce = fl + 1.0f;
  if (ce >= nr) ce = 0;
  r.frac = w - fl;
  r.omf = 1.0f - r.frac;
  r.lo = (int)fl;
  r.hi = (int)ce;
  return r;
}
/* Interpolated read of a parameter-dependent value (REAL arithmetic). */
static inline REAL lerp_rows(const RowLerp* r, REAL a, REAL b) { return (REAL)r->omf * a + (REAL)r->frac * b; }
/* Interpolated read of data (f0, uv): fp32 in both builds. */
static inline float lerp_data(const RowLerp* r, float a, float b) { return r->omf * a + r->frac * b; }

/* ------------------------------------------------------------------------ */
/* Config 1: deterministic phasor bank -> sum -> one-pole history.          */
/* ------------------------------------------------------------------------ */

/* deterministicPhasor: Sources/DGen/Emit+State.swift:370-387;
 * Signal.phasor(Tensor): Sources/DGenLazy/SignalTensor.swift:67-80.
 * sin(phase * 2pi): Sources/DGen/Renderer/CRenderer.swift:825-827.
 * history one-pole y = x + 0.9*y[n-1]: Sources/DGen/Emit+State.swift:150-224
 * (read returns the previous frame's write). */
void FN(dgen_oracle_oscbank)(const float* freqs, const float* amps, int n_osc, float sr, float pole,
                             int frames, float* out) {
  REAL y = 0;
  for (int n = 0; n < frames; ++n) {
    REAL x = 0;
    for (int k = 0; k < n_osc; ++k) {
      REAL inc = (REAL)freqs[k] / (REAL)sr;
      REAL raw = inc * (REAL)n;
      REAL phase = raw - R_FLOOR(raw);
      x = x + R_SIN(phase * TWO_PI_F32) * (REAL)amps[k];
    }
    y = x + (REAL)pole * y;
    out[n] = (float)sanitize(y);
  }
}

/* One block of the bank as a streaming process call (dgen_process_v1 with
 * realize(preserveState: true), Sources/DGenLazy/Realize.swift:553-563).
 * state: [n_osc] phases, then y[n-1] of the history one-pole, carried from
 * the previous call.  stateful = 0: Signal.phasor(Tensor), the deterministic
 * phasor, whose frame index n restarts at 0 in every call
 * (Emit+State.swift:370-387 uses the frame index of the call); stateful = 1:
 * one Signal.phasor(Float) per oscillator, the u_phasor accumulator
 * (Definitions.swift:96-102, 215-246) carried in state.  The sum over the
 * oscillators keeps their order; out stores map non-finite values to 0. */
void FN(dgen_oracle_oscbank_stream)(const float* freqs, const float* amps, int n_osc, float sr, float pole, int frames,
                                    int stateful, REAL* state, float* out) {
  REAL y = state[n_osc];
  for (int n = 0; n < frames; ++n) {
    REAL x = 0;
    for (int k = 0; k < n_osc; ++k) {
      REAL phase;
      if (stateful) {
        float ph = (float)state[k];
        phase = (REAL)phasor_step(&ph, freqs[k], sr);
        state[k] = (REAL)ph;
      } else {
        REAL inc = (REAL)freqs[k] / (REAL)sr;
        REAL raw = inc * (REAL)n;
        phase = raw - R_FLOOR(raw);
      }
      x = x + R_SIN(phase * TWO_PI_F32) * (REAL)amps[k];
    }
    y = x + (REAL)pole * y;
    out[n] = (float)sanitize(y);
  }
  state[n_osc] = y;
}

/* ------------------------------------------------------------------------ */
/* Config 3: batched harmonic + FIR-noise synth, MLP decoder, MSS loss.      */
/* ------------------------------------------------------------------------ */

/* Control layout: one row of NC = K + 2 + NF floats per (b, f), row index
 * m = b*F + f (reference: controls.reshape([B, F, ...]),
 * Examples/HarmonicE2E/Synth.swift:72-75).  Columns: [0,K) harmonic amps,
 * K harmonic gain, K+1 noise gain, [K+2, K+2+NF) FIR taps. */

/* The playhead of Examples/HarmonicE2E/Synth.swift:60-71: accum of
 * step = (F-1)/(T-1) wrapping at F-1, clipped to [0, F-1-1e-4].  It depends
 * on no parameter, so both builds evaluate it in fp32 exactly as the C backend
 * does (the fp32 accumulation drifts and can wrap to row 0 in the last frames
 * of long runs; that is reference behaviour). */
static void playhead_real(int F, int T, REAL* out) {
  float fmaxi = (float)(F > 1 ? F - 1 : 0);
  float denom = (float)(T > 2 ? T - 1 : 1);
  float step = fmaxi / denom;
  float hi = fmaxi - 1e-4f > 0.f ? fmaxi - 1e-4f : 0.f;
  /* the accumulator's wrap span: fmaxi, or 1 for a single control row (a
   * zero span would divide 0 by 0; with step 0 the playhead stays at row
   * 0 either way), as the schedule's accumulator table is set up */
  float span = F > 1 ? fmaxi : 1.0f;
  float st = 0;
  for (int t = 0; t < T; ++t) {
    float acc = st;
    float next = acc + step;
    float k = floorf(next / span);
    float w = next - k * span;
    if (w >= span) w = w - span;
    st = w;
    float p = acc < 0.f ? 0.f : acc;
    out[t] = (REAL)(p > hi ? hi : p);
  }
}
#ifdef ORACLE_COMMON
static void playhead_real_f32(int F, int T, float* out) {
  REAL* p = (REAL*)malloc(sizeof(REAL) * T);
  playhead_real(F, T, p);
  for (int t = 0; t < T; ++t) out[t] = (float)p[t];
  free(p);
}
#endif
void FN(dgen_oracle_playhead)(int F, int T, float* out) {
  REAL* p = (REAL*)malloc(sizeof(REAL) * T);
  playhead_real(F, T, p);
  for (int t = 0; t < T; ++t) out[t] = (float)p[t];
  free(p);
}

/* The shared xorshift32 stream of Signal.noise() for T frames, starting from
 * a zeroed cell (CRenderer.swift:685-693).  Precision-independent: emitted
 * once, by the fp32 build. */
void dgen_oracle_noise_stream(int T, float* out);
#ifdef ORACLE_COMMON
void dgen_oracle_noise_stream(int T, float* out) {
  uint32_t s = 0;
  for (int t = 0; t < T; ++t) out[t] = noise_step(&s);
}
#endif

/* Stateful phasor (pre-increment output) driven by a per-frame frequency:
 * Sources/DGen/Definitions.swift:96-102,215-246 (u_phasor / u_accum order),
 * Sources/DGenLazy/Signal.swift:183-225.  Precision-independent (fp32). */
void dgen_oracle_phasor(const float* freq, int T, float sr, float* out);
/* Frame-rate sampleRow read of a [F][B] data table through the playhead of
 * Examples/HarmonicE2E/Synth.swift:60-71 (Emit+RowSelection.swift:164-197):
 * out[b][t].  Precision-independent (fp32). */
void dgen_oracle_lerp_frames(const float* src, int B, int F, int T, float* out);
/* Phase of harmonic lane (b, k), freq = (k+1) * f0f[b][t], at the start of
 * every seg-frame segment: out[s][b][k] (the tensor phasor of
 * Emit+State.swift:322-369 evaluated sequentially in fp32). */
void dgen_oracle_phase_checkpoints(const float* f0f, int B, int K, int T, float sr, int seg, float* out);
#ifdef ORACLE_COMMON
void dgen_oracle_phasor(const float* freq, int T, float sr, float* out) {
  float st = 0.0f;
  for (int t = 0; t < T; ++t) out[t] = phasor_step(&st, freq[t], sr);
}
void dgen_oracle_lerp_frames(const float* src, int B, int F, int T, float* out) {
  float* play = (float*)malloc(sizeof(float) * T);
  playhead_real_f32(F, T, play);
  for (int t = 0; t < T; ++t) {
    RowLerp r = row_lerp(play[t], F);
    for (int b = 0; b < B; ++b) out[(size_t)b * T + t] = lerp_data(&r, src[r.lo * B + b], src[r.hi * B + b]);
  }
  free(play);
}
void dgen_oracle_phase_checkpoints(const float* f0f, int B, int K, int T, float sr, int seg, float* out) {
  const int nseg = (T + seg - 1) / seg;
  for (int b = 0; b < B; ++b)
    for (int k = 0; k < K; ++k) {
      float ph = 0.0f;
      for (int t = 0; t < T; ++t) {
        if (t % seg == 0) out[((size_t)(t / seg) * B + b) * K + k] = ph;
        (void)phasor_step(&ph, (float)(k + 1) * f0f[(size_t)b * T + t], sr);
      }
    }
  (void)nseg;
}
#endif

/* Forward synth: HarmonicSynth.renderBatchedSignal,
 * Examples/HarmonicE2E/Synth.swift:47-102, with nyquistNormalizedHarmonicsBatched
 * (:158-167).  ctrl: [B*F][NC]; f0, uv: [F][B]; y: [B][T] (lane-major).
 * Frame-sequential exactly like the C backend: per frame the playhead accum,
 * the sampleRow reads, the tensor phasor update and the noise buffer write.
 * With dy != NULL it instead accumulates the adjoint into dctrl (the graph AD
 * of the same expressions: Gradients.swift rules for mul/div/sum and the
 * sampleInline gradient scatter, Emit+RowSelection.swift:100-141; f0, uv and
 * noise are data and carry no gradient). */
static void synth_core(const REAL* ctrl, const float* f0, const float* uv, int B, int F, int T, int K, int NF,
                       float sr, float graph_sr, float hscale, float nscale, REAL* y, const REAL* dy, REAL* dctrl) {
  const int NC = K + 2 + NF;
  REAL* play = (REAL*)malloc(sizeof(REAL) * T);
  float* noise = (float*)malloc(sizeof(float) * T);
  float* ph = (float*)calloc((size_t)B * K, sizeof(float));
  float* freq = (float*)malloc(sizeof(float) * K);
  REAL* masked = (REAL*)malloc(sizeof(REAL) * K);
  REAL* sines = (REAL*)malloc(sizeof(REAL) * K);
  playhead_real(F, T, play);
  dgen_oracle_noise_stream(T, noise);
  if (dctrl) memset(dctrl, 0, sizeof(REAL) * (size_t)B * F * NC);
  /* phase increments divide by the host sample rate (u_phasor,
   * Definitions.swift:96-102); the Nyquist mask uses the graph's
   * DGenConfig.sampleRate (Synth.swift:158-167) */
  const float nyq = graph_sr * 0.5f;
  for (int t = 0; t < T; ++t) {
    RowLerp r = row_lerp((float)play[t], F);
    for (int b = 0; b < B; ++b) {
      const REAL* c0 = ctrl + (size_t)(b * F + r.lo) * NC;
      const REAL* c1 = ctrl + (size_t)(b * F + r.hi) * NC;
      float f0i = lerp_data(&r, f0[r.lo * B + b], f0[r.hi * B + b]);
      REAL uvi = (REAL)lerp_data(&r, uv[r.lo * B + b], uv[r.hi * B + b]);
      REAL den = 0;
      for (int k = 0; k < K; ++k) {
        freq[k] = (float)(k + 1) * f0i;
        REAL a = lerp_rows(&r, c0[k], c1[k]);
        masked[k] = a * (freq[k] < nyq ? (REAL)1 : (REAL)0);
        den = den + masked[k];
      }
      den = den + (REAL)1e-8f;
      REAL hsum = 0;
      for (int k = 0; k < K; ++k) {
        float p = phasor_step(&ph[b * K + k], freq[k], sr);
        sines[k] = R_SIN((REAL)(p * (2.0f * 3.14159265358979323846f)));
        hsum = hsum + sines[k] * (masked[k] / den);
      }
      REAL gain = lerp_rows(&r, c0[K], c1[K]);
      REAL ngain = lerp_rows(&r, c0[K + 1], c1[K + 1]);
      /* bufferView window: oldest first, ends at the current frame, zero
       * before frame 0 (HigherOps.swift:738-792). */
      REAL filt = 0;
      for (int i = 0; i < NF; ++i) {
        int tt = t - (NF - 1) + i;
        REAL w = tt >= 0 ? (REAL)noise[tt] : (REAL)0;
        filt = filt + w * lerp_rows(&r, c0[K + 2 + i], c1[K + 2 + i]);
      }
      REAL hout = ((hsum * gain) * uvi) * (REAL)hscale;
      REAL nout = ((filt * ngain) * (REAL)0.12f) * (REAL)nscale;
      if (y) y[(size_t)b * T + t] = sanitize(hout + nout);
      if (!dy) continue;
      REAL* d0 = dctrl + (size_t)(b * F + r.lo) * NC;
      REAL* d1 = dctrl + (size_t)(b * F + r.hi) * NC;
      const REAL omf = (REAL)r.omf, frac = (REAL)r.frac;
      REAL g = dy[(size_t)b * T + t];
      REAL dhsum = g * gain * uvi * (REAL)hscale;
      REAL dgain = g * hsum * uvi * (REAL)hscale;
      /* amps = masked/den:  d masked_k = (dA_k - sum_j dA_j amps_j) / den */
      REAL dot = 0;
      for (int k = 0; k < K; ++k) dot = dot + dhsum * sines[k] * (masked[k] / den);
      for (int k = 0; k < K; ++k) {
        REAL mk = freq[k] < nyq ? (REAL)1 : (REAL)0;
        REAL dm = (dhsum * sines[k] - dot) / den * mk;
        d0[k] += omf * dm;
        d1[k] += frac * dm;
      }
      d0[K] += omf * dgain;
      d1[K] += frac * dgain;
      REAL dfilt = g * ngain * (REAL)0.12f * (REAL)nscale;
      REAL dngain = g * filt * (REAL)0.12f * (REAL)nscale;
      d0[K + 1] += omf * dngain;
      d1[K + 1] += frac * dngain;
      for (int i = 0; i < NF; ++i) {
        int tt = t - (NF - 1) + i;
        REAL w = tt >= 0 ? (REAL)noise[tt] : (REAL)0;
        d0[K + 2 + i] += omf * (dfilt * w);
        d1[K + 2 + i] += frac * (dfilt * w);
      }
    }
  }
  free(play);
  free(noise);
  free(ph);
  free(freq);
  free(masked);
  free(sines);
}

static REAL* to_real(const float* a, size_t n) {
  REAL* r = (REAL*)malloc(sizeof(REAL) * (n ? n : 1));
  for (size_t i = 0; i < n; ++i) r[i] = (REAL)a[i];
  return r;
}
static void to_float(const REAL* a, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = (float)a[i];
}

void FN(dgen_oracle_synth_fwd)(const float* ctrl, const float* f0, const float* uv, int B, int F, int T, int K,
                               int NF, float sr, float hscale, float nscale, float* y) {
  size_t nc = (size_t)B * F * (K + 2 + NF);
  REAL* c = to_real(ctrl, nc);
  REAL* yr = (REAL*)malloc(sizeof(REAL) * (size_t)B * T);
  synth_core(c, f0, uv, B, F, T, K, NF, sr, sr, hscale, nscale, yr, NULL, NULL);
  to_float(yr, (size_t)B * T, y);
  free(c);
  free(yr);
}

/* The forward with a host sample rate (phase increments) that differs from
 * the graph's (the Nyquist mask): dgen_process_v1's context.sample_rate
 * against DGenConfig.sampleRate. */
void FN(dgen_oracle_synth_fwd_rates)(const float* ctrl, const float* f0, const float* uv, int B, int F, int T, int K,
                                     int NF, float host_sr, float graph_sr, float hscale, float nscale, float* y) {
  size_t nc = (size_t)B * F * (K + 2 + NF);
  REAL* c = to_real(ctrl, nc);
  REAL* yr = (REAL*)malloc(sizeof(REAL) * (size_t)B * T);
  synth_core(c, f0, uv, B, F, T, K, NF, host_sr, graph_sr, hscale, nscale, yr, NULL, NULL);
  to_float(yr, (size_t)B * T, y);
  free(c);
  free(yr);
}

void FN(dgen_oracle_synth_bwd)(const float* ctrl, const float* f0, const float* uv, const float* dy, int B, int F,
                               int T, int K, int NF, float sr, float hscale, float nscale, float* dctrl) {
  size_t nc = (size_t)B * F * (K + 2 + NF);
  REAL* c = to_real(ctrl, nc);
  REAL* d = to_real(dy, (size_t)B * T);
  REAL* dc = (REAL*)malloc(sizeof(REAL) * nc);
  synth_core(c, f0, uv, B, F, T, K, NF, sr, sr, hscale, nscale, NULL, d, dc);
  to_float(dc, nc, dctrl);
  free(c);
  free(d);
  free(dc);
}

/* softplus(x) = max(x,0) + log(1 + exp(-|x|)): Examples/HarmonicE2E/Model.swift:153-157. */
static inline REAL softplus(REAL x) { return r_max(x, 0) + R_LOG((REAL)1 + R_EXP(-R_ABS(x))); }
/* Its derivative through the reference's AD rules (Gradients.swift:398-408 max,
 * :429-433 abs, :479-490 exp/log): [x>=0] - sign(x)*e^{-|x|}/(1+e^{-|x|}). */
static inline REAL softplus_grad(REAL x) {
  REAL e = R_EXP(-R_ABS(x));
  return (x >= 0 ? (REAL)1 : (REAL)0) - r_sign(x) * (e / ((REAL)1 + e));
}

/* Parameter blob layout (floats, this order): W1[DIN][H] b1[H] W2[H][H] b2[H]
 * ... (L trunk layers), then Wh[H][NC] bh[NC], where the head columns
 * concatenate W_harm | W_gain | W_noise | W_noiseFilter
 * (Examples/HarmonicE2E/Model.swift:36-83). */
static size_t mlp_param_count(int din, int hid, int layers, int nc) {
  size_t n = 0;
  for (int l = 0; l < layers; ++l) n += (size_t)(l == 0 ? din : hid) * hid + hid;
  return n + (size_t)hid * nc + nc;
}
size_t FN(dgen_oracle_mlp_param_count)(int din, int hid, int layers, int nc) {
  return mlp_param_count(din, hid, layers, nc);
}

/* HarmonicDecoderModel.forward: Examples/HarmonicE2E/Model.swift:96-120.
 * X: [M][DIN].  acts (optional, L*M*H) keeps the trunk outputs for the
 * backward; zh (optional): head pre-activations [M][NC]; ctrl: [M][NC]. */
static void mlp_forward(const float* X, const REAL* P, int M, int din, int hid, int layers, int K, int NF,
                        REAL* acts, REAL* zh, REAL* ctrl) {
  const int NC = K + 2 + NF;
  REAL* h = (REAL*)malloc(sizeof(REAL) * (hid > din ? hid : din));
  REAL* hn = (REAL*)malloc(sizeof(REAL) * hid);
  REAL* z = (REAL*)malloc(sizeof(REAL) * NC);
  for (int m = 0; m < M; ++m) {
    const REAL* p = P;
    int fan = din;
    for (int i = 0; i < din; ++i) h[i] = (REAL)X[(size_t)m * din + i];
    for (int l = 0; l < layers; ++l) {
      const REAL* W = p;
      const REAL* bb = p + (size_t)fan * hid;
      for (int j = 0; j < hid; ++j) {
        REAL s = 0;
        for (int i = 0; i < fan; ++i) s = s + h[i] * W[(size_t)i * hid + j];
        hn[j] = R_TANH(s + bb[j]);
      }
      memcpy(h, hn, sizeof(REAL) * hid);
      if (acts) memcpy(acts + ((size_t)l * M + m) * hid, h, sizeof(REAL) * hid);
      p += (size_t)fan * hid + hid;
      fan = hid;
    }
    const REAL* Wh = p;
    const REAL* bh = p + (size_t)hid * NC;
    for (int c = 0; c < NC; ++c) {
      REAL s = 0;
      for (int i = 0; i < hid; ++i) s = s + h[i] * Wh[(size_t)i * NC + c];
      z[c] = s + bh[c];
      if (zh) zh[(size_t)m * NC + c] = z[c];
    }
    REAL* out = ctrl + (size_t)m * NC;
    /* harmonic amps: softplus, normalised by sum + 1e-6 (Model.swift:102-106) */
    REAL den = 0;
    for (int k = 0; k < K; ++k) den = den + softplus(z[k]);
    den = den + (REAL)1e-6f;
    for (int k = 0; k < K; ++k) out[k] = softplus(z[k]) / den;
    out[K] = softplus(z[K]);         /* harmonic gain (:107) */
    out[K + 1] = softplus(z[K + 1]); /* noise gain (:108) */
    /* FIR taps: tanh, normalised by sum|.| + 1e-4 (:109-113) */
    REAL nrm = 0;
    for (int i = 0; i < NF; ++i) nrm = nrm + R_ABS(R_TANH(z[K + 2 + i]));
    nrm = nrm + (REAL)1e-4f;
    for (int i = 0; i < NF; ++i) out[K + 2 + i] = R_TANH(z[K + 2 + i]) / nrm;
  }
  free(h);
  free(hn);
  free(z);
}

/* Backward of the MLP + heads (graph AD of Model.swift:96-120 with the rules
 * of Gradients.swift: matmul/sum, tanh :470-477, softplus via max/abs/exp/log).
 * dctrl: [M][NC]; dP: same layout as P (overwritten). */
static void mlp_backward(const float* X, const REAL* P, const REAL* dctrl, int M, int din, int hid, int layers,
                         int K, int NF, REAL* dP) {
  const int NC = K + 2 + NF;
  size_t np = mlp_param_count(din, hid, layers, NC);
  REAL* acts = (REAL*)malloc(sizeof(REAL) * (size_t)layers * M * hid);
  REAL* zh = (REAL*)malloc(sizeof(REAL) * (size_t)M * NC);
  REAL* ctrl = (REAL*)malloc(sizeof(REAL) * (size_t)M * NC);
  memset(dP, 0, sizeof(REAL) * np);
  mlp_forward(X, P, M, din, hid, layers, K, NF, acts, zh, ctrl);
  size_t* woff = (size_t*)malloc(sizeof(size_t) * (layers + 1));
  size_t off = 0;
  for (int l = 0; l < layers; ++l) {
    woff[l] = off;
    off += (size_t)(l == 0 ? din : hid) * hid + hid;
  }
  woff[layers] = off;
  REAL* dz = (REAL*)malloc(sizeof(REAL) * NC);
  REAL* dh = (REAL*)malloc(sizeof(REAL) * hid);
  REAL* dhp = (REAL*)malloc(sizeof(REAL) * hid);
  for (int m = 0; m < M; ++m) {
    const REAL* z = zh + (size_t)m * NC;
    const REAL* dc = dctrl + (size_t)m * NC;
    REAL den = 0;
    for (int k = 0; k < K; ++k) den = den + softplus(z[k]);
    den = den + (REAL)1e-6f;
    REAL dot = 0;
    for (int k = 0; k < K; ++k) dot = dot + dc[k] * (softplus(z[k]) / den);
    for (int k = 0; k < K; ++k) dz[k] = (dc[k] - dot) / den * softplus_grad(z[k]);
    dz[K] = dc[K] * softplus_grad(z[K]);
    dz[K + 1] = dc[K + 1] * softplus_grad(z[K + 1]);
    REAL nrm = 0;
    for (int i = 0; i < NF; ++i) nrm = nrm + R_ABS(R_TANH(z[K + 2 + i]));
    nrm = nrm + (REAL)1e-4f;
    REAL dot2 = 0;
    for (int i = 0; i < NF; ++i) dot2 = dot2 + dc[K + 2 + i] * (R_TANH(z[K + 2 + i]) / nrm);
    for (int i = 0; i < NF; ++i) {
      REAL s = R_TANH(z[K + 2 + i]);
      REAL ds = (dc[K + 2 + i] - r_sign(s) * dot2) / nrm;
      dz[K + 2 + i] = ds * ((REAL)1 - s * s);
    }
    const REAL* h3 = acts + ((size_t)(layers - 1) * M + m) * hid;
    const REAL* Wh = P + woff[layers];
    REAL* dWh = dP + woff[layers];
    REAL* dbh = dWh + (size_t)hid * NC;
    for (int c = 0; c < NC; ++c) dbh[c] += dz[c];
    for (int i = 0; i < hid; ++i) {
      REAL s = 0;
      for (int c = 0; c < NC; ++c) {
        dWh[(size_t)i * NC + c] += h3[i] * dz[c];
        s = s + dz[c] * Wh[(size_t)i * NC + c];
      }
      dh[i] = s;
    }
    for (int l = layers - 1; l >= 0; --l) {
      int fan = l == 0 ? din : hid;
      const REAL* hl = acts + ((size_t)l * M + m) * hid;
      const REAL* W = P + woff[l];
      REAL* dW = dP + woff[l];
      REAL* db = dW + (size_t)fan * hid;
      for (int j = 0; j < hid; ++j) dh[j] = dh[j] * ((REAL)1 - hl[j] * hl[j]);
      for (int j = 0; j < hid; ++j) db[j] += dh[j];
      for (int i = 0; i < fan; ++i) {
        REAL hin = l == 0 ? (REAL)X[(size_t)m * din + i] : acts[((size_t)(l - 1) * M + m) * hid + i];
        REAL s = 0;
        for (int j = 0; j < hid; ++j) {
          dW[(size_t)i * hid + j] += hin * dh[j];
          s = s + dh[j] * W[(size_t)i * hid + j];
        }
        if (l > 0) dhp[i] = s;
      }
      if (l > 0) memcpy(dh, dhp, sizeof(REAL) * hid);
    }
  }
  free(acts);
  free(zh);
  free(ctrl);
  free(woff);
  free(dz);
  free(dh);
  free(dhp);
}

void FN(dgen_oracle_mlp_fwd)(const float* X, const float* P, int M, int din, int hid, int layers, int K, int NF,
                             float* ctrl) {
  size_t np = mlp_param_count(din, hid, layers, K + 2 + NF);
  REAL* p = to_real(P, np);
  REAL* c = (REAL*)malloc(sizeof(REAL) * (size_t)M * (K + 2 + NF));
  mlp_forward(X, p, M, din, hid, layers, K, NF, NULL, NULL, c);
  to_float(c, (size_t)M * (K + 2 + NF), ctrl);
  free(p);
  free(c);
}

void FN(dgen_oracle_mlp_bwd)(const float* X, const float* P, const float* dctrl, int M, int din, int hid,
                             int layers, int K, int NF, float* dP_out) {
  size_t np = mlp_param_count(din, hid, layers, K + 2 + NF);
  REAL* p = to_real(P, np);
  REAL* dc = to_real(dctrl, (size_t)M * (K + 2 + NF));
  REAL* dp = (REAL*)malloc(sizeof(REAL) * np);
  mlp_backward(X, p, dc, M, din, hid, layers, K, NF, dp);
  to_float(dp, np, dP_out);
  free(p);
  free(dc);
  free(dp);
}

/* ---- radix-2 FFT exactly as the spectral-loss kernels emit it ----------- */
/* Tables: Sources/DGen/HigherOps.swift:71-99 (symmetric Hann over N-1, Float
 * twiddles cos/sin(2*pi*k/(2*half)) at offset half-1, bit reversal).        */
typedef struct {
  int n, stages;
  float* hann;
  float* twre;
  float* twim;
  int* bitrev;
} FftTables;

static void fft_tables_init(FftTables* t, int n, int rect) {
  t->n = n;
  t->stages = 0;
  while ((1 << t->stages) < n) t->stages++;
  t->hann = (float*)malloc(sizeof(float) * n);
  t->twre = (float*)malloc(sizeof(float) * (n > 1 ? n - 1 : 1));
  t->twim = (float*)malloc(sizeof(float) * (n > 1 ? n - 1 : 1));
  t->bitrev = (int*)malloc(sizeof(int) * n);
  /* useHannWindow: false keeps the all-1.0 window (HigherOps.swift:69-76) */
  for (int i = 0; i < n; ++i)
    t->hann[i] = rect ? 1.0f : (float)(0.5 * (1.0 - cos(2.0 * M_PI * (double)i / (double)(n - 1))));
  for (int s = 0; s < t->stages; ++s) {
    int half = 1 << s;
    for (int k = 0; k < half; ++k) {
      double ang = 2.0 * M_PI * (double)k / (double)(2 * half);
      t->twre[half - 1 + k] = (float)cos(ang);
      t->twim[half - 1 + k] = (float)sin(ang);
    }
  }
  for (int i = 0; i < n; ++i) {
    int rev = 0, bits = i;
    for (int s = 0; s < t->stages; ++s) {
      rev = rev * 2 + (bits & 1);
      bits >>= 1;
    }
    t->bitrev[i] = rev;
  }
}
static void fft_tables_free(FftTables* t) {
  free(t->hann);
  free(t->twre);
  free(t->twim);
  free(t->bitrev);
}

/* In-place radix-2 DIT, forward (twiddle exp(-i...)) when sign<0, inverse
 * without 1/N when sign>0: Emit+SpectralLoss.swift:802-848 (forward),
 * :1085-1160 (gradient IFFT). */
static void fft_inplace(const FftTables* t, REAL* re, REAL* im, int sign) {
  int n = t->n;
  for (int i = 0; i < n; ++i) {
    int r = t->bitrev[i];
    if (i < r) {
      REAL a = re[i];
      re[i] = re[r];
      re[r] = a;
      a = im[i];
      im[i] = im[r];
      im[r] = a;
    }
  }
  for (int s = 0; s < t->stages; ++s) {
    int half = 1 << s, size = half * 2;
    for (int g = 0; g < n / size; ++g) {
      for (int k = 0; k < half; ++k) {
        REAL wr = (REAL)t->twre[half - 1 + k];
        REAL wi = sign < 0 ? -(REAL)t->twim[half - 1 + k] : (REAL)t->twim[half - 1 + k];
        int i = g * size + k, j = i + half;
        REAL tr = wr * re[j] - wi * im[j];
        REAL ti = wr * im[j] + wi * re[j];
        REAL ar = re[i], ai = im[i];
        re[i] = ar + tr;
        im[i] = ai + ti;
        re[j] = ar - tr;
        im[j] = ai - ti;
      }
    }
  }
}

/* Forward FFT of one hop window ending at frame f (window covers f-N+1..f,
 * zero outside [0,T)): Emit+SpectralLoss.swift:776-800. */
static void window_fft(const FftTables* tb, const REAL* x, int T, int f, REAL* re, REAL* im) {
  int n = tb->n;
  for (int i = 0; i < n; ++i) {
    int tt = f - (n - 1) + i;
    REAL s = (tt >= 0 && tt < T) ? x[tt] : (REAL)0;
    re[i] = s * (REAL)tb->hann[i];
    im[i] = 0;
  }
  fft_inplace(tb, re, im, -1);
}

#define LOG_EPS ((REAL)1e-8f) /* DGenSpectralConfig.logMagnitudeEpsilon, GradientConfig.swift:38 */
/* Loss-mode bits of the multi-scale loss (one spectralLossFFT call per term
 * and size in the reference, HigherOps.swift:49-65, Functions.swift:870-910):
 * the magnitude term's and the log-magnitude term's lossMode (.l1 default of
 * the trainer, .l2 the API default), useSmoothLogMagnitude for the log term,
 * and useHannWindow: false for both. */
#define MSS_L2_LIN 1
#define MSS_L2_LOG 2
#define MSS_SMOOTH_LOG 4
#define MSS_RECT_WINDOW 8

/* Multi-scale spectral loss, HarmonicE2E Trainer.fullBatchedLoss
 * (Examples/HarmonicE2E/Trainer.swift:538-583) over spectralLossFFTBatched +
 * BatchedReduce (Emit+SpectralLoss.swift:719-938) with normalize
 * (Sources/DGenLazy/Functions.swift:945-955: / maxFrameCount), and the
 * trainer's time-domain term mseLossWeight * sum_b (y - tgt)^2 / B per frame
 * (Trainer.swift:547-551).
 * x, tgt: [B][T].  lf[T]: the per-frame loss signal.  mode: MSS_* bits.
 * Per bin the forward follows Emit+SpectralLoss.swift:150-188: m = sqrt(re^2 +
 * im^2) (with MSS_SMOOTH_LOG the log term's magnitude is sqrt(re^2 + im^2 +
 * eps^2) and its difference log(m1) - log(m2), else log(m1+eps) -
 * log(m2+eps)); L1 accumulates |diff|, L2 diff^2.
 * With dx != NULL also writes d sum_frames(loss) / d x: GradSpec
 * (Emit+SpectralLoss.swift:196-291: scale sign(diff) (L1) or 2 diff (L2),
 * / (m+eps) or / m_smooth for the log term, times X / max(m, 1e-8) or
 * X / m_smooth, bins above N/2 zeroed), the unnormalised positive-twiddle
 * IFFT (:1032-1160), window multiply, and the per-sample gather over the hop
 * windows containing it (:1163-1235); plus the MSE term's 2 w (y - tgt) / B. */
static double mss_core(const REAL* x, const REAL* tgt, int B, int T, const int* sizes, int n_sizes, int hop_div,
                       float w_lin, float w_log, float max_frames, int mode, float w_mse, REAL* lf, REAL* dx) {
  memset(lf, 0, sizeof(REAL) * T);
  if (dx) memset(dx, 0, sizeof(REAL) * (size_t)B * T);
  const int l2lin = (mode & MSS_L2_LIN) != 0, l2log = (mode & MSS_L2_LOG) != 0;
  const int smooth = (mode & MSS_SMOOTH_LOG) != 0;
  if (w_mse != 0.0f) {
    /* batchMSE = (diff*diff).sum() * (1/B), times mseLossWeight, first in
     * the frame's total */
    const REAL inv_b = (REAL)(1.0f / (float)B);
    for (int t = 0; t < T; ++t) {
      REAL s = 0;
      for (int b = 0; b < B; ++b) {
        const REAL d = x[(size_t)b * T + t] - tgt[(size_t)b * T + t];
        s = s + d * d;
        if (dx) dx[(size_t)b * T + t] = (REAL)w_mse * ((REAL)2 * d) * inv_b;
      }
      lf[t] = s * inv_b * (REAL)w_mse;
    }
  }
  for (int si = 0; si < n_sizes; ++si) {
    int N = sizes[si], H = N / hop_div > 0 ? N / hop_div : 1;
    FftTables tb;
    fft_tables_init(&tb, N, (mode & MSS_RECT_WINDOW) != 0);
    REAL *r1 = (REAL*)malloc(sizeof(REAL) * N), *i1 = (REAL*)malloc(sizeof(REAL) * N);
    REAL *r2 = (REAL*)malloc(sizeof(REAL) * N), *i2 = (REAL*)malloc(sizeof(REAL) * N);
    REAL *gr = (REAL*)malloc(sizeof(REAL) * N), *gi = (REAL*)malloc(sizeof(REAL) * N);
    REAL wl = (REAL)(w_lin / (float)n_sizes), wg = (REAL)(w_log / (float)n_sizes);
    /* upstream gradient of each batched spectral node, scaled by 1/B (:960) */
    REAL gl = wl / (REAL)max_frames / (REAL)B;
    REAL gg = wg / (REAL)max_frames / (REAL)B;
    for (int f = 0; f < T; f += H) {
      REAL lin = 0, lg = 0;
      for (int b = 0; b < B; ++b) {
        window_fft(&tb, x + (size_t)b * T, T, f, r1, i1);
        window_fft(&tb, tgt + (size_t)b * T, T, f, r2, i2);
        REAL bl = 0, bg = 0;
        for (int k = 0; k < N; ++k) gr[k] = gi[k] = 0;
        for (int k = 0; k <= N / 2; ++k) {
          REAL p1 = r1[k] * r1[k] + i1[k] * i1[k];
          REAL p2 = r2[k] * r2[k] + i2[k] * i2[k];
          REAL m1 = R_SQRT(p1);
          REAL m2 = R_SQRT(p2);
          /* the log term's denominators: m + eps, or the smooth magnitude */
          REAL s1 = smooth ? R_SQRT(p1 + LOG_EPS * LOG_EPS) : m1 + LOG_EPS;
          REAL s2 = smooth ? R_SQRT(p2 + LOG_EPS * LOG_EPS) : m2 + LOG_EPS;
          REAL dlin = m1 - m2;
          REAL dlog = R_LOG(s1) - R_LOG(s2);
          bl = bl + (l2lin ? dlin * dlin : R_ABS(dlin));
          bg = bg + (l2log ? dlog * dlog : R_ABS(dlog));
          if (dx) {
            REAL sl = l2lin ? (REAL)2 * dlin : r_sign(dlin);
            REAL sg = l2log ? (REAL)2 * dlog : r_sign(dlog);
            REAL sm = r_max(m1, (REAL)1e-8f);
            if (!smooth) {
              REAL dmag = gl * sl + gg * sg / (m1 + LOG_EPS);
              gr[k] = dmag * r1[k] / sm;
              gi[k] = dmag * i1[k] / sm;
            } else {
              /* the two calls' spectra: lin over max(m, 1e-8), log over the
               * smooth magnitude twice (1/m_s from the log, X/m_s) */
              REAL cl = gl * sl / sm, cg = gg * sg / s1 / s1;
              gr[k] = cl * r1[k] + cg * r1[k];
              gi[k] = cl * i1[k] + cg * i1[k];
            }
          }
        }
        lin = lin + bl;
        lg = lg + bg;
        if (dx) {
          fft_inplace(&tb, gr, gi, +1);
          for (int i = 0; i < N; ++i) {
            int tt = f - (N - 1) + i;
            if (tt >= 0 && tt < T) dx[(size_t)b * T + tt] += gr[i] * (REAL)tb.hann[i];
          }
        }
      }
      lin = lin / (REAL)B / (REAL)max_frames;
      lg = lg / (REAL)B / (REAL)max_frames;
      lf[f] = lf[f] + lin * wl + lg * wg;
    }
    free(r1);
    free(i1);
    free(r2);
    free(i2);
    free(gr);
    free(gi);
    fft_tables_free(&tb);
  }
  double total = 0;
  for (int t = 0; t < T; ++t) total += (double)lf[t];
  return total;
}

double FN(dgen_oracle_mss_fwd)(const float* x, const float* tgt, int B, int T, const int* sizes, int n_sizes,
                               int hop_div, float w_lin, float w_log, float max_frames, int mode, float w_mse,
                               float* loss_frames) {
  REAL* xr = to_real(x, (size_t)B * T);
  REAL* tr = to_real(tgt, (size_t)B * T);
  REAL* lf = (REAL*)malloc(sizeof(REAL) * T);
  double tot = mss_core(xr, tr, B, T, sizes, n_sizes, hop_div, w_lin, w_log, max_frames, mode, w_mse, lf, NULL);
  if (loss_frames) to_float(lf, T, loss_frames);
  free(xr);
  free(tr);
  free(lf);
  return tot;
}

/* As dgen_oracle_mss_fwd with the prediction in this build's precision, so
 * finite differences can perturb it below fp32 resolution. */
double FN(dgen_oracle_mss_fwd_real)(const REAL* x, const float* tgt, int B, int T, const int* sizes, int n_sizes,
                                    int hop_div, float w_lin, float w_log, float max_frames, int mode, float w_mse) {
  REAL* tr = to_real(tgt, (size_t)B * T);
  REAL* lf = (REAL*)malloc(sizeof(REAL) * T);
  double tot = mss_core(x, tr, B, T, sizes, n_sizes, hop_div, w_lin, w_log, max_frames, mode, w_mse, lf, NULL);
  free(tr);
  free(lf);
  return tot;
}

void FN(dgen_oracle_mss_bwd)(const float* x, const float* tgt, int B, int T, const int* sizes, int n_sizes,
                             int hop_div, float w_lin, float w_log, float max_frames, int mode, float w_mse,
                             float* dx_out) {
  REAL* xr = to_real(x, (size_t)B * T);
  REAL* tr = to_real(tgt, (size_t)B * T);
  REAL* lf = (REAL*)malloc(sizeof(REAL) * T);
  REAL* dx = (REAL*)malloc(sizeof(REAL) * (size_t)B * T);
  mss_core(xr, tr, B, T, sizes, n_sizes, hop_div, w_lin, w_log, max_frames, mode, w_mse, lf, dx);
  to_float(dx, (size_t)B * T, dx_out);
  free(xr);
  free(tr);
  free(lf);
  free(dx);
}

/* One whole config-3 training step in this build's precision: MLP -> synth ->
 * MSS loss, and (dP != NULL) the full backward to the parameters.  P and dP
 * use REAL (double in the fp64 build), so finite differences can perturb the
 * parameters far below fp32 resolution.  tgt: [B][T].  y_out (optional): the
 * prediction.  Returns sum_frames(loss). */
double FN(dgen_oracle_harmonic_step)(const float* X, const REAL* P, const float* f0, const float* uv,
                                     const float* tgt, int B, int F, int T, int K, int NF, int din, int hid,
                                     int layers, float sr, float hscale, float nscale, const int* sizes,
                                     int n_sizes, int hop_div, float w_lin, float w_log, float max_frames,
                                     int mode, float w_mse, REAL* dP, float* y_out) {
  const int NC = K + 2 + NF;
  const int M = B * F;
  REAL* ctrl = (REAL*)malloc(sizeof(REAL) * (size_t)M * NC);
  REAL* y = (REAL*)malloc(sizeof(REAL) * (size_t)B * T);
  REAL* tr = to_real(tgt, (size_t)B * T);
  REAL* lf = (REAL*)malloc(sizeof(REAL) * T);
  mlp_forward(X, P, M, din, hid, layers, K, NF, NULL, NULL, ctrl);
  synth_core(ctrl, f0, uv, B, F, T, K, NF, sr, sr, hscale, nscale, y, NULL, NULL);
  if (y_out) to_float(y, (size_t)B * T, y_out);
  double tot;
  if (dP) {
    REAL* dy = (REAL*)malloc(sizeof(REAL) * (size_t)B * T);
    REAL* dc = (REAL*)malloc(sizeof(REAL) * (size_t)M * NC);
    tot = mss_core(y, tr, B, T, sizes, n_sizes, hop_div, w_lin, w_log, max_frames, mode, w_mse, lf, dy);
    synth_core(ctrl, f0, uv, B, F, T, K, NF, sr, sr, hscale, nscale, NULL, dy, dc);
    mlp_backward(X, P, dc, M, din, hid, layers, K, NF, dP);
    free(dy);
    free(dc);
  } else {
    tot = mss_core(y, tr, B, T, sizes, n_sizes, hop_div, w_lin, w_log, max_frames, mode, w_mse, lf, NULL);
  }
  free(ctrl);
  free(y);
  free(tr);
  free(lf);
  return tot;
}

/* Adam.step: Sources/DGenLazy/Optimizers.swift:164-204 (bias corrections in
 * Float, update p -= lr*mHat/(sqrt(vHat)+eps)). step = t after increment. */
void FN(dgen_oracle_adam)(float* p, const float* g, float* m, float* v, size_t n, float lr, float b1, float b2,
                          float eps, int step) {
  float bc1 = 1.0f - powf(b1, (float)step);
  float bc2 = 1.0f - powf(b2, (float)step);
  for (size_t j = 0; j < n; ++j) {
    REAL gj = g[j];
    REAL mj = (REAL)b1 * (REAL)m[j] + ((REAL)1 - (REAL)b1) * gj;
    REAL vj = (REAL)b2 * (REAL)v[j] + ((REAL)1 - (REAL)b2) * gj * gj;
    REAL mh = mj / (REAL)bc1, vh = vj / (REAL)bc2;
    p[j] = (float)((REAL)p[j] - (REAL)lr * mh / (R_SQRT(vh) + (REAL)eps));
    m[j] = (float)mj;
    v[j] = (float)vj;
  }
}

/* ------------------------------------------------------------------------ */
/* Temporal gradient of stateful accumulators (phasor, accum).              */
/* ------------------------------------------------------------------------ */

/* The reset-aware exclusive suffix scan of Emit+TemporalGradient.swift:56-81
 * (temporalIncrementGradient, Gradients.swift:209-261): per element, frames
 * in reverse, active = reset[n] > 0 ? 0 : carry; out[n] = active;
 * carry = g[n] + active.  out[n] is d(sum of g . y)/d increment[n] for an
 * accumulator whose output y[n] is the state before frame n's increment.
 * g, out: [T][E]; reset: [T] or NULL.  fp32, the reference's order. */
void dgen_oracle_temporal_scan(const float* g, const float* reset, int T, int E, float* out);
#ifdef ORACLE_COMMON
void dgen_oracle_temporal_scan(const float* g, const float* reset, int T, int E, float* out) {
  for (int e = 0; e < E; ++e) {
    float carry = 0.0f;
    for (int n = T - 1; n >= 0; --n) {
      const float active = (reset && reset[n] > 0.0f) ? 0.0f : carry;
      out[(size_t)n * E + e] = active;
      carry = g[(size_t)n * E + e] + active;
    }
  }
}
#endif

/* The swept-phasor bank of Tests/DGenLazyTests/TemporalGradientTests.swift:
 * 24-60, per lane e: time = accum(1/sr) (fp32, data), frequency
 * f[n] = base + slope[e] * time[n], phase = statefulPhasor(f, reset) (the
 * u_phasor / u_accum order of Definitions.swift:96-102, 215-246, in this
 * build's precision), loss = sum over frames and lanes of
 * (phase - target)^2 (u_mse, Definitions.swift:206-213), or with smooth = 1 of
 * (sin(2 pi phase) - target)^2.  reset[n] = 1 for
 * n >= reset_from (reset_from < 0: never).  With grad != NULL the gradient
 * d loss / d slope[e]: upstream 2 (phase - target), the temporal scan above
 * (with the scan's increment gradient divided by sr, the phasor's
 * scaleBySampleRate), times d f / d slope = time[n], summed over frames.
 * phase_out (optional): [T][E].  Returns the loss. */
double FN(dgen_oracle_swept_phasor_step)(const REAL* slope, int E, int T, float sr, float base, float target,
                                         int reset_from, int smooth, REAL* grad, float* phase_out) {
  float* time = (float*)malloc(sizeof(float) * T);
  {
    float st = 0.0f;
    const float step = 1.0f / sr; /* Signal.constant(1.0 / sampleRate), a Float */
    for (int n = 0; n < T; ++n) {
      float acc = st;
      float next = acc + step;
      float w = next - floorf(next / 1.0f) * 1.0f;
      if (w >= 1.0f) w = w - 1.0f;
      st = w;
      time[n] = acc;
    }
  }
  REAL* gup = grad ? (REAL*)malloc(sizeof(REAL) * (size_t)T * E) : NULL;
  double loss = 0.0;
  for (int e = 0; e < E; ++e) {
    REAL ph = 0;
    for (int n = 0; n < T; ++n) {
      const int rs = reset_from >= 0 && n >= reset_from;
      const REAL f = (REAL)base + slope[e] * (REAL)time[n];
      const REAL acc = ph;
      REAL next = rs ? (REAL)0 : acc + f / (REAL)sr;
      REAL w = next - R_FLOOR(next);
      if (w >= (REAL)1) w = w - (REAL)1;
      if (rs) w = 0;
      ph = w;
      /* smooth: the loss reads sin(2 pi phase) (CRenderer.swift:825-827),
       * which the phase's wrap leaves continuous */
      const REAL v = smooth ? R_SIN(acc * TWO_PI_F32) : acc;
      const REAL d = v - (REAL)target;
      loss += (double)(d * d);
      if (phase_out) phase_out[(size_t)n * E + e] = (float)acc;
      if (gup) gup[(size_t)n * E + e] = smooth ? (REAL)2 * d * (R_COS(acc * TWO_PI_F32) * TWO_PI_F32) : (REAL)2 * d;
    }
  }
  if (grad) {
    for (int e = 0; e < E; ++e) {
      REAL carry = 0, sum = 0;
      for (int n = T - 1; n >= 0; --n) {
        const int rs = reset_from >= 0 && n >= reset_from;
        const REAL active = rs ? (REAL)0 : carry;
        sum = sum + (active / (REAL)sr) * (REAL)time[n];
        carry = gup[(size_t)n * E + e] + active;
      }
      grad[e] = sum;
    }
    free(gup);
  }
  free(time);
  return loss;
}

/* ------------------------------------------------------------------------ */
/* Config 4: tensor biquad bank, forward and BPTT adjoint.                  */
/* ------------------------------------------------------------------------ */


/* w0 per Hz: the reference hardcodes 2*pi/44100 as a Float constant
 * (Sources/DGen/HigherOps.swift:446-447), whatever the graph's sample rate. */
#define BQ_W0_PER_HZ ((REAL)0.00014247585730565955f)

typedef struct {
  REAL c, s, q, alpha, r, P, D;  /* cos, sin, |Q|, div18, recip24, div11, add10 */
  REAL b0, b1, b2, a1, a2;
} BqCoef;

/* RBJ low-pass coefficients (mode 0, gain 1) in the reference graph's
 * operation order, node names as in Sources/DGen/HigherOps.swift:443-556:
 * selector(mode+1 == 1, ...) picks the first option and the shelf branch
 * (mode >= 6) is not taken.  mult26 = recip24 * gain with gain = 1. */
static inline void bq_coef(REAL fc, REAL Q, BqCoef* k) {
  REAL abs6 = R_ABS(fc);
  REAL mult7 = abs6 * BQ_W0_PER_HZ;
  REAL cos8 = R_COS(mult7);
  REAL mult9 = cos8 * (REAL)-1;
  REAL add10 = mult9 + (REAL)1;
  REAL div11 = add10 / (REAL)2;
  REAL sin14 = R_SIN(mult7);
  REAL mult15 = sin14 * (REAL)0.5;
  REAL abs17 = R_ABS(Q);
  REAL div18 = mult15 / abs17;
  REAL add22 = div18 + (REAL)1;
  REAL recip24 = (REAL)1 / add22;
  REAL mult26 = recip24 * (REAL)1;
  REAL mult31 = mult9 * (REAL)2;
  REAL not_sub35 = (REAL)1 - div18;
  k->c = cos8;
  k->s = sin14;
  k->q = abs17;
  k->alpha = div18;
  k->r = recip24;
  k->P = div11;
  k->D = add10;
  k->b2 = div11 * mult26;           /* selector23 -> b2_scaled */
  k->b1 = add10 * mult26;           /* selector32 -> b1_scaled */
  k->b0 = div11 * mult26;           /* selector36 -> b0_scaled */
  k->a2 = not_sub35 * recip24;      /* a2_orig */
  k->a1 = mult31 * recip24;         /* a1_orig */
}

/* One Direct Form I step, HigherOps.swift:535-568: history3 = x[n-2],
 * history2 = x[n-1], history0 = y[n-2], history1 = y[n-1]. */
static inline REAL bq_step(const BqCoef* k, REAL x0, REAL x1, REAL x2, REAL y1, REAL y2) {
  REAL mult28 = x2 * k->b2;
  REAL mult34 = x1 * k->b1;
  REAL mult38 = x0 * k->b0;
  REAL add39 = (mult28 + mult34) + mult38;
  REAL mult42 = y2 * k->a2;
  REAL mult44 = y1 * k->a1;
  REAL add45 = mult42 + mult44;
  return add39 - add45;
}

/* cutoff[n][k] = base[k] * m[n] (the per-lane base times the shared
 * modulation signal; m == NULL means unmodulated).  The product is the
 * graph's `mul` node, so it is rounded in this build's precision. */
static inline REAL bq_cutoff(const float* m, const REAL* base, int n, int k) {
  return m ? base[k] * (REAL)m[n] : base[k];
}

/* Forward of the bank from the history state st ([B][4]: x[n-1], x[n-2],
 * y[n-1], y[n-2] per lane, updated in place): x, y are [T][B] (frame-major,
 * lane-minor). */
static void bq_forward_state(const float* x, const float* m, const REAL* base, const REAL* Q, int B, int T, REAL* st,
                             REAL* y) {
  for (int n = 0; n < T; ++n) {
    for (int k = 0; k < B; ++k) {
      REAL* s = st + 4 * k;
      BqCoef c;
      bq_coef(bq_cutoff(m, base, n, k), Q[k], &c);
      REAL x0 = (REAL)x[(size_t)n * B + k];
      REAL v = bq_step(&c, x0, s[0], s[1], s[2], s[3]);
      s[1] = s[0];
      s[0] = x0;
      s[3] = s[2];
      s[2] = v;
      y[(size_t)n * B + k] = v;
    }
  }
}

/* From zero state (history cells zeroed by zeroAllBuffers). */
static void bq_forward(const float* x, const float* m, const REAL* base, const REAL* Q, int B, int T, REAL* y) {
  REAL* st = (REAL*)calloc((size_t)4 * B, sizeof(REAL)); /* x1 x2 y1 y2 per lane */
  bq_forward_state(x, m, base, Q, B, T, st, y);
  free(st);
}

/* One block of the bank as a streaming process call (dgen_process_v1 with
 * realize(preserveState: true), Sources/DGenLazy/Realize.swift:553-563): the
 * history cells state[B][4] carry over from the previous call; m: this
 * block's modulation (or NULL); y: the block's outputs, non-finite stored as
 * 0 (CRenderer.swift:1021-1039) while the history keeps the raw value. */
void FN(dgen_oracle_biquad_stream)(const float* x, const float* m, const REAL* base, const REAL* Q, int B, int T,
                                   REAL* state, float* y_out) {
  REAL* y = (REAL*)malloc(sizeof(REAL) * (size_t)B * T);
  bq_forward_state(x, m, base, Q, B, T, state, y);
  for (size_t i = 0; i < (size_t)B * T; ++i) y_out[i] = (float)sanitize(y[i]);
  free(y);
}

void FN(dgen_oracle_biquad_fwd)(const float* x, const float* m, const REAL* base, const REAL* Q, int B, int T,
                                float* y_out) {
  REAL* y = (REAL*)malloc(sizeof(REAL) * (size_t)B * T);
  bq_forward(x, m, base, Q, B, T, y);
  to_float(y, (size_t)B * T, y_out);
  free(y);
}

/* One config-4 training step in this build's precision: forward, loss
 * sum_n sum_k (y - tgt)^2 (u_mse per element, Sources/DGen/Definitions.swift:
 * 206-213, summed over lanes and frames), and (grad != NULL) the BPTT
 * gradient [2][B] = (d/d base_k, d/d Q_k).
 *
 * Adjoint: with g[n] = 2 (y[n] - tgt[n]) and lambda[n] = dL/dy[n] in total,
 *   lambda[n] = g[n] - a1[n+1] lambda[n+1] - a2[n+2] lambda[n+2],
 * run backwards with two carries (v1, v2) = the contributions already owed
 * to lambda[n-1] and lambda[n-2].  The coefficient derivatives follow the
 * chain rule through the nodes of bq_coef (pinned by finite differences of
 * this function's fp64 build). */
double FN(dgen_oracle_biquad_step)(const float* x, const float* m, const REAL* base, const REAL* Q,
                                   const float* tgt, int B, int T, float* y_out, REAL* grad) {
  const size_t N = (size_t)B * T;
  REAL* y = (REAL*)malloc(sizeof(REAL) * N);
  bq_forward(x, m, base, Q, B, T, y);
  if (y_out) to_float(y, N, y_out);
  double loss = 0.0;
  for (size_t i = 0; i < N; ++i) {
    REAL d = y[i] - (REAL)tgt[i];
    loss += (double)(d * d);
  }
  if (grad) {
    REAL* v = (REAL*)calloc((size_t)2 * B, sizeof(REAL));
    for (int k = 0; k < 2 * B; ++k) grad[k] = 0;
    for (int n = T - 1; n >= 0; --n) {
      for (int k = 0; k < B; ++k) {
        const size_t i = (size_t)n * B + k;
        REAL fc = bq_cutoff(m, base, n, k);
        BqCoef c;
        bq_coef(fc, Q[k], &c);
        REAL x0 = (REAL)x[i];
        REAL x1 = n >= 1 ? (REAL)x[i - B] : 0;
        REAL x2 = n >= 2 ? (REAL)x[i - 2 * (size_t)B] : 0;
        REAL y1 = n >= 1 ? y[i - B] : 0;
        REAL y2 = n >= 2 ? y[i - 2 * (size_t)B] : 0;
        REAL lam = (REAL)2 * (y[i] - (REAL)tgt[i]) + v[2 * k];
        v[2 * k] = v[2 * k + 1] - c.a1 * lam;
        v[2 * k + 1] = -c.a2 * lam;
        /* dL/d(coefficient) at this frame */
        REAL gb0 = lam * x0, gb2 = lam * x2, gb1 = lam * x1;
        REAL ga1 = -lam * y1, ga2 = -lam * y2;
        /* b0 = b2 = P r, b1 = D r, a1 = (-2c) r, a2 = (1 - alpha) r */
        REAL dr = (gb0 + gb2) * c.P + gb1 * c.D + ga1 * ((REAL)-2 * c.c) + ga2 * ((REAL)1 - c.alpha);
        REAL dP = (gb0 + gb2) * c.r;
        REAL dD = gb1 * c.r + dP / (REAL)2;
        REAL dc = -dD + ga1 * ((REAL)-2 * c.r);
        REAL dalpha = -ga2 * c.r - dr * c.r * c.r;
        REAL ds = dalpha * (REAL)0.5 / c.q;
        REAL dq = -dalpha * c.alpha / c.q;
        REAL dw = -c.s * dc + c.c * ds;
        REAL dfc = dw * BQ_W0_PER_HZ * r_sign(fc);
        grad[k] += dfc * (m ? (REAL)m[n] : (REAL)1);
        grad[B + k] += dq * r_sign(Q[k]);
      }
    }
    free(v);
  }
  free(y);
  return loss;
}

/* ------------------------------------------------------------------------ */
/* Two-cell ZDF state-variable filter bank (low-pass) and its BPTT.         */
/* ------------------------------------------------------------------------ */

/* The hand-rolled Cytomic/TPT SVF of Tests/DGenLazyTests/
 * SVFBPTTScratchTests.swift:21-34 (the MonologueVoice filter): two history
 * cells ic1, ic2 written with pass-through values, soft saturation
 * s = ic / (1 + |kSat ic|), and the cutoff drive of :56-63,
 * (fBase + envelope).clip(20, 20000) -> g = tan((pi * fc) / sr).  Per lane k
 * and frame n, in the graph's node order:
 *   fc  = clip(base[k] * m[n] + env[n], 20, 20000)   (m = 1, env = 0 if absent;
 *         clip = max(min(v, 20000), 20), Functions.swift:780-782)
 *   g   = tan((pi * fc) / sr);  kd = 1 / res[k]
 *   a1  = 1 / (1 + g * (g + kd));  a2 = g * a1
 *   s1  = ic1 / (1 + |ks ic1|);  s2 = ic2 / (1 + |ks ic2|)
 *   v3  = x - s2;  v1 = a1 s1 + a2 v3
 *   ic1 <- 2 v1 - s1;  v1p = (ic1 + s1) * 0.5
 *   v2  = s2 + g v1p;  ic2 <- 2 v2 - s2
 *   y   = (ic2 + s2) * 0.5
 * pi and sr enter as Float constants.  With ks = 0 this is the TPT low-pass
 * H(s) = 1 / (s^2 + kd s + 1) under the prewarped bilinear transform. */
typedef struct {
  REAL g, kd, a1, a2, u, Q;
  int pass; /* the clip passes its input's gradient */
} SvfCoef;

#define SVF_PI ((REAL)3.14159265358979323846f)

static inline void svf_coef(REAL raw, REAL kd, float sr, SvfCoef* c) {
  const REAL fc = r_max(r_min(raw, (REAL)20000), (REAL)20);
  /* min passes for raw <= hi, max for min(raw, hi) >= lo (Gradients.swift:386-410) */
  c->pass = raw <= (REAL)20000 && r_min(raw, (REAL)20000) >= (REAL)20;
  c->u = (SVF_PI * fc) / (REAL)sr;
  c->g = R_TAN(c->u);
  c->kd = kd;
  c->Q = (REAL)1 + c->g * (c->g + kd);
  c->a1 = (REAL)1 / c->Q;
  c->a2 = c->g * c->a1;
}

static inline REAL svf_raw_cutoff(const float* m, const float* env, REAL base, int n) {
  REAL v = base * (m ? (REAL)m[n] : (REAL)1);
  return env ? v + (REAL)env[n] : v;
}

static inline REAL svf_sat(REAL c, REAL ks) { return c / ((REAL)1 + R_ABS(ks * c)); }

/* One frame: state (c1, c2) -> next state; returns y. */
static inline REAL svf_frame(const SvfCoef* k, REAL ks, REAL x, REAL* c1, REAL* c2) {
  const REAL s1 = svf_sat(*c1, ks), s2 = svf_sat(*c2, ks);
  const REAL v3 = x - s2;
  const REAL v1 = k->a1 * s1 + k->a2 * v3;
  const REAL ic1 = (REAL)2 * v1 - s1;
  const REAL v1p = (ic1 + s1) * (REAL)0.5;
  const REAL v2 = s2 + k->g * v1p;
  const REAL ic2 = (REAL)2 * v2 - s2;
  *c1 = ic1;
  *c2 = ic2;
  return (ic2 + s2) * (REAL)0.5;
}

/* Forward over [T][B] lanes from state[2][B] (ic1 | ic2, updated in place;
 * NULL: zero state).  ks NULL: kSat is the constant 0.  states (optional,
 * [2][T][B]): the cells entering every frame. */
static void svf_forward(const float* x, const float* m, const float* env, const REAL* base, const REAL* res,
                        const REAL* ks, int B, int T, float sr, REAL* state, REAL* y, REAL* states) {
  /* lanes are independent: each runs its frames in order on one thread */
#pragma omp parallel for schedule(static)
  for (int k = 0; k < B; ++k) {
    REAL c1 = state ? state[k] : 0, c2 = state ? state[B + k] : 0;
    const REAL kd = (REAL)1 / res[k];
    const REAL kk = ks ? ks[k] : (REAL)0;
    for (int n = 0; n < T; ++n) {
      const size_t i = (size_t)n * B + k;
      SvfCoef c;
      svf_coef(svf_raw_cutoff(m, env, base[k], n), kd, sr, &c);
      if (states) {
        states[i] = c1;
        states[(size_t)T * B + i] = c2;
      }
      y[i] = svf_frame(&c, kk, (REAL)x[i], &c1, &c2);
    }
    if (state) {
      state[k] = c1;
      state[B + k] = c2;
    }
  }
}

void FN(dgen_oracle_svf_fwd)(const float* x, const float* m, const float* env, const REAL* base, const REAL* res,
                             const REAL* ks, int B, int T, float sr, REAL* state, float* y_out) {
  REAL* y = (REAL*)malloc(sizeof(REAL) * (size_t)B * T);
  svf_forward(x, m, env, base, res, ks, B, T, sr, state, y, NULL);
  to_float(y, (size_t)B * T, y_out);
  free(y);
}

/* Forward, loss = sum (y - tgt)^2 over frames and lanes, and (grad, [3][B] =
 * d/d base | d/d res | d/d ks; the last is 0 when ks is NULL) the BPTT
 * gradient: the reverse-time adjoint (lambda1, lambda2) of the two cells
 * through every node above, reading the stored cells of each frame (the
 * reference's stored-forward-value reverse loop, BPTTEmission.swift:133-160,
 * with the per-node rules of Gradients.swift: abs -> sign, min/max ->
 * pass masks, tan -> 1/(cos cos), div).  xbar (optional, [T][B]) = d loss /
 * d x. */
double FN(dgen_oracle_svf_step)(const float* x, const float* m, const float* env, const REAL* base,
                                const REAL* res, const REAL* ks, const float* tgt, int B, int T, float sr,
                                float* y_out, REAL* grad, REAL* xbar) {
  const size_t N = (size_t)B * T;
  REAL* y = (REAL*)malloc(sizeof(REAL) * N);
  REAL* st = grad || xbar ? (REAL*)malloc(sizeof(REAL) * 2 * N) : NULL;
  svf_forward(x, m, env, base, res, ks, B, T, sr, NULL, y, st);
  if (y_out) to_float(y, N, y_out);
  double loss = 0.0;
  for (size_t i = 0; i < N; ++i) {
    const REAL d = y[i] - (REAL)tgt[i];
    loss += (double)(d * d);
  }
  if (st) {
#pragma omp parallel for schedule(static)
    for (int k = 0; k < B; ++k) {
      const REAL kd = (REAL)1 / res[k];
      const REAL kk = ks ? ks[k] : (REAL)0;
      REAL l1 = 0, l2 = 0, gb = 0, gkd = 0, gks = 0;
      for (int n = T - 1; n >= 0; --n) {
        const size_t i = (size_t)n * B + k;
        SvfCoef c;
        svf_coef(svf_raw_cutoff(m, env, base[k], n), kd, sr, &c);
        const REAL c1 = st[i], c2 = st[N + i];
        const REAL D1 = (REAL)1 + R_ABS(kk * c1), D2 = (REAL)1 + R_ABS(kk * c2);
        const REAL s1 = c1 / D1, s2 = c2 / D2;
        const REAL v3 = (REAL)x[i] - s2;
        const REAL v1 = c.a1 * s1 + c.a2 * v3;
        const REAL ic1 = (REAL)2 * v1 - s1;
        const REAL v1p = (ic1 + s1) * (REAL)0.5;
        /* adjoints, last node first */
        const REAL e = (REAL)2 * (y[i] - (REAL)tgt[i]);
        const REAL ic2_b = (REAL)0.5 * e + l2;
        REAL s2_b = (REAL)0.5 * e - ic2_b;
        const REAL v2_b = (REAL)2 * ic2_b;
        s2_b += v2_b;
        REAL g_b = v2_b * v1p;
        const REAL v1p_b = v2_b * c.g;
        const REAL ic1_b = l1 + (REAL)0.5 * v1p_b;
        REAL s1_b = (REAL)0.5 * v1p_b - ic1_b;
        const REAL v1_b = (REAL)2 * ic1_b;
        REAL a1_b = v1_b * s1;
        s1_b += v1_b * c.a1;
        const REAL a2_b = v1_b * v3;
        const REAL v3_b = v1_b * c.a2;
        if (xbar) xbar[i] = v3_b;
        s2_b -= v3_b;
        /* s = c / D, D = 1 + |ks c|: ds/dc = 1/D - (c/D^2) sgn(ks c) ks, ds/dks = -(c/D^2) sgn(ks c) c */
        const REAL q1 = (c1 / (D1 * D1)) * r_sign(kk * c1), q2 = (c2 / (D2 * D2)) * r_sign(kk * c2);
        l1 = s1_b * ((REAL)1 / D1 - q1 * kk);
        l2 = s2_b * ((REAL)1 / D2 - q2 * kk);
        gks += -(s1_b * q1 * c1) - s2_b * q2 * c2;
        g_b += a2_b * c.a1;
        a1_b += a2_b * c.g;
        /* a1 = 1 / Q, Q = 1 + g (g + kd) */
        const REAL Q_b = -a1_b / (c.Q * c.Q);
        g_b += Q_b * ((c.g + c.kd) + c.g);
        gkd += Q_b * c.g;
        /* g = tan(u), u = (pi fc) / sr */
        const REAL cu = R_COS(c.u);
        const REAL u_b = g_b * ((REAL)1 / (cu * cu));
        const REAL fc_b = (u_b / (REAL)sr) * SVF_PI;
        if (c.pass) gb += fc_b * (m ? (REAL)m[n] : (REAL)1);
      }
      if (grad) {
        grad[k] = gb;
        grad[B + k] = gkd * (-(REAL)1 / (res[k] * res[k]));
        grad[2 * B + k] = ks ? gks : (REAL)0;
      }
    }
    free(st);
  }
  free(y);
  return loss;
}

/* ------------------------------------------------------------------------ */
/* Config 2: hop-gated STFT round trip with learnable per-bin gains.        */
/* ------------------------------------------------------------------------ */

/* tensorFFT / tensorIFFT (Sources/DGen/HigherOps+FFT.swift:16-123): bit
 * reversal by reshape/transpose, then log2 N radix-2 stages on blocks
 * [blocks][2][half] with twiddle w[j] = (cos a, sin a),
 * a = sign * 2 * Float.pi * Float(j) / Float(2*half) evaluated in Float
 * (:84-91); t = odd * w, top = even + t, bot = even - t. */
typedef struct {
  int n, stages;
  float* twre; /* [stage half-1 + j], cos a (same for both signs) */
  float* twim; /* sin a for the positive (inverse) angle */
  int* bitrev;
} TfPlan;

static void tf_plan_init(TfPlan* p, int n) {
  p->n = n;
  p->stages = 0;
  while ((1 << p->stages) < n) p->stages++;
  p->twre = (float*)malloc(sizeof(float) * (n > 1 ? n - 1 : 1));
  p->twim = (float*)malloc(sizeof(float) * (n > 1 ? n - 1 : 1));
  p->bitrev = (int*)malloc(sizeof(int) * n);
  const float two_pi = 2.0f * 3.14159265358979323846f;
  for (int s = 0; s < p->stages; ++s) {
    int half = 1 << s;
    for (int j = 0; j < half; ++j) {
      float ang = two_pi * (float)j / (float)(2 * half);
      p->twre[half - 1 + j] = cosf(ang);
      p->twim[half - 1 + j] = sinf(ang);
    }
  }
  for (int i = 0; i < n; ++i) {
    int rev = 0, bits = i;
    for (int s = 0; s < p->stages; ++s) {
      rev = rev * 2 + (bits & 1);
      bits >>= 1;
    }
    p->bitrev[i] = rev;
  }
}

static void tf_plan_free(TfPlan* p) {
  free(p->twre);
  free(p->twim);
  free(p->bitrev);
}

/* In place; inverse: positive angles and the 1/N scale of tensorIFFT. */
static void tf_fft(const TfPlan* p, REAL* re, REAL* im, int inverse) {
  const int n = p->n;
  for (int i = 0; i < n; ++i) {
    int r = p->bitrev[i];
    if (i < r) {
      REAL a = re[i];
      re[i] = re[r];
      re[r] = a;
      a = im[i];
      im[i] = im[r];
      im[r] = a;
    }
  }
  for (int s = 0; s < p->stages; ++s) {
    const int half = 1 << s, size = 2 * half;
    for (int b = 0; b < n / size; ++b) {
      for (int j = 0; j < half; ++j) {
        const REAL wr = (REAL)p->twre[half - 1 + j];
        const REAL wi = inverse ? (REAL)p->twim[half - 1 + j] : -(REAL)p->twim[half - 1 + j];
        const int e = b * size + j, o = e + half;
        const REAL t_re = re[o] * wr - im[o] * wi;
        const REAL t_im = re[o] * wi + im[o] * wr;
        const REAL er = re[e], ei = im[e];
        re[e] = er + t_re;
        im[e] = ei + t_im;
        re[o] = er - t_re;
        im[o] = ei - t_im;
      }
    }
  }
  if (inverse) {
    const REAL sc = (REAL)(1.0f / (float)n);
    for (int i = 0; i < n; ++i) {
      re[i] *= sc;
      im[i] *= sc;
    }
  }
}

void FN(dgen_oracle_tensor_fft)(int n, int inverse, REAL* re, REAL* im) {
  TfPlan p;
  tf_plan_init(&p, n);
  tf_fft(&p, re, im, inverse);
  tf_plan_free(&p);
}

/* The gain applied to bin k of the full N-point spectrum: the one-sided
 * Hermitian reconstruction g0, 2 g_k (0 < k < N/2), g_{N/2}, 0 above. */
static inline REAL stft_gain(const REAL* g, int N, int k) {
  if (k == 0 || k == N / 2) return g[k];
  return k < N / 2 ? (REAL)2 * g[k] : (REAL)0;
}

/* One config-2 step over S signals x [S][T]:
 *   hop frames h = 0, H, 2H, ... < T (bufferView's counter fires on 0,
 *   HigherOps.swift:770-783); window a[i] = win[i] * x[h-N+1+i], zero before
 *   frame 0 (the ring starts zeroed, HigherOps.swift:738-765);
 *   X = tensorFFT(a); X'[k] = X[k] * stft_gain(k); z = tensorIFFT(X');
 *   overlapAdd (Emit+FFT.swift:6-62): y[t] = sum_h z_h[t-h], 0 <= t-h < N.
 * loss = sum_s sum_t (y - x)^2 / T.  dg (optional, [N/2+1]):
 *   dL/dg_k = sum_h (c_k/N) Re(X_h[k] conj(E_h[k])), E_h = tensorFFT of the
 *   output gradient over the window's outputs, c_k = 1 (k = 0, N/2) or 2:
 * the derivative of the forward above (pinned by finite differences).  The
 * reference's own overlapAdd backward reads element 0's gradient from frame
 * h+N instead of h (Emit+FFT.swift:93-97); this function does not follow it. */
double FN(dgen_oracle_stft_step)(const float* x, int S, int T, int N, int H, const float* win, const REAL* g,
                                 float* y_out, REAL* dg) {
  TfPlan p;
  tf_plan_init(&p, N);
  REAL* re = (REAL*)malloc(sizeof(REAL) * N);
  REAL* im = (REAL*)malloc(sizeof(REAL) * N);
  REAL* y = (REAL*)malloc(sizeof(REAL) * (size_t)T);
  REAL* ere = dg ? (REAL*)malloc(sizeof(REAL) * N) : NULL;
  REAL* eim = dg ? (REAL*)malloc(sizeof(REAL) * N) : NULL;
  if (dg)
    for (int k = 0; k <= N / 2; ++k) dg[k] = 0;
  double loss = 0.0;
  for (int s = 0; s < S; ++s) {
    const float* xs = x + (size_t)s * T;
    for (int t = 0; t < T; ++t) y[t] = 0;
    for (int h = 0; h < T; h += H) {
      for (int i = 0; i < N; ++i) {
        const int t = h - N + 1 + i;
        re[i] = (REAL)win[i] * (t >= 0 ? (REAL)xs[t] : (REAL)0);
        im[i] = 0;
      }
      tf_fft(&p, re, im, 0);
      for (int k = 0; k < N; ++k) {
        const REAL gk = stft_gain(g, N, k);
        re[k] *= gk;
        im[k] *= gk;
      }
      tf_fft(&p, re, im, 1);
      for (int i = 0; i < N && h + i < T; ++i) y[h + i] += re[i];
    }
    for (int t = 0; t < T; ++t) {
      const REAL d = y[t] - (REAL)xs[t];
      loss += (double)(d * d) / (double)T;
      if (y_out) y_out[(size_t)s * T + t] = (float)y[t];
    }
    if (!dg) continue;
    /* dL/dy = 2 (y - x) / T; recompute each window's spectrum */
    for (int h = 0; h < T; h += H) {
      for (int i = 0; i < N; ++i) {
        const int t = h - N + 1 + i;
        re[i] = (REAL)win[i] * (t >= 0 ? (REAL)xs[t] : (REAL)0);
        im[i] = 0;
        const int u = h + i;
        ere[i] = u < T ? (REAL)2 * (y[u] - (REAL)xs[u]) / (REAL)T : (REAL)0;
        eim[i] = 0;
      }
      tf_fft(&p, re, im, 0);
      tf_fft(&p, ere, eim, 0);
      for (int k = 0; k <= N / 2; ++k) {
        const REAL ck = (k == 0 || k == N / 2) ? (REAL)1 : (REAL)2;
        dg[k] += ck / (REAL)N * (re[k] * ere[k] + im[k] * eim[k]);
      }
    }
  }
  free(re);
  free(im);
  free(y);
  free(ere);
  free(eim);
  tf_plan_free(&p);
  return loss;
}

/* ------------------------------------------------------------------------ */
/* Config 5: 2D membrane (damped wave equation on an R x C grid).           */
/* ------------------------------------------------------------------------ */

/* 3x3 Laplacian [[0,1,0],[1,-4,1],[0,1,0]] as conv2d "same" with zero
 * padding (Sources/DGen/Emit+Tensor.swift:173-205; the pad + conv2d form of
 * Examples/BendingMetal/main.swift:114-121 gives the same values): the taps
 * accumulate ky-major from 0; zero taps add nothing. */
static inline REAL mem_lap(const REAL* u, int R, int C, int y, int x) {
  const size_t i = (size_t)y * C + x;
  REAL n = y > 0 ? u[i - C] : (REAL)0;
  REAL w = x > 0 ? u[i - 1] : (REAL)0;
  REAL e = x + 1 < C ? u[i + 1] : (REAL)0;
  REAL s = y + 1 < R ? u[i + C] : (REAL)0;
  return (((n + w) + u[i] * (REAL)-4) + e) + s;
}

/* u_next = 2 u - u1 + c2 L(u) - d (u - u1), evaluated left to right as the
 * graph states it: ((u*2 - u1) + L*c2) - (u - u1)*d. */
static void mem_step(const REAL* u, const REAL* u1, REAL* un, int R, int C, REAL c2, REAL d) {
  for (int y = 0; y < R; ++y)
    for (int x = 0; x < C; ++x) {
      const size_t i = (size_t)y * C + x;
      const REAL b = u[i] * (REAL)2 - u1[i];
      const REAL c = mem_lap(u, R, C, y, x) * c2;
      const REAL g = (u[i] - u1[i]) * d;
      un[i] = (b + c) - g;
    }
}

/* One config-5 training step in this build's precision.  The state history
 * starts at u_{-1} = u_0 = u0 (TensorHistory initial data); frame n reads
 * u_n, u_{n-1} and writes u_{n+1}; the pickup output is out[n] = u_{n+1}[p]
 * (Examples/BendingMetal/main.swift:96-169).  loss = sum_n (out[n] - tgt[n])^2.
 *
 * grad (optional, [2] = d/d c2, d/d d): discrete adjoint.  With L symmetric,
 *   lambda_n = g_n + (2-d) lambda_{n+1} + c2 L lambda_{n+1} - (1-d) lambda_{n+2},
 *   g_n = 2 (out[n-1] - tgt[n-1]) at p, lambda_{T+1} = lambda_{T+2} = 0;
 *   dL/dc2 = sum_n <lambda_n, L u_{n-1}>, dL/dd = sum_n <lambda_n, u_{n-2} - u_{n-1}>
 * for n = T..1.  The states are recomputed from checkpoints every `ck`
 * steps (memory ~ (T/ck + ck) fields). */
double FN(dgen_oracle_membrane_step)(const float* u0, int R, int C, int T, REAL c2, REAL d, int py, int px,
                                     const float* tgt, float* out, REAL* grad) {
  const size_t G = (size_t)R * C;
  const size_t ip = (size_t)py * C + px;
  REAL* a = (REAL*)malloc(sizeof(REAL) * G);
  REAL* b = (REAL*)malloc(sizeof(REAL) * G);
  REAL* cbuf = (REAL*)malloc(sizeof(REAL) * G);
  for (size_t i = 0; i < G; ++i) a[i] = b[i] = (REAL)u0[i];
  int ck = 1;
  while ((long)ck * ck < T) ++ck;
  const int nck = (T + ck - 1) / ck + 1;
  REAL* cks = grad ? (REAL*)malloc(sizeof(REAL) * G * 2 * nck) : NULL; /* (u_{m-1}, u_m) at m = j*ck */
  REAL* o = (REAL*)malloc(sizeof(REAL) * (T > 0 ? T : 1));
  REAL *um1 = a, *u = b, *un = cbuf;  /* u_{n-1}, u_n, u_{n+1} */
  for (int n = 0; n < T; ++n) {
    if (grad && n % ck == 0) {
      memcpy(cks + G * 2 * (n / ck), um1, sizeof(REAL) * G);
      memcpy(cks + G * (2 * (n / ck) + 1), u, sizeof(REAL) * G);
    }
    mem_step(u, um1, un, R, C, c2, d);
    o[n] = un[ip];
    REAL* t = um1;
    um1 = u;
    u = un;
    un = t;
  }
  double loss = 0.0;
  for (int n = 0; n < T; ++n) {
    if (out) out[n] = (float)o[n];
    const REAL e = o[n] - (REAL)tgt[n];
    loss += (double)(e * e);
  }
  if (grad) {
    grad[0] = grad[1] = 0;
    REAL* l1 = (REAL*)calloc(G, sizeof(REAL)); /* lambda_{n+1} */
    REAL* l2 = (REAL*)calloc(G, sizeof(REAL)); /* lambda_{n+2} */
    REAL* seg = (REAL*)malloc(sizeof(REAL) * G * (ck + 1));  /* u_{m-1} .. u_{m+ck-1} */
    for (int m = ((T - 1) / ck) * ck; m >= 0; m -= ck) {
      const int len = (m + ck <= T ? ck : T - m);
      /* states u_{m-1} .. u_{m+len-1} of this segment */
      memcpy(seg, cks + G * 2 * (m / ck), sizeof(REAL) * G);
      memcpy(seg + G, cks + G * (2 * (m / ck) + 1), sizeof(REAL) * G);
      for (int q = 1; q < len; ++q) mem_step(seg + G * q, seg + G * (q - 1), seg + G * (q + 1), R, C, c2, d);
      /* lambda_n for n = m+len .. m+1 needs u_{n-1} = seg[n-m], u_{n-2} = seg[n-1-m] */
      for (int n = m + len; n >= m + 1; --n) {
        const REAL* v1 = seg + G * (size_t)(n - m);
        const REAL* v2 = seg + G * (size_t)(n - 1 - m);
        for (int y = 0; y < R; ++y)
          for (int x = 0; x < C; ++x) {
            const size_t i = (size_t)y * C + x;
            REAL lam = ((REAL)2 - d) * l1[i] + c2 * mem_lap(l1, R, C, y, x) - ((REAL)1 - d) * l2[i];
            if (i == ip) lam += (REAL)2 * (o[n - 1] - (REAL)tgt[n - 1]);
            cbuf[i] = lam;
          }
        for (int y = 0; y < R; ++y)
          for (int x = 0; x < C; ++x) {
            const size_t i = (size_t)y * C + x;
            grad[0] += cbuf[i] * mem_lap(v1, R, C, y, x);
            grad[1] += cbuf[i] * (v2[i] - v1[i]);
          }
        REAL* t = l2;
        l2 = l1;
        l1 = cbuf;
        cbuf = t;
      }
    }
    free(l1);
    free(l2);
    free(seg);
  }
  free(a);
  free(b);
  free(cbuf);
  free(cks);
  free(o);
  return loss;
}
