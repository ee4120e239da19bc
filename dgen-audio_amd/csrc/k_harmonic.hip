// Batched harmonic + FIR-noise synth (HarmonicSynth.renderBatchedSignal,
// Examples/HarmonicE2E/Synth.swift:47-102) and its adjoint.
//
// Time is cut into segments of kSeg = 64 frames.  The only true recurrence
// is the tensor phasor (Sources/DGen/Emit+State.swift:322-369): one lane per
// (batch, harmonic) accumulates phase sequentially in fp32.  k_phasor_carry
// runs that chain once over the whole signal and stores the phase at every
// segment start; the synth kernels restart the chain from those checkpoints,
// so all remaining work is parallel over (segment, batch) and the phases are
// bit-identical to one sequential evaluation.
//
// The chain step is the reference's u_accum/phasor order:
//   inc = freq / sr;  next = ph + inc;  w = next - floor(next);  if (w >= 1) w -= 1
// - freq / sr uses the fma-corrected reciprocal product (q0 = x*r,
//   e = fma(-q0, sr, x), q = fma(e, r, q0)), which equals the IEEE quotient
//   for every normal |x| in [2^-20, 2^24) (checked exhaustively for the
//   sample rates in use by tests/test_fastdiv.py); outside that range the
//   kernel divides.
// - for ph in [0,1) and a finite inc >= 0, next >= 0, next - floor(next) is
//   exact and < 1, so the step is fract(ph + inc) (one v_fract_f32); chunks
//   holding a negative or non-finite increment take the literal form.
//
// Layouts: ctrl rows [B*F][ldc] (row = b*F + f); f0f, uvf [B][T] (frame-rate
// interpolated f0 and uv); lerp [T][8] = lo, hi, frac, 1-frac, slot(lo),
// slot(hi); seg_rows [nseg][4]; checkpoints [nseg][B][K]; noise [T];
// y, dy [B][T]; partials [B][nseg][4][ldc].
#pragma clang fp contract(off)

#include <type_traits>

#include "dev_math.h"
#include "internal.h"

namespace dgen {

constexpr int kSeg = 64;      // frames per segment = checkpoint spacing
constexpr int kSlots = 4;     // distinct control rows a segment may touch
// Harmonics run one per lane, in groups of 64 (a wave's lanes).  The
// narrow layout (one group, <= 128 control columns) is the common case;
// the wide one takes up to four groups and 512 columns, at about twice the
// LDS per wave.
constexpr int kMaxK = 64;        // narrow: harmonics
constexpr int kMaxNC = 128;      // narrow: control columns
constexpr int kMaxKWide = 256;   // wide: harmonics (four groups)
constexpr int kMaxNCWide = 512;  // wide: control columns

__device__ __forceinline__ float phasor_wrap(float next) {
  float w = next - floorf(next);
  return w >= 1.0f ? w - 1.0f : w;
}

// x / sr for a constant sr with r = RN(1/sr): IEEE-exact on the validated range.
__device__ __forceinline__ float div_sr(float x, float sr, float rsr) {
  const float ax = fabsf(x);
  if (ax >= 0x1p-20f && ax < 0x1p24f) {
    const float q0 = x * rsr;
    const float e = fmaf(-q0, sr, x);
    return fmaf(e, rsr, q0);
  }
  return x / sr;
}

// sin(p * 2pi_f32), the expression the reference evaluates
// (CRenderer.swift:825-827), for p in [0, 1): the hardware sine of 2 pi p
// with the first-order correction for the fp32 constant's excess
// (sin_2pif_hw).  Against the reference's own fp32 evaluation,
// sinf(RN(p * 2pi_f32)), it is within 3.0e-7 (rms 7.5e-8; the argument's
// rounding dominates), against the exact sin(p * 2pi_f32) within 1.4e-7.
// The uncorrected sin(2 pi p) put a phase-proportional error into the
// prediction that doubled the gradient's distance from finite differences
// through the log-magnitude loss (B=4, T=64000: the whole gradient 4.2%
// from fp64, against 2.3% with the correction and 2.6% for the fp32
// oracle).
__device__ __forceinline__ float sin2pi(float p) { return sin_2pif_hw(p); }

// ------------------------------------------------------------ frame-rate data
// out[b][t] = (1-frac_t) * src[lo_t][b] + frac_t * src[hi_t][b]: the sampleRow
// read of a [F][B] data table (Emit+RowSelection.swift:164-197).
__global__ void k_lerp_frames(const float* __restrict__ src, const float* __restrict__ lerp, float* __restrict__ out,
                              int B, int T) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (t >= T) return;
  const float4 e = *reinterpret_cast<const float4*>(lerp + (size_t)t * 8);
  const int lo = (int)e.x, hi = (int)e.y;
  out[(size_t)b * T + t] = e.w * src[(size_t)lo * B + b] + e.z * src[(size_t)hi * B + b];
}

int launch_lerp_frames(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=src ([F][B]) [1]=lerp ([T][8]) [2]=out ([B][T]) [3]=B [4]=F [5]=T
  const int64_t src = op.arg[0], lerp = op.arg[1], out = op.arg[2], B = op.arg[3], F = op.arg[4], T = op.arg[5];
  DGEN_REQUIRE(B > 0 && B <= 65535 && F > 0 && T > 0 && T <= (1 << 26), "lerp_frames: B %lld F %lld T %lld",
               (long long)B, (long long)F, (long long)T);
  DGEN_REQUIRE(lerp % 4 == 0, "lerp_frames: lerp table must be 16-byte aligned");
  DGEN_CHECK_CELL(L, src, F * B, "lerp_frames.src");
  DGEN_CHECK_CELL(L, lerp, T * 8, "lerp_frames.lerp");
  DGEN_CHECK_CELL(L, out, B * T, "lerp_frames.out");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_lerp_frames, dim3((unsigned)((T + 255) / 256), (unsigned)B), dim3(256), 0, L.stream,
                     cell(L, src), cell(L, lerp), cell(L, out), (int)B, (int)T);
  DGEN_LAUNCH_CHECK("k_lerp_frames");
  return 0;
}

// ------------------------------------------------------------ carry pass
// One workgroup per batch lane b.  Wave 0 runs the K phase chains
// (lane = k); at 2 dependent VALU ops per step its 64-step segment costs
// ~128 issue slots, so everything else is kept off its path:
// - waves 1..kProducers compute increments into a ring of kCarryBufs
//   segment buffers, kIv segments per barrier interval, kIv + 1 segments
//   ahead of the chain, so the chain reads the next interval's first
//   segment before the barrier that ends its interval and steps on from
//   registers after it; producer p owns float4 frame groups
//   kSplit[p] .. kSplit[p+1]-1 of every segment, lane = k;
// - a producer's time goes to the latency of its LDS reads and increment
//   chains, not to issue: measured against the chain, four producers of
//   four groups each had ~12% slack, five groups left none and six made
//   the producer the bound; seven producers (two or three groups, two
//   waves on most SIMDs, overlapping each other's latency) give the chain
//   the most room (331 against 339 us alone for four);
// - increments are stored k-major ([k][frame], stride 68 floats), so the
//   chain reads a lane's 64 increments with 16 ds_read_b128 and producers
//   write them with ds_write_b128, both bank-conflict free;
// - f0 is staged from global memory kRing segments at a time into a
//   double-buffered LDS ring, a block's loads issued an interval before
//   they are committed, so load latency is paid once per block and hidden;
//   the fast-step test (every f0 of the block in the exact range) is voted
//   once per block while committing it;
// - the chain wave reads segment s+1's increments into registers while it
//   steps segment s, and has issue priority on its SIMD.
constexpr int kProducers = 7;
constexpr int kCarryWaves = 1 + kProducers;
// A segment's 16 float4 frame groups over the producers
constexpr int kSplit[kProducers + 1] = {0, 2, 4, 6, 8, 10, 13, 16};
static_assert(kSplit[kProducers] * 4 == kSeg, "the producers cover a segment");
constexpr int kIv = 4;                  // segments per barrier interval
constexpr int kAhead = kIv + 1;         // producers write segments s0 + kAhead .. s0 + kAhead + kIv - 1
constexpr int kCarryBufs = kIv + kAhead;  // increment ring: the chain's interval and its next segment, the producers'
constexpr int kRing = 3 * kIv;          // segments per f0 block
constexpr int kIncLd = kSeg + 4;        // k-major row stride (floats)

// f0lim = 2^24 / (64 G) for G harmonic groups (2^18 for one): every
// increment (k+1)*f0/sr, k < 64 G, is then computed by the exact
// reciprocal-product form and is finite and >= 0
__device__ __forceinline__ bool fast_f0(float f0, float f0lim) {
  return f0 == 0.0f || (f0 >= 0x1p-20f && f0 < f0lim);
}

__host__ __device__ constexpr int harmonic_groups(int K) { return (K + 63) / 64; }
inline float fast_f0_limit(int K) { return 0x1p24f / (float)(64 * harmonic_groups(K)); }

// In-kernel timer record of one workgroup (TIMED): shader-clock cycles
// (s_memtime) the chain wave and the first producer wave spent from their
// arrival at each interval barrier to its release, summed; the chain's
// first and last cycle and the matching 100 MHz real-time stamps; and the
// interval count.
enum CarryTimer { kTmChainWait, kTmProdWait, kTmCycle0, kTmCycle1, kTmReal0, kTmReal1, kTmIntervals, kTmWords = 8 };

template <int P, class F>
__device__ __forceinline__ void dispatch_producer(int wave, F& body) {
  if constexpr (P < kProducers) {
    if (wave == P + 1)
      body(std::integral_constant<int, kSplit[P]>{}, std::integral_constant<int, kSplit[P + 1] - kSplit[P]>{});
    else
      dispatch_producer<P + 1>(wave, body);
  }
}

// Grid (B, harmonic groups): workgroup (b, g) runs harmonics 64 g .. 64 g + 63.
template <bool TIMED>
__global__ __launch_bounds__(64 * kCarryWaves) void k_phasor_carry(const float* __restrict__ f0f,
                                                                   float* __restrict__ ckpt, int B, int K, int T,
                                                                   float sr, float rsr, float f0lim,
                                                                   unsigned long long* __restrict__ timer) {
  __shared__ __align__(16) float s_inc[kCarryBufs][64 * kIncLd];  // [k][frame]
  __shared__ __align__(16) float s_f0[2][kRing * kSeg];
  __shared__ __align__(16) int s_blkbad[2][8];  // producer p's part of an f0 block holds a value outside the fast range
  __shared__ int s_vote[2];                      // the block's parts combined (producer wave 1, an interval after the commit)
  const int b = blockIdx.x, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int k0 = 64 * (int)blockIdx.y;  // first harmonic of the group
  const int nseg = (T + kSeg - 1) / kSeg;
  const int nblk = (nseg + kRing - 1) / kRing;
  const float* f0b = f0f + (size_t)b * T;
  const int ptid = threadIdx.x - 64;  // producer thread index
  // An f0 block is loaded in two parts: issue (every load of the thread in
  // flight at once, from in-bounds clamped addresses) and commit (registers
  // -> LDS, and the fast-range vote), so that its latency overlaps the
  // produce work of an interval.
  constexpr int kBlkLoads = (kRing * kSeg + 64 * kProducers - 1) / (64 * kProducers);
  float blk_v[kBlkLoads];
  auto issue_block = [&](int blk) {
    const int t0 = blk * kRing * kSeg;
#pragma unroll
    for (int j = 0; j < kBlkLoads; ++j) {
      const int i = min(ptid + j * 64 * kProducers, kRing * kSeg - 1);
      blk_v[j] = f0b[min(t0 + i, T - 1)];
    }
  };
  auto commit_block = [&](int blk) {
    float* dst = s_f0[blk & 1];
    const int t0 = blk * kRing * kSeg;
    int bad = 0;
#pragma unroll
    for (int j = 0; j < kBlkLoads; ++j) {
      const int i = ptid + j * 64 * kProducers;
      if (i < kRing * kSeg) {
        const float v = t0 + i < T ? blk_v[j] : 0.0f;
        bad |= !fast_f0(v, f0lim);
        dst[i] = v;
      }
    }
    bad = __any(bad);
    if (lane == 0) s_blkbad[blk & 1][wave - 1] = bad;
  };
  auto load_block = [&](int blk) {
    issue_block(blk);
    commit_block(blk);
  };
  auto inc_fast = [&](float x) {
    const float q0 = x * rsr;
    return fmaf(fmaf(-q0, sr, x), rsr, q0);
  };
  // one producer's float4 frame groups [G0, G0 + NG) of segment s
  auto produce = [&](int s, auto g0c, auto ngc) __attribute__((always_inline)) {
    constexpr int G0 = decltype(g0c)::value, NG = decltype(ngc)::value;
    const int par = (s / kRing) & 1;
    const float4* f4 = reinterpret_cast<const float4*>(&s_f0[par][(s % kRing) * kSeg]) + G0;
    const bool fast = s_vote[par] == 0;
    const float kf = (float)(k0 + lane + 1);
    float4* dst = reinterpret_cast<float4*>(&s_inc[s % kCarryBufs][lane * kIncLd]) + G0;
    if (fast) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const float4 f = f4[g];
        dst[g] = make_float4(inc_fast(kf * f.x), inc_fast(kf * f.y), inc_fast(kf * f.z), inc_fast(kf * f.w));
      }
    } else {
      for (int g = 0; g < NG; ++g) {
        const float4 f = f4[g];
        dst[g] = make_float4(div_sr(kf * f.x, sr, rsr), div_sr(kf * f.y, sr, rsr), div_sr(kf * f.z, sr, rsr),
                             div_sr(kf * f.w, sr, rsr));
      }
    }
  };
  // the kIv segments next .. next + kIv - 1 (all before the end): every
  // LDS read first (the interval's f0 values and block votes), then the
  // increments, so the producer pays one LDS round trip per interval
  auto produce_interval = [&](int next, auto g0c, auto ngc) __attribute__((always_inline)) {
    constexpr int G0 = decltype(g0c)::value, NG = decltype(ngc)::value;
    float4 f[kIv][NG > 0 ? NG : 1];
    int anybad = 0;
#pragma unroll
    for (int q = 0; q < kIv; ++q) {
      const int sq = next + q, par = (sq / kRing) & 1;
      const float4* f4 = reinterpret_cast<const float4*>(&s_f0[par][(sq % kRing) * kSeg]) + G0;
#pragma unroll
      for (int g = 0; g < NG; ++g) f[q][g] = f4[g];
      anybad |= s_vote[par];
    }
    const float kf = (float)(k0 + lane + 1);
    if (__builtin_expect(!anybad, 1)) {
#pragma unroll
      for (int q = 0; q < kIv; ++q) {
        float4* dst = reinterpret_cast<float4*>(&s_inc[(next + q) % kCarryBufs][lane * kIncLd]) + G0;
#pragma unroll
        for (int g = 0; g < NG; ++g)
          dst[g] = make_float4(inc_fast(kf * f[q][g].x), inc_fast(kf * f[q][g].y), inc_fast(kf * f[q][g].z),
                               inc_fast(kf * f[q][g].w));
      }
    } else {
      for (int q = 0; q < kIv; ++q) produce(next + q, g0c, ngc);
    }
  };
  // chain: v[32h .. 32h+31] <- half h of segment s's increments
  auto fetch_half = [&](int s, float* v, int h) {
    const float4* src = reinterpret_cast<const float4*>(&s_inc[s % kCarryBufs][lane * kIncLd]) + 8 * h;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 u = src[q];
      v[32 * h + 4 * q] = u.x;
      v[32 * h + 4 * q + 1] = u.y;
      v[32 * h + 4 * q + 2] = u.z;
      v[32 * h + 4 * q + 3] = u.w;
    }
  };
  float ph = 0.0f;  // the phasor state cell is zero at the start of every run
  // steps segment s from v; if nv, loads segment s+1 into nv half by half in
  // between so at most ~8 LDS reads are in flight
  // Checkpoints: the chain writes the phase entering segment s into the
  // padding word of its lane's row of the segment's ring slot (word kSeg,
  // which no producer writes and no increment read covers; an LDS write
  // costs the chain less than a store to memory), and producer wave 1
  // copies an interval's checkpoints to memory during the next interval
  // (the slot's padding is next written by the chain for segment s + 9,
  // two intervals later).  The copies go through a buffer resource bounded
  // to this batch lane's rows: lanes >= K get an offset past the bound and
  // the hardware drops their store, so the store needs no branch around it.
  static_assert(kIncLd > kSeg && kCarryBufs > 2 * kIv, "a free word per row, not rewritten for two intervals");
  const auto ck_rsrc = __builtin_amdgcn_make_buffer_rsrc(ckpt + (size_t)b * K + k0, 0,
                                                         (int)(4u * (unsigned)((nseg - 1) * B * K + K - k0)),
                                                         0x00020000);
  const unsigned ck_voff = k0 + lane < K ? 4u * (unsigned)lane : 0x80000000u;
  const int ck_stride = 4 * B * K;  // bytes per segment of checkpoints
  auto keep_ckpt = [&](int slot) { s_inc[slot][lane * kIncLd + kSeg] = ph; };
  auto copy_ckpts = [&](int iv) {  // producer wave 1: interval iv's checkpoints to memory
    for (int q = 0; q < kIv; ++q) {
      const int s = iv * kIv + q;
      if (s < nseg)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, s_inc[s % kCarryBufs][lane * kIncLd + kSeg]),
                                              ck_rsrc, ck_voff, s * ck_stride, 0);
    }
  };
  auto step_seg = [&](int s, const float* v, int slow, float* nv, auto has_next) {
    constexpr bool kNext = decltype(has_next)::value;
    keep_ckpt(s % kCarryBufs);
    if (!slow) {
      if constexpr (kNext) fetch_half(s + 1, nv, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < kSeg / 2; ++i) ph = __builtin_amdgcn_fractf(ph + v[i]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kNext) fetch_half(s + 1, nv, 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = kSeg / 2; i < kSeg; ++i) ph = __builtin_amdgcn_fractf(ph + v[i]);
    } else {
      if constexpr (kNext) {
        fetch_half(s + 1, nv, 0);
        fetch_half(s + 1, nv, 1);
      }
      const float* inc = &s_inc[s % kCarryBufs][lane * kIncLd];
      const int nt = min(kSeg, T - s * kSeg);
      for (int i = 0; i < nt; ++i) ph = phasor_wrap(ph + inc[i]);
    }
  };

  const int nint = (nseg + kIv - 1) / kIv;
  if (threadIdx.x < 16) s_blkbad[0][threadIdx.x] = 0;
  lds_barrier();
  if (wave > 0) {
    load_block(0);
    load_block(1);
  }
  lds_barrier();
  // block m's vote: the OR of its producers' parts
  auto combine_votes = [&](int m) {
    int v = 0;
#pragma unroll
    for (int w = 0; w < kProducers; ++w) v |= s_blkbad[m & 1][w];
    s_vote[m & 1] = v;
  };
  if (wave == 1 && lane == 0) {
    combine_votes(0);
    combine_votes(1);
  }
  lds_barrier();
  // producer p's frame groups, as constants of its code
  auto as_producer = [&](auto body) __attribute__((always_inline)) { dispatch_producer<0>(wave, body); };

  if (wave > 0)
    as_producer([&](auto g0c, auto ngc) __attribute__((always_inline)) {
      for (int s = 0; s < kAhead && s < nseg; ++s) produce(s, g0c, ngc);
    });
  lds_barrier();
  // (TIMED: each barrier's stamps are summed at the next barrier, where
  // its wait has returned them, so the chain never waits for a stamp)
  unsigned long long tm_wait = 0, tm_b = 0, tm_a = 0, tm_c0 = 0, tm_r0 = 0;
  if constexpr (TIMED) {
    tm_c0 = __builtin_amdgcn_s_memtime();
    tm_r0 = __builtin_amdgcn_s_memrealtime();
  }
  auto interval_barrier = [&]() {
    if constexpr (TIMED) {
      const unsigned long long t = __builtin_amdgcn_s_memtime();
      lds_barrier();
      tm_wait += tm_a - tm_b;
      tm_b = t;
      tm_a = __builtin_amdgcn_s_memtime();
    } else {
      lds_barrier();
    }
  };
  // The chain and the producers run loops of their own with the same
  // barriers (in one loop the compiler reconciles the two roles' registers
  // with copies on the chain's path at every interval).
  if (wave == 0) {
    __builtin_amdgcn_s_setprio(3);
    // The fast-step vote of the f0 block an interval lies in (an interval
    // never spans two blocks): committed by the producers at least four
    // intervals before the chain reads it, and overwritten (by block + 2)
    // only after the chain has passed that block's last interval.
    static_assert(kRing % kIv == 0, "an interval lies in one f0 block");
    auto block_vote = [&](int s0) { return s_vote[(s0 / kRing) & 1]; };
    int nbad = block_vote(0);  // the next interval's vote, read an interval ahead
    // va holds the interval's first segment on entry (read before the
    // barrier that ends the previous interval)
    float va[kSeg], vb[kSeg];
    fetch_half(0, va, 0);
    fetch_half(0, va, 1);
    int iv = 0;
    while (iv < nint) {
      // Intervals whose segments are all full-length in the fast form, in
      // a loop of their own: the steps, the next interval's vote and the
      // barrier, without a branch over the general form or a per-lane flag
      // vote (each cost the chain hundreds of cycles an interval).
      for (;;) {
        const int s0 = iv * kIv;
        if (__builtin_amdgcn_readfirstlane(nbad) != 0 || (s0 + kIv) * kSeg > T) break;
        // Four rotating half-segment buffers A, B, C, D: each half steps
        // while the half two ahead loads into the buffer the half before
        // freed, ending with the next interval's first segment in A, B
        // (the empty asm statements keep every load at its place).  Past
        // the last interval that read lands in the ring, in bounds, unused.
        static_assert(kIv == 4, "the run below covers four segments");
        float* A = va;
        float* B = va + kSeg / 2;
        float* C = vb;
        float* D = vb + kSeg / 2;
        // (ring slots from the interval's base, so the chain wave issues a
        // few scalar adds per segment instead of a modulo)
        const int b0 = s0 % kCarryBufs;
        auto ld = [&](int k, int h, float* d) {
          asm volatile("" ::: "memory");
          const int bk = b0 + k >= kCarryBufs ? b0 + k - kCarryBufs : b0 + k;
          const float4* src = reinterpret_cast<const float4*>(&s_inc[bk][lane * kIncLd]) + 8 * h;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const float4 u = src[q];
            d[4 * q] = u.x;
            d[4 * q + 1] = u.y;
            d[4 * q + 2] = u.z;
            d[4 * q + 3] = u.w;
          }
          asm volatile("" ::: "memory");
        };
        auto st = [&](const float* v) {
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < kSeg / 2; ++i) ph = __builtin_amdgcn_fractf(ph + v[i]);
          __builtin_amdgcn_sched_barrier(0);
        };
        auto ck = [&](int k) { keep_ckpt(b0 + k >= kCarryBufs ? b0 + k - kCarryBufs : b0 + k); };
        ck(0);
        ld(1, 0, C); st(A); ld(1, 1, D); st(B);
        ck(1);
        // (read here, combined after the run: its wait then costs nothing)
        const int vote = block_vote(s0 + kIv);
        ld(2, 0, A); st(C); ld(2, 1, B); st(D);
        ck(2);
        ld(3, 0, C); st(A); ld(3, 1, D); st(B);
        ck(3);
        ld(kIv, 0, A); st(C); ld(kIv, 1, B); st(D);
        nbad = vote;
        interval_barrier();
        if (++iv >= nint) break;
      }
      if (iv >= nint) break;
      {
        // one interval in the general form: a segment of a block with an
        // f0 outside the fast range, past the end or shorter than kSeg
        // takes the literal wrap form
        const int s0 = iv * kIv;
        const int bad = __builtin_amdgcn_readfirstlane(nbad);
        int fl[kIv];
#pragma unroll
        for (int q = 0; q < kIv; ++q) fl[q] = bad != 0 || (T - (s0 + q) * kSeg) < kSeg;
        int fa = fl[0], fb = 0;
#pragma unroll
        for (int q = 0; q < kIv; ++q) {
          const int s = s0 + q;
          if (s >= nseg) break;
          // the next segment's increments are loaded while this one steps
          const bool more = q + 1 < kIv && s + 1 < nseg;
          if (q % 2 == 0) {
            if (more) {
              fb = fl[q + 1];
              step_seg(s, va, fa, vb, std::true_type{});
            } else {
              step_seg(s, va, fa, vb, std::false_type{});
            }
          } else {
            if (more) {
              fa = fl[q + 1];
              step_seg(s, vb, fb, va, std::true_type{});
            } else {
              step_seg(s, vb, fb, va, std::false_type{});
            }
          }
        }
        nbad = block_vote(s0 + kIv);
        fetch_half(s0 + kIv, va, 0);
        fetch_half(s0 + kIv, va, 1);
        interval_barrier();
        ++iv;
      }
    }
  } else {
    // Interval iv produces segments 4 iv + 5 .. 4 iv + 8, so f0 block j
    // (segments 12 j .. 12 j + 11) is read in intervals 3 j - 2 .. 3 j + 1.
    // Block m replaces block m - 2 in its buffer: its loads are issued in
    // interval 3 m - 5 and committed in 3 m - 4, after block m - 2's last
    // reader and three intervals before block m's first (blocks 0 and 1
    // are loaded before the loop).  Producer wave 1 combines block m's
    // votes in interval 3 m - 3; the producers read the vote from 3 m - 2
    // and the chain from 3 m - 1, both until 3 m + 1, before block m + 2's
    // combine (3 m + 3) overwrites it.
    static_assert(kAhead == 5 && kRing == 12 && kIv == 4, "the block schedule below");
    as_producer([&](auto g0c, auto ngc) __attribute__((always_inline)) {
      for (int iv = 0; iv < nint; ++iv) {
        const int next = iv * kIv + kAhead;
        if ((iv + 5) % 3 == 0 && (iv + 5) / 3 < nblk) issue_block((iv + 5) / 3);
        if (__builtin_expect(next + kIv <= nseg, 1)) {
          produce_interval(next, g0c, ngc);
        } else {
          for (int s = next; s < nseg; ++s) produce(s, g0c, ngc);
        }
        if ((iv + 4) % 3 == 0 && (iv + 4) / 3 < nblk) commit_block((iv + 4) / 3);
        if (wave == 1 && lane == 0 && iv % 3 == 0 && iv / 3 + 1 < nblk && iv > 0) combine_votes(iv / 3 + 1);
        if (wave == 1 && iv > 0) copy_ckpts(iv - 1);
        interval_barrier();
      }
      if (wave == 1) copy_ckpts(nint - 1);
    });
  }
  if constexpr (TIMED) {
    tm_wait += tm_a - tm_b;
    const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    unsigned long long* rec = timer + ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * kTmWords;
    if (wave == 0 && lane == 0) {
      rec[kTmChainWait] = tm_wait;
      rec[kTmCycle0] = tm_c0;
      rec[kTmCycle1] = c1;
      rec[kTmReal0] = tm_r0;
      rec[kTmReal1] = r1;
      rec[kTmIntervals] = (unsigned long long)nint;
      rec[kTmIntervals + 1] = 0;
    }
    if (wave == 1 && lane == 0) rec[kTmProdWait] = tm_wait;
  }
}

int launch_phasor_carry(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=f0f ([B][T]) [1]=checkpoints ([nseg][B][K]) [2]=B [3]=K [4]=T
  //      [5]=timer cell ([G][B][8] uint64, read only if [6] == 1) [6]=timed   farg: [0]=sr
  const int64_t f0f = op.arg[0], ck = op.arg[1], B = op.arg[2], K = op.arg[3], T = op.arg[4];
  const bool timed = op.arg[6] == 1;
  DGEN_REQUIRE(B > 0 && B <= 65535 && K > 0 && K <= kMaxKWide && T > 0 && T <= (1 << 26),
               "phasor_carry: B %lld K %lld T %lld", (long long)B, (long long)K, (long long)T);
  DGEN_REQUIRE(op.farg[0] > 0.f && op.farg[0] < 1e30f, "phasor_carry: sample rate %g", (double)op.farg[0]);
  const int64_t nseg = (T + kSeg - 1) / kSeg;
  DGEN_CHECK_CELL(L, f0f, B * T, "phasor_carry.f0_frames");
  DGEN_CHECK_CELL(L, ck, nseg * B * K, "phasor_carry.checkpoints");
  DGEN_REQUIRE(nseg * B * K < (1ll << 29), "phasor_carry: %lld checkpoints (< 2^29)", (long long)(nseg * B * K));
  DGEN_REQUIRE(op.arg[6] == 0 || op.arg[6] == 1, "phasor_carry: timed flag %lld", (long long)op.arg[6]);
  const int64_t G = harmonic_groups((int)K);
  if (timed) DGEN_CHECK_CELL(L, op.arg[5], 2 * kTmWords * G * B, "phasor_carry.timer");
  if (L.dry) return 0;
  const float sr = host_rate(L, op.farg[0]), rsr = 1.0f / sr;
  const dim3 grid((unsigned)B, (unsigned)G);
  if (timed)
    hipLaunchKernelGGL(k_phasor_carry<true>, grid, dim3(64 * kCarryWaves), 0, L.stream, cell(L, f0f), cell(L, ck),
                       (int)B, (int)K, (int)T, sr, rsr, fast_f0_limit((int)K),
                       reinterpret_cast<unsigned long long*>(cell(L, op.arg[5])));
  else
    hipLaunchKernelGGL(k_phasor_carry<false>, grid, dim3(64 * kCarryWaves), 0, L.stream, cell(L, f0f), cell(L, ck),
                       (int)B, (int)K, (int)T, sr, rsr, fast_f0_limit((int)K), nullptr);
  DGEN_LAUNCH_CHECK("k_phasor_carry");
  return 0;
}

// ------------------------------------------------------------ shared pieces
struct SynthArgs {
  const float* ctrl;
  const float* f0f;
  const float* uvf;
  const float* lerp;
  const float* seg_rows;
  const float* noise;
  const float* ckpt;
  int ldc, B, K, NF, F, T;
  float sr, rsr, hscale, nscale;
  float nyq;  // half the graph's sample rate: the Nyquist mask (Synth.swift:158-167)
  float f0lim;  // fast-step bound of f0 (fast_f0)
};

// Per-frame values of a segment, staged in LDS and read as broadcasts.
struct FrameRec {
  float f0, frac, omf;
  int slots;  // slot(lo) | slot(hi) << 8
};

// Per-wave LDS of the synth kernels, for up to MAXK harmonics and MAXNC
// control columns (the narrow layout SegLds, or the wide one).
template <int MAXK, int MAXNC, bool PRE = true>
struct SegLdsT {
  static constexpr int kMaxK = MAXK, kMaxNC = MAXNC, kGroups = MAXK / 64;
  FrameRec fr[kSeg];
  // per-frame weights of the four row slots: a frame's control value is
  // sum_j wt[i][j] * row[j][c] = (1-frac) row[lo][c] + frac row[hi][c]
  float4 wt[kSeg];
  // control rows touched by the segment; the stride (4 mod 64 words) puts
  // one column of the four slots in different banks, as the FIR's lanes
  // (frames) read rows lo and hi of their own frames
  float row[kSlots][MAXNC + 4];
  float pre[kSlots][PRE ? MAXK + 1 : 1];  // prefix sums of the harmonic columns of each row (forward)
  float noise[kSeg + MAXNC];      // noise[t0 - (NF-1) ... t0 + 63]
  // per-frame scalars of the backward: (f0, hs, coef, dfl) as one 16-byte
  // record (the harmonic pass reads all four per frame), and dg, dng
  float4 pk[kSeg];
  float dg[kSeg];
  float dng[kSeg];
};
using SegLds = SegLdsT<kMaxK, kMaxNC>;
using SegLdsWide = SegLdsT<kMaxKWide, kMaxNCWide>;
// the backward's layouts (no prefix sums)
using SegLdsBwd = SegLdsT<kMaxK, kMaxNC, false>;
using SegLdsBwdWide = SegLdsT<kMaxKWide, kMaxNCWide, false>;

// Stage the segment's frame records and slot weights, rows, their harmonic
// prefix sums (if want_pre) and the noise window; nslot_out = the number of
// row slots in use, pairs_out = every frame reads two distinct rows.
// Returns 1 if every frame's f0 admits the fast chain step.
template <class SL>
__device__ __forceinline__ int stage_segment(const SynthArgs& a, SL& L, int s, int b, int lane, int nt,
                                             bool want_pre, int& nslot_out, bool& pairs_out) {
  const int t0 = s * kSeg;
  const int NC = a.K + 2 + a.NF;
  int ok = 1;
  {
    FrameRec r{0.f, 0.f, 1.f, 0};
    if (lane < nt) {
      const int t = t0 + lane;
      const float4 e0 = *reinterpret_cast<const float4*>(a.lerp + (size_t)t * 8);
      const float4 e1 = *reinterpret_cast<const float4*>(a.lerp + (size_t)t * 8 + 4);
      r.f0 = a.f0f[(size_t)b * a.T + t];
      r.frac = e0.z;
      r.omf = e0.w;
      r.slots = (int)e1.x | ((int)e1.y << 8);
      ok = fast_f0(r.f0, a.f0lim) ? 1 : 0;
    }
    L.fr[lane] = r;
    const int slo = r.slots & 255, shi = r.slots >> 8;
    float w[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) w[j] = (slo == j ? r.omf : 0.0f) + (shi == j ? r.frac : 0.0f);
    L.wt[lane] = make_float4(w[0], w[1], w[2], w[3]);
    pairs_out = __all(lane >= nt || slo != shi);
  }
  int nslot = 0;
  for (int j = 0; j < kSlots; ++j) {
    const float r = a.seg_rows[(size_t)s * kSlots + j];
    if (r < 0.0f) break;
    const float* src = a.ctrl + ((size_t)b * a.F + (int)r) * a.ldc;
    for (int c = lane; c < NC; c += 64) L.row[j][c] = src[c];
    ++nslot;
  }
  nslot_out = nslot;
  for (int i = lane; i < a.NF - 1 + kSeg; i += 64) {
    const int tt = t0 - (a.NF - 1) + i;
    L.noise[i] = (tt >= 0 && tt < a.T) ? a.noise[tt] : 0.0f;
  }
  wave_sync();
  if (want_pre) {
    // inclusive wave scan of each row's first K columns -> pre[j][k+1], a
    // group of 64 harmonics at a time, each group's scan added to the sum
    // of the groups before it
    for (int j = 0; j < nslot; ++j) {
      float carry = 0.0f;
      for (int g = 0; g < SL::kGroups; ++g) {
        const int k = 64 * g + lane;
        if (64 * g >= a.K) break;
        float v = k < a.K ? L.row[j][k] : 0.0f;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const float u = __shfl_up(v, d, 64);
          if (lane >= d) v += u;
        }
        if (g > 0) v = carry + v;
        if (k < a.K) L.pre[j][k + 1] = v;
        carry = __shfl(v, 63, 64);
      }
      if (lane == 0) L.pre[j][0] = 0.0f;
    }
    wave_sync();
  }
  return __all(ok) && nt == kSeg;
}

// Number of harmonics k < K with (k+1)*f0 < nyq (a prefix of k, since
// (k+1)*f0 is monotone in k).
__device__ __forceinline__ int below_nyquist(float f0, float nyq, int K) {
  int lo = 0, hi = K;  // answer in [lo, hi]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((float)mid * f0 < nyq) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// The phase chain runs in blocks of kBlk steps whose LDS reads (frame
// records, row values) are all issued before the block's arithmetic.
constexpr int kBlk = 8;

// FIR noise branch for frame i: sum_j noise[t-(NF-1)+j] * tap_j(t).
template <class SL>
__device__ __forceinline__ float frame_fir(const SynthArgs& a, const SL& L, int i, const FrameRec& r) {
  const float* rl = &L.row[r.slots & 255][a.K + 2];
  const float* rh = &L.row[r.slots >> 8][a.K + 2];
  const float* w = &L.noise[i];
  float flo = 0.0f, fhi = 0.0f;
  for (int j = 0; j < a.NF; ++j) {
    flo = fmaf(w[j], rl[j], flo);
    fhi = fmaf(w[j], rh[j], fhi);
  }
  return r.omf * flo + r.frac * fhi;
}

// ------------------------------------------------------------ forward
// Writes y and the per-frame tape aux = [hsum | den | filt] ([3][B][T]) that
// the backward reuses.
constexpr int kWavesFwd = 2;

// Row-slot arithmetic of a frame.  NS = 2, 3 or 4: the slot-weight form over
// the slots that can be nonzero (a weight-0 slot contributes 0 * value, so
// the operands must be finite: the kernels vote for it per segment).
// NS = 0: the exact per-frame form of the reference's sampleRow lerp and its
// gradient, which touches only the frame's rows lo and hi (non-finite
// values stay in the frames and rows that read them).
// A lane's control value of a frame (slot weights w) from its row-slot
// values rv (0 past the slots in use); the exact form reads rows lo and hi.
// Products and sums are rounded one by one (no fma): with finite rows and
// lo != hi the two nonzero terms are (1-frac) row[lo] and frac row[hi] and
// the others add a signed zero, so the value is the exact form's bit for bit.
template <int NS>
__device__ __forceinline__ float slot_lerp(const float4& w, const float (&rv)[kSlots]) {
  static_assert(NS == 2 || NS == 3 || NS == kSlots, "slot-weight form");
  float v = w.x * rv[0] + w.y * rv[1];
  if constexpr (NS > 2) v = v + w.z * rv[2];
  if constexpr (NS > 3) v = v + w.w * rv[3];
  return v;
}

// Adds a frame's gradient x of one control column into the row slots.
template <int NS>
__device__ __forceinline__ void slot_acc(float (&acc)[kSlots], const FrameRec& r, const float4& w, float x) {
  if constexpr (NS == 0) {
    const int slo = r.slots & 255, shi = r.slots >> 8;
    const float vl = r.omf * x, vh = r.frac * x;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      acc[j] += slo == j ? vl : 0.0f;
      acc[j] += shi == j ? vh : 0.0f;
    }
  } else {
    acc[0] = fmaf(w.x, x, acc[0]);
    acc[1] = fmaf(w.y, x, acc[1]);
    if constexpr (NS > 2) acc[2] = fmaf(w.z, x, acc[2]);
    if constexpr (NS > 3) acc[3] = fmaf(w.w, x, acc[3]);
  }
}

// Chain pass of the forward held in registers: v[i] = sin(2 pi phase_k(i)) *
// masked amplitude for frame i of this lane's harmonic k (0 for lanes >= K
// and frames >= nt).  The phase steps are those of the reference's stateful
// phasor (pre-increment output, wrap), the backward's pass repeats them bit
// for bit.  rv = this lane's amplitude column in each row slot; kh = the
// lane's harmonic (lane + 64 g in group g).
// MASKC: no harmonic crosses the Nyquist limit inside the segment and the
// caller has zeroed rv of the lanes masked throughout (and of lanes >= K),
// so no frame tests the mask: those lanes add sin * 0.
// ADD: v[i] += the term (harmonic groups after the first), else v[i] = it.
template <bool FAST, int NS, bool MASKC = false, bool ADD = false, class SL>
__device__ __forceinline__ void chain_regs(const SynthArgs& a, const SL& L, float (&v)[kSeg], int kh, int nt,
                                           float ph, const float (&rv)[kSlots]) {
  static_assert(!MASKC || (FAST && NS != 0), "the constant mask is a fast slot-weight form");
  const float kf = (float)(kh + 1);
  const float nyq = a.nyq;
  const bool harm = kh < a.K;
  const int kk = harm ? kh : 0;
#pragma unroll
  for (int i0 = 0; i0 < kSeg; i0 += kBlk) {
    // the block's reads are issued at its start, not hoisted over the
    // whole segment (which would hold every frame's values in registers)
    asm volatile("" ::: "memory");
    FrameRec r[kBlk];
    float4 w[kBlk];
    float al[kBlk], ah[kBlk];  // exact form: the lane's values in rows lo and hi
#pragma unroll
    for (int j = 0; j < kBlk; ++j) {
      if constexpr (NS == 0) {
        r[j] = L.fr[i0 + j];
        al[j] = L.row[r[j].slots & 255][kk];
        ah[j] = L.row[r[j].slots >> 8][kk];
      } else if constexpr (NS == 3) {
        // three slots: the record's fourth word holds the frame's f0
        w[j] = L.wt[i0 + j];
        r[j].f0 = w[j].w;
      } else {
        r[j].f0 = L.fr[i0 + j].f0;
        w[j] = L.wt[i0 + j];
      }
    }
#pragma unroll
    for (int j = 0; j < kBlk; ++j) {
      const int i = i0 + j;
      if (!FAST && i >= nt) {
        if constexpr (!ADD) v[i] = 0.0f;
        continue;
      }
      const float freq = kf * r[j].f0;
      float inc;
      if (FAST) {
        const float q0 = freq * a.rsr;
        inc = fmaf(fmaf(-q0, a.sr, freq), a.rsr, q0);
      } else {
        inc = div_sr(freq, a.sr, a.rsr);
      }
      const float p = ph;
      ph = FAST ? __builtin_amdgcn_fractf(ph + inc) : phasor_wrap(ph + inc);
      float amp;
      if constexpr (NS == 0)
        amp = r[j].omf * al[j] + r[j].frac * ah[j];
      else
        amp = slot_lerp<NS>(w[j], rv);
      const float term = MASKC ? sin2pi(p) * amp : ((harm && freq < nyq) ? sin2pi(p) * amp : 0.0f);
      if constexpr (ADD)
        v[i] = v[i] + term;
      else
        v[i] = term;
    }
  }
}

// Butterfly reduce-scatter across the wave: on entry v[i] is this lane's
// term of frame i; on return v[0] is the sum over all 64 lanes of frame
// `lane`'s terms.  Stage D keeps the half of the frames selected by bit D of
// the lane and adds a partner's copy of that half, the partner being a lane
// with the other bit D that holds the same frames: lane ^ 32 and lane ^ 16
// by v_permlane32_swap / v_permlane16_swap (x's upper lanes trade places
// with y's lower lanes, so x + y is each lane's kept half plus its
// partner's, no selects), then the row mirror (lane ^ 15 in a row of 16),
// the half-row mirror (^ 7) and two quad permutations (^ 2, ^ 1) by DPP.
// The swaps need two wait states after a VALU write of their operands.
#define DGEN_SWAP4(OP, D, j)                                                                                        \
  asm("s_nop 1\n\t" OP " %0, %1\n\t" OP " %2, %3\n\t" OP " %4, %5\n\t" OP " %6, %7"                             \
      : "+v"(v[j]), "+v"(v[j + D]), "+v"(v[j + 1]), "+v"(v[j + 1 + D]), "+v"(v[j + 2]), "+v"(v[j + 2 + D]),         \
        "+v"(v[j + 3]), "+v"(v[j + 3 + D]))

template <int D>
__device__ __forceinline__ void rs_swap_stage(float (&v)[kSeg]) {
  static_assert(D == 32 || D == 16, "lane-swap stages");
#pragma unroll
  for (int j = 0; j < D; j += 4) {
    if constexpr (D == 32)
      DGEN_SWAP4("v_permlane32_swap_b32", 32, j);
    else
      DGEN_SWAP4("v_permlane16_swap_b32", 16, j);
  }
#pragma unroll
  for (int j = 0; j < D; ++j) v[j] = v[j] + v[j + D];
}
#undef DGEN_SWAP4

template <int D, int CTRL>
__device__ __forceinline__ void rs_dpp_stage(float (&v)[kSeg], int lane) {
  const bool up = (lane & D) != 0;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const float send = up ? v[j] : v[j + D];
    const float keep = up ? v[j + D] : v[j];
    const float got = __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), CTRL, 0xf, 0xf, false));
    v[j] = keep + got;
  }
}

__device__ __forceinline__ float reduce_scatter64(float (&v)[kSeg], int lane) {
  static_assert(kSeg == 64, "one frame per lane");
  rs_swap_stage<32>(v);
  rs_swap_stage<16>(v);
  rs_dpp_stage<8, 0x140>(v, lane);  // row_mirror
  rs_dpp_stage<4, 0x141>(v, lane);  // row_half_mirror
  rs_dpp_stage<2, 0x4e>(v, lane);   // quad_perm [2,3,0,1]
  rs_dpp_stage<1, 0xb1>(v, lane);   // quad_perm [1,0,3,2]
  return v[0];
}

// The chain pass of harmonic kh = lane + 64 g of one group into v (ADD: v +=).
// ns: the row-slot form; [flo, fhi]: the segment's f0 range (fast slot forms).
template <bool ADD, class SL>
__device__ __forceinline__ void fwd_group(const SynthArgs& a, const SL& L, float (&v)[kSeg], int kh, int s, int b,
                                          int nt, int fast, int ns, int nslot, float flo, float fhi) {
  const int kk = kh < a.K ? kh : 0;
  const float ph = a.ckpt[((size_t)s * a.B + b) * a.K + kk];
  float rv[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; ++j) rv[j] = j < nslot ? L.row[j][kk] : 0.0f;
  // Nyquist mask of harmonic k over the segment, from the frames' extreme
  // f0 (RN((k+1) f0) is monotone in f0): on in every frame, off in every
  // frame, or mixed (the per-frame test)
  bool mixed = false, zero = kh >= a.K;
  if (fast && ns != 0) {
    const float kf = (float)(kh + 1);
    const bool on = kf * fhi < a.nyq, off = !(kf * flo < a.nyq);
    mixed = kh < a.K && !on && !off;
    zero = zero || off;
  }
  if (fast && ns != 0 && !__any(mixed)) {
    // finite rows (ns != 0): a zeroed lane adds sin * 0 = +-0, which leaves
    // every frame's sum as the per-frame form's
    float rz[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) rz[j] = zero ? 0.0f : rv[j];
    if (ns == 2)
      chain_regs<true, 2, true, ADD>(a, L, v, kh, nt, ph, rz);
    else if (ns == 3)
      chain_regs<true, 3, true, ADD>(a, L, v, kh, nt, ph, rz);
    else
      chain_regs<true, kSlots, true, ADD>(a, L, v, kh, nt, ph, rz);
  } else if (fast && ns == 2)
    chain_regs<true, 2, false, ADD>(a, L, v, kh, nt, ph, rv);
  else if (fast && ns == 3)
    chain_regs<true, 3, false, ADD>(a, L, v, kh, nt, ph, rv);
  else if (fast && ns == kSlots)
    chain_regs<true, kSlots, false, ADD>(a, L, v, kh, nt, ph, rv);
  else if (fast)
    chain_regs<true, 0, false, ADD>(a, L, v, kh, nt, ph, rv);
  else
    chain_regs<false, 0, false, ADD>(a, L, v, kh, nt, ph, rv);
}

template <class SL>
__global__ __launch_bounds__(64 * kWavesFwd) void k_synth_fwd(SynthArgs a, float* __restrict__ y,
                                                              float* __restrict__ aux) {
  __shared__ SL lds[kWavesFwd];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int nseg = (a.T + kSeg - 1) / kSeg;
  const int s = blockIdx.x * kWavesFwd + wave, b = blockIdx.y;
  if (s >= nseg) return;
  SL& L = lds[wave];
  const int t0 = s * kSeg, nt = min(kSeg, a.T - t0);
  int nslot;
  bool pairs;
  const int fast = stage_segment(a, L, s, b, lane, nt, true, nslot, pairs);
  float v[kSeg];
  {
    bool fin = true;
    for (int g = 0; g < SL::kGroups; ++g) {
      if (64 * g >= a.K) break;
      const int kh = 64 * g + lane, kk = kh < a.K ? kh : 0;
#pragma unroll
      for (int j = 0; j < kSlots; ++j) fin = fin && isfinite(j < nslot ? L.row[j][kk] : 0.0f);
    }
    // slot weights need finite rows and two distinct rows per frame; else
    // the exact per-frame form.  With three slots (nearly every segment when
    // control rows are about a segment apart) the weight record's unused
    // fourth word takes the frame's f0, so a frame's chain step reads one
    // 16-byte record and forms its amplitude from three slots.
    const int ns = !(__all(fin) && pairs) ? 0 : (nslot <= 2 ? 2 : (nslot == 3 ? 3 : kSlots));
    if (ns == 3) {
      L.wt[lane].w = L.fr[lane].f0;
      wave_sync();
    }
    float flo = 0.0f, fhi = 0.0f;
    if (fast && ns != 0) {
      flo = fhi = L.fr[lane].f0;
#pragma unroll
      for (int d = 32; d > 0; d >>= 1) {
        flo = fminf(flo, __shfl_xor(flo, d, 64));
        fhi = fmaxf(fhi, __shfl_xor(fhi, d, 64));
      }
    }
    fwd_group<false>(a, L, v, lane, s, b, nt, fast, ns, nslot, flo, fhi);
    for (int g = 1; g < SL::kGroups; ++g) {
      if (64 * g >= a.K) break;
      fwd_group<true>(a, L, v, 64 * g + lane, s, b, nt, fast, ns, nslot, flo, fhi);
    }
  }
  const float num = reduce_scatter64(v, lane);  // frame = lane
  if (lane < nt) {
    const int t = t0 + lane;
    const FrameRec r = L.fr[lane];
    const int slo = r.slots & 255, shi = r.slots >> 8;
    const int n = below_nyquist(r.f0, a.nyq, a.K);
    const float den = r.omf * L.pre[slo][n] + r.frac * L.pre[shi][n] + 1e-8f;
    const float hsum = num / den;
    const float gain = r.omf * L.row[slo][a.K] + r.frac * L.row[shi][a.K];
    const float ngain = r.omf * L.row[slo][a.K + 1] + r.frac * L.row[shi][a.K + 1];
    const float filt = frame_fir(a, L, lane, r);
    const float uv = a.uvf[(size_t)b * a.T + t];
    const float hout = ((hsum * gain) * uv) * a.hscale;
    const float nout = ((filt * ngain) * 0.12f) * a.nscale;
    const float o = hout + nout;
    const size_t bt = (size_t)b * a.T + t, plane = (size_t)a.B * a.T;
    y[bt] = isfinite(o) ? o : 0.0f;  // dgen_runtime.h:58-85 containment
    if (aux) {
      aux[bt] = hsum;
      aux[plane + bt] = den;
      aux[2 * plane + bt] = filt;
    }
  }
}

// ------------------------------------------------------------ backward
// Per (segment, batch) wave: recompute the phases, then accumulate every
// control column's gradient into <= 4 row slots:
//   d amp_k = dhsum * (sin_k - hsum) / den * mask_k       (normalised amps)
//   d gain  = g * hsum * uv * hscale,  d ngain = g * filt * 0.12 * nscale
//   d tap_j = g * ngain * 0.12 * nscale * noise[t-(NF-1)+j]
// each scattered to rows lo/hi with weights 1-frac / frac
// (sampleInline gradient, Emit+RowSelection.swift:100-141).
//
// A workgroup owns a run of kRunSegs consecutive segments of one lane (a
// wave each).  Each wave leaves its four row-slot sums per column in its own
// LDS (over the staged rows, which the passes no longer read); then the
// workgroup sums, for every control row its segments touch, the run's
// entries of that row in the row list's (segment) order.  A row whose
// entries all lie in the run is final and goes to d ctrl; a row shared
// with other runs (at most two per run boundary, and row 0 when the
// playhead wraps in the last frame) goes to its boundary partial
// [B][F][kRunParts][ldc] at the index of the run among the row's runs, and
// DGEN_HIP_K_SYNTH_BWD_REDUCE adds those partials in run order.  A row's
// at most 16 entries come from consecutive segments plus the wrap, so it
// meets at most 6 runs of 4.  Four segments a run: five workgroups (20
// waves, the registers' limit) per CU, one wave per SIMD each; larger
// runs left some SIMDs a wave short (8: 16 waves per CU, 193 against
// 155 us; 10: 273 us).
constexpr int kRunSegs = 4;
constexpr int kRunParts = 6;

// Column passes of the backward, each accumulating its column's gradient
// into the four row slots with the frames' slot weights.  The harmonic
// passes (one per group of 64 harmonics) run the phase chain (harmonic
// kh = lane + 64 g, the forward's chain bit for bit) and accumulate harmonic
// column kh in the same loop, so no per-frame sine table is staged; in the
// last group the lanes past K take the last non-harmonic columns
// (K + 64 P + kh - K).  The P gain passes take columns K + 64 p + lane
// (gain, noise gain, taps), P the fewest that cover the rest; with one
// group and NC <= 128, P = 1 and the spare lanes' columns are lane + 64.
// MASKC: no harmonic crosses the Nyquist limit inside the segment, so each
// lane's mask is one value for all its frames (the caller zeroes the sums
// of lanes that are masked throughout) and no frame tests it.
template <bool FAST, int NS, bool MASKC = false, class SL>
__device__ __forceinline__ void bwd_harmonic_pass(const SynthArgs& a, const SL& L, float (&acc)[kSlots], int kh,
                                                  int nt, float ph, int nidx_spare) {
  static_assert(!MASKC || (FAST && NS != 0), "the constant mask is a fast slot-weight form");
  const float kf = (float)(kh + 1);
  const float nyq = a.nyq;
  const bool harm = kh < a.K;
  const int n = FAST ? kSeg : nt;
  // (rolled: the blocks' reads and sums stay within a few registers)
#pragma unroll 1
  for (int i0 = 0; i0 < n; i0 += kBlk) {
    FrameRec r[kBlk];
    float hs[kBlk], cf[kBlk], ex[kBlk];
    float4 w[kBlk];
#pragma unroll
    for (int j = 0; j < kBlk; ++j) {
      const int i = i0 + j;
      if constexpr (NS == 0) {
        r[j] = L.fr[i];
        hs[j] = L.pk[i].y;
        cf[j] = L.pk[i].z;
        ex[j] = L.pk[i].w * L.noise[i + nidx_spare];
      } else {
        const float4 q = L.pk[i];
        r[j].f0 = q.x;
        hs[j] = q.y;
        cf[j] = q.z;
        ex[j] = q.w * L.noise[i + nidx_spare];
      }
      w[j] = L.wt[i];
    }
#pragma unroll
    for (int j = 0; j < kBlk; ++j) {
      const int i = i0 + j;
      if (!FAST && i >= nt) break;
      const float freq = kf * r[j].f0;
      float inc;
      if (FAST) {
        const float q0 = freq * a.rsr;
        inc = fmaf(fmaf(-q0, a.sr, freq), a.rsr, q0);
      } else {
        inc = div_sr(freq, a.sr, a.rsr);
      }
      const float p = ph;
      ph = FAST ? __builtin_amdgcn_fractf(ph + inc) : phasor_wrap(ph + inc);
      // every lane evaluates the sine (opaque to the compiler), so the
      // selects below stay branch-free instead of nested exec-mask regions
      float sv = sin2pi(p);
      asm volatile("" : "+v"(sv));
      const float hm = (sv - hs[j]) * cf[j];
      const float dm = harm ? (MASKC || freq < nyq ? hm : 0.0f) : ex[j];
      slot_acc<NS>(acc, r[j], w[j], dm);
    }
  }
}

// A gain pass: column K + q (q = 0: gain, 1: noise gain, q >= 2: tap q-2;
// columns past NC read the window's last tap and are not stored).
template <int NS, class SL>
__device__ __forceinline__ void bwd_gain_pass(const SL& L, float (&acc)[kSlots], int q, int nt, int NF) {
  const int nidx = min(max(q - 2, 0), NF - 1);
#pragma unroll 1
  for (int i0 = 0; i0 < nt; i0 += kBlk) {
    FrameRec r[kBlk];
    float ex[kBlk];
    float4 w[kBlk];
#pragma unroll
    for (int j = 0; j < kBlk; ++j) {
      const int i = i0 + j;
      if constexpr (NS == 0) r[j] = L.fr[i];
      w[j] = L.wt[i];
      ex[j] = q == 0 ? L.dg[i] : (q == 1 ? L.dng[i] : L.pk[i].w * L.noise[i + nidx]);
    }
#pragma unroll
    for (int j = 0; j < kBlk; ++j) {
      if (i0 + j >= nt) break;
      slot_acc<NS>(acc, r[j], w[j], ex[j]);
    }
  }
}

// A column's four slot sums into the wave's LDS (the staged rows' space).
template <class SL>
__device__ __forceinline__ void store_slots(const float (&acc)[kSlots], SL& L, int c) {
#pragma unroll
  for (int j = 0; j < kSlots; ++j) L.row[j][c] = acc[j];
}

// MssGrad: with part, the prediction's gradient is gathered here from the
// spectral loss's tile partials (plus the time-domain MSE term) and also
// stored to dy, instead of in a launch of its own between the two kernels.
struct MssGrad {
  const float* part;  // [B][ntiles][kMssAcc] or null: read dy
  const float* x;     // the prediction and the target ([B][T]) for the MSE term
  const float* tgt;
  int ntiles;
  float w_mse;
};

template <class SL>
__device__ __forceinline__ void bwd_segment(const SynthArgs& a, SL& L, float* __restrict__ dy, const MssGrad& mg,
                                            const float* __restrict__ aux, int s, int b, int lane) {
  const int t0 = s * kSeg, nt = min(kSeg, a.T - t0);
  int nslot;
  bool pairs;  // (the backward's slot-weight sums need no distinct rows)
  const int fast = stage_segment(a, L, s, b, lane, nt, false, nslot, pairs);
  // the slot-weight form needs every per-frame factor of the column
  // gradients (and the noise window) below 2^50 in magnitude, so that no
  // weight-0 term is 0 * inf or 0 * NaN and no sum overflows
  bool bnd;
  {
    float hs = 0.f, coef = 0.f, dg = 0.f, dng = 0.f, dfl = 0.f;
    if (lane < nt) {
      const int t = t0 + lane;
      const FrameRec r = L.fr[lane];
      const int slo = r.slots & 255, shi = r.slots >> 8;
      const size_t bt = (size_t)b * a.T + t, plane = (size_t)a.B * a.T;
      const float hsum = aux[bt], den = aux[plane + bt], filt = aux[2 * plane + bt];
      const float gain = r.omf * L.row[slo][a.K] + r.frac * L.row[shi][a.K];
      const float ngain = r.omf * L.row[slo][a.K + 1] + r.frac * L.row[shi][a.K + 1];
      const float uv = a.uvf[bt];
      float g;
      if (mg.part) {
        // the two tiles whose accumulators hold sample t, in the order the
        // separate gather added them, then the MSE term's 2 w (x - tgt) / B
        const int tile = t / kMssTile, ta = tile * kMssTile;
        const float* pp = mg.part + ((size_t)b * mg.ntiles + tile) * kMssAcc;
        g = pp[t - ta + kMssHalo];
        if (tile + 1 < mg.ntiles && t >= ta + kMssTile - kMssHalo) g += pp[kMssAcc + (t - ta - kMssTile + kMssHalo)];
        if (mg.w_mse != 0.f) g += mg.w_mse * (2.f * (mg.x[bt] - mg.tgt[bt])) * (1.0f / (float)a.B);
        dy[bt] = g;
      } else {
        g = dy[bt];
      }
      hs = hsum;
      coef = (((g * gain) * uv) * a.hscale) / den;
      dg = ((g * hsum) * uv) * a.hscale;
      dng = ((g * filt) * 0.12f) * a.nscale;
      dfl = ((g * ngain) * 0.12f) * a.nscale;
    }
    L.pk[lane] = make_float4(L.fr[lane].f0, hs, coef, dfl);
    L.dg[lane] = dg;
    L.dng[lane] = dng;
    constexpr float kBig = 0x1p50f;
    bnd = fabsf(hs) < kBig && fabsf(coef) < kBig && fabsf(dg) < kBig && fabsf(dng) < kBig && fabsf(dfl) < kBig;
    for (int i = lane; i < a.NF - 1 + kSeg; i += 64) bnd = bnd && fabsf(L.noise[i]) < kBig;
  }
  wave_sync();
  const int ns = !__all(bnd) ? 0 : (nslot <= 2 ? 2 : kSlots);

  const int NC = a.K + 2 + a.NF;
  const int spare = 64 * harmonic_groups(a.K) - a.K;          // lanes past K in the last group
  const int npass = max(1, (NC - a.K - spare + 63) / 64);      // gain passes
  // the segment's f0 range, for the harmonics' Nyquist masks
  float flo = 0.0f, fhi = 0.0f;
  if (fast) {
    flo = fhi = L.fr[lane].f0;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
      flo = fminf(flo, __shfl_xor(flo, d, 64));
      fhi = fmaxf(fhi, __shfl_xor(fhi, d, 64));
    }
  }
  for (int g = 0; g < SL::kGroups; ++g) {
    if (64 * g >= a.K) break;
    // harmonic kh, or (kh >= K) the tap column K + 64 npass + kh - K
    const int kh = 64 * g + lane;
    const bool harm = kh < a.K;
    const int c = harm ? kh : a.K + 64 * npass + (kh - a.K);
    const int nidx = harm ? 0 : min(c - a.K - 2, a.NF - 1);
    const float ph = a.ckpt[((size_t)s * a.B + b) * a.K + (harm ? kh : 0)];
    float acc[kSlots] = {0.f, 0.f, 0.f, 0.f};
    // Nyquist mask of harmonic kh over the segment: freq = RN((k+1) f0)
    // is monotone in f0, so the frames' extreme f0 decide whether every
    // frame is below (on) or none is (off); a lane between the two needs
    // the per-frame test
    bool mixed = false, off = false;
    if (fast) {
      const float kf = (float)(kh + 1);
      const bool on = kf * fhi < a.nyq;
      off = !(kf * flo < a.nyq);
      mixed = harm && !on && !off;
    }
    const bool maskc = !__any(mixed);
    if (fast && ns == 2 && maskc)
      bwd_harmonic_pass<true, 2, true>(a, L, acc, kh, nt, ph, nidx);
    else if (fast && ns == kSlots && maskc)
      bwd_harmonic_pass<true, kSlots, true>(a, L, acc, kh, nt, ph, nidx);
    else if (fast && ns == 2)
      bwd_harmonic_pass<true, 2>(a, L, acc, kh, nt, ph, nidx);
    else if (fast && ns == kSlots)
      bwd_harmonic_pass<true, kSlots>(a, L, acc, kh, nt, ph, nidx);
    else if (fast)
      bwd_harmonic_pass<true, 0>(a, L, acc, kh, nt, ph, nidx);
    else
      bwd_harmonic_pass<false, 0>(a, L, acc, kh, nt, ph, nidx);
    if (fast && ns != 0 && maskc && harm && off) {
      // masked in every frame: the per-frame form adds only zeros
#pragma unroll
      for (int j = 0; j < kSlots; ++j) acc[j] = 0.0f;
    }
    if (c < NC) store_slots(acc, L, c);
  }
  for (int pp = 0; pp < npass; ++pp) {
    // gain pass pp: column K + 64 pp + lane
    const int q = 64 * pp + lane, c = a.K + q;
    float acc[kSlots] = {0.f, 0.f, 0.f, 0.f};
    if (ns == 2)
      bwd_gain_pass<2>(L, acc, q, nt, a.NF);
    else if (ns == kSlots)
      bwd_gain_pass<kSlots>(L, acc, q, nt, a.NF);
    else
      bwd_gain_pass<0>(L, acc, q, nt, a.NF);
    if (c < NC) store_slots(acc, L, c);
  }
}

// Head backward of one control row (the rules of k_heads_bwd,
// Model.swift:100-114) on one wave: lane l holds d ctrl of columns
// l + 64 q (q < QN) in s[q] and Z of those columns in zin[q] (read for
// columns below K + 2 + NF) and gets dZ of those columns in out[q].  The
// row sums (softplus over the K amplitudes, |tanh| over the NF noise taps,
// then the two dot products) add each 64-column block's wave sum in block
// order.  Columns past K + 2 + NF get 0.
template <int QN>
__device__ __forceinline__ void head_row_bwd(const float (&s)[QN], const float (&zin)[QN], float (&out)[QN],
                                             int lane, int K, int NF) {
  float z[QN], sp[QN], th[QN];
  float den = 0.f, nrm = 0.f;
#pragma unroll
  for (int q = 0; q < QN; ++q) {
    const int c = lane + 64 * q;
    const bool amp = c < K, noise = c >= K + 2 && c < K + 2 + NF;
    z[q] = c < K + 2 + NF ? zin[q] : 0.f;
    sp[q] = amp ? softplus(z[q]) : 0.f;
    th[q] = noise ? fast_tanh(z[q]) : 0.f;
  }
#pragma unroll
  for (int q = 0; q < QN; ++q) {
    den += wave_sum(sp[q]);
    nrm += wave_sum(fabsf(th[q]));
  }
  den += 1e-6f;
  nrm += 1e-4f;
  const float rden = rcp_rn(den), rnrm = rcp_rn(nrm);
  float dot = 0.f, dot2 = 0.f;
#pragma unroll
  for (int q = 0; q < QN; ++q) {
    const int c = lane + 64 * q;
    const bool amp = c < K, noise = c >= K + 2 && c < K + 2 + NF;
    dot += wave_sum(amp ? s[q] * (sp[q] * rden) : 0.f);
    dot2 += wave_sum(noise ? s[q] * (th[q] * rnrm) : 0.f);
  }
#pragma unroll
  for (int q = 0; q < QN; ++q) {
    const int c = lane + 64 * q;
    const bool amp = c < K, gain = c == K || c == K + 1, noise = c >= K + 2 && c < K + 2 + NF;
    float o = 0.f;  // padding columns stay exactly zero
    if (amp) {
      o = (s[q] - dot) * rden * softplus_grad(z[q]);
    } else if (gain) {
      o = s[q] * softplus_grad(z[q]);
    } else if (noise) {
      const float sg = th[q] > 0.f ? 1.f : (th[q] < 0.f ? -1.f : 0.f);
      o = (s[q] - sg * dot2) * rnrm * (1.f - th[q] * th[q]);
    }
    out[q] = o;
  }
}

// The row table of the backward runs (a static table, from the segment
// rows and the row list): per run, entry 0 = {rows, 0, 0, 0}, then one
// entry per control row its segments touch, in order of the row's first
// in-run (segment, slot) entry: {row, before | outside << 8 | n << 16,
// entries lo, hi}: where the run's sum goes (d ctrl when no entry of the row
// lies outside the run, else the boundary partial at index `before`, the
// number of runs listed before this one) and the run's n entries of the row
// in list order, 4 bits each: (segment - s0) * 4 + slot.
constexpr int kRunRows = kRunSegs * kSlots;
static_assert(kRunRows <= 16 && kRowEntries <= 16, "run entries pack into 64 bits");

__global__ void k_run_table(const float* __restrict__ seg_rows, const float* __restrict__ row_list,
                            uint4* __restrict__ tab, int nseg) {
  // one wave per run, one lane per (segment, slot) of the run: the lane
  // holding its row's first in-run entry lists the row
  const int run = blockIdx.x, lane = threadIdx.x;
  const int s0 = run * kRunSegs, s1 = min(s0 + kRunSegs, nseg);
  const int nq = (s1 - s0) * kSlots;
  int r = -1;
  if (lane < nq) {
    const float rf = seg_rows[(size_t)s0 * kSlots + lane];
    r = rf >= 0.0f ? (int)rf : -1;
  }
  float e[kRowEntries];
#pragma unroll
  for (int i = 0; i < kRowEntries; ++i) e[i] = r >= 0 ? row_list[(size_t)r * kRowEntries + i] : -1.0f;
  int first = -1, before = 0, prev = -1, n = 0;
  bool outside = false, live = true;
  unsigned long long ent = 0;
#pragma unroll
  for (int i = 0; i < kRowEntries; ++i) {
    live = live && e[i] >= 0.0f;
    if (live) {
      const int en = (int)e[i], rr = en / kSlots / kRunSegs;
      if (rr == run) {
        if (first < 0) first = en;
        ent |= (unsigned long long)(en - s0 * kSlots) << (4 * n);
        ++n;
      } else {
        outside = true;
        if (first < 0 && rr != prev) ++before;
      }
      prev = rr;
    }
  }
  const bool own = r >= 0 && first == s0 * kSlots + lane;
  const unsigned long long m = __ballot(own);
  uint4* t = tab + (size_t)run * (kRunRows + 1);
  if (own) {
    const int idx = __popcll(m & ((1ull << lane) - 1ull));
    t[1 + idx] = make_uint4((unsigned)r, (unsigned)(before | (outside ? 1 : 0) << 8 | n << 16), (unsigned)ent,
                            (unsigned)(ent >> 32));
  }
  if (lane == 0) t[0] = make_uint4((unsigned)__popcll(m), 0u, 0u, 0u);
}

int launch_run_table(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=segment rows ([nseg][4]) [1]=row list ([F][16]) [2]=run table ([nruns][17] x 16 bytes) [3]=nseg [4]=F
  const int64_t segr = op.arg[0], rowl = op.arg[1], tab = op.arg[2], nseg = op.arg[3], F = op.arg[4];
  DGEN_REQUIRE(nseg > 0 && nseg <= (1 << 22) && F > 0 && F <= (1 << 22), "run_table: nseg %lld F %lld",
               (long long)nseg, (long long)F);
  const int64_t nruns = (nseg + kRunSegs - 1) / kRunSegs;
  DGEN_CHECK_CELL(L, segr, nseg * kSlots, "run_table.seg_rows");
  DGEN_CHECK_CELL(L, rowl, F * kRowEntries, "run_table.row_list");
  DGEN_CHECK_CELL(L, tab, nruns * (kRunRows + 1) * 4, "run_table.table");
  DGEN_REQUIRE(tab % 4 == 0, "run_table: table cell must be 16-byte aligned");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_run_table, dim3((unsigned)nruns), dim3(64), 0, L.stream, cell(L, segr), cell(L, rowl),
                     reinterpret_cast<uint4*>(cell(L, tab)), (int)nseg);
  DGEN_LAUNCH_CHECK("k_run_table");
  return 0;
}

template <class SL>
__global__ __launch_bounds__(64 * kRunSegs) void k_synth_bwd(SynthArgs a, float* __restrict__ dy,
                                                             const float* __restrict__ aux,
                                                             const uint4* __restrict__ runtab,
                                                             float* __restrict__ dctrl, float* __restrict__ bpart,
                                                             MssGrad mg) {
  __shared__ SL lds[kRunSegs];
  __shared__ uint4 s_tab[kRunRows + 1];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int nseg = (a.T + kSeg - 1) / kSeg;
  const int run = blockIdx.x, b = blockIdx.y;
  const int s0 = run * kRunSegs;
  // the run's row table, loaded at the start and staged after wave 0's segment
  uint4 tv = make_uint4(0u, 0u, 0u, 0u);
  if (wave == 0 && lane <= kRunRows) tv = runtab[(size_t)run * (kRunRows + 1) + lane];
  if (s0 + wave < nseg) bwd_segment(a, lds[wave], dy, mg, aux, s0 + wave, b, lane);
  if (wave == 0 && lane <= kRunRows) s_tab[lane] = tv;
  __syncthreads();
  // each row's sum over the run's entries in list order, a wave per row
  // (lane l: columns l + 64 q)
  constexpr int QN = SL::kMaxNC / 64;
  const int NC = a.K + 2 + a.NF;
  const int ntab = (int)s_tab[0].x;
  for (int t = wave; t < ntab; t += kRunSegs) {
    const uint4 rr = s_tab[1 + t];
    const int before = rr.y & 255, n_in = rr.y >> 16;
    const bool outside = ((rr.y >> 8) & 255) != 0;
    const unsigned long long ent = (unsigned long long)rr.z | (unsigned long long)rr.w << 32;
    const size_t row = (size_t)b * a.F + rr.x;
    float* dst = outside ? bpart + (row * kRunParts + min(before, kRunParts - 1)) * a.ldc : dctrl + row * a.ldc;
#pragma unroll
    for (int q = 0; q < QN; ++q) {
      const int c = lane + 64 * q;
      float sum = 0.0f;
      if (c < NC)
        for (int i = 0; i < n_in; ++i) {
          const int le = (int)((ent >> (4 * i)) & 15ull);
          sum += lds[le / kSlots].row[le % kSlots][c];
        }
      // a row in more runs than the partials hold (not produced by a
      // playhead that wraps once) is marked NaN
      if (c < a.ldc) dst[c] = before < kRunParts ? sum : __builtin_nanf("");
    }
  }
}

// d ctrl rows the synth backward left as boundary partials, a wave per row
// (lane l: columns l + 64 q): row f's runs (the distinct runs of its listed
// entries, in list order) each left one partial; they are added in that
// order.  A row no segment touches is zero.  A row within one run was
// completed by the synth backward (with Z it is read here for the head
// backward; else skipped).  With Z, the head backward of every row.
template <bool HEADS, int QN>
__global__ __launch_bounds__(256) void k_synth_bwd_reduce(const float* __restrict__ bpart,
                                                          const float* __restrict__ row_list, float* __restrict__ dctrl,
                                                          int B, int NC, int ldc, int F, const float* __restrict__ Z,
                                                          float* __restrict__ dZ, int K, int NF) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int f = blockIdx.x * 4 + wave, b = blockIdx.y;
  if (f >= F) return;
  const size_t row = (size_t)b * F + f;
  // Every load that does not depend on the row's run count is issued
  // first: the row list (entry e on lane e), d ctrl as the synth backward
  // left it (used when the row is complete) and, with the heads, Z.  The
  // partials are the only dependent stage, for shared rows.
  const float* lst = row_list + (size_t)f * kRowEntries;
  const float ef = lane < kRowEntries ? lst[lane] : -1.0f;
  float dc[QN], zr[QN];
#pragma unroll
  for (int q = 0; q < QN; ++q) {
    const int c = lane + 64 * q;
    dc[q] = c < NC ? dctrl[row * ldc + c] : 0.f;
    zr[q] = HEADS && c < NC ? Z[row * ldc + c] : 0.f;
  }
  // the row's runs: the entries before the first negative one, a new run
  // wherever an entry's run differs from the previous entry's (uniform)
  const int nvalid = (int)__builtin_ctzll(__ballot(lane >= kRowEntries || ef < 0.0f));
  const int rr = lane < nvalid ? (int)ef / kSlots / kRunSegs : -1;
  const int rprev = __shfl_up(rr, 1, 64);
  const int nruns = (int)__popcll(__ballot(lane < nvalid && (lane == 0 || rr != rprev)));
  const bool done = nruns == 1;  // completed by the synth backward
  if (done && !HEADS) return;
  float s[QN];
#pragma unroll
  for (int q = 0; q < QN; ++q) {
    const int c = lane + 64 * q;
    float v = 0.f;
    if (done) {
      s[q] = dc[q];
      continue;
    }
    if (c < NC) {
      const float* bp = bpart + row * kRunParts * ldc + c;
      float u[kRunParts];
#pragma unroll
      for (int p = 0; p < kRunParts; ++p) u[p] = p < nruns ? bp[(size_t)p * ldc] : 0.f;
#pragma unroll
      for (int p = 0; p < kRunParts; ++p)
        if (p < nruns) v += u[p];
      if (nruns > kRunParts) v = __builtin_nanf("");
    }
    s[q] = v;
    if (c < ldc) dctrl[row * ldc + c] = v;
  }
  if constexpr (HEADS) {
    float dz[QN];
    head_row_bwd<QN>(s, zr, dz, lane, K, NF);
#pragma unroll
    for (int q = 0; q < QN; ++q)
      if (lane + 64 * q < ldc) dZ[row * ldc + lane + 64 * q] = dz[q];
  }
}

static int synth_args(const Launch& L, const dgen_hip_op& op, SynthArgs& a, const char* who) {
  // arg: [0]=ctrl [1]=f0 frames [2]=uv frames [3]=lerp [4]=checkpoints [5]=y/dy [6]=B [7]=K [8]=NF [9]=F [10]=T
  //      [11]=seg (64) [12]=partials (bwd) [13]=noise [14]=ldc [15]=seg_rows
  const int64_t B = op.arg[6], K = op.arg[7], NF = op.arg[8], F = op.arg[9], T = op.arg[10], seg = op.arg[11];
  const int64_t ldc = op.arg[14];
  DGEN_REQUIRE(B > 0 && B <= 65535 && K > 0 && K <= kMaxKWide && NF > 0 && F > 0 && T > 0 && T <= (1 << 26) &&
                   seg == kSeg && K + 2 + NF <= kMaxNCWide && ldc >= K + 2 + NF,
               "%s: B %lld K %lld NF %lld F %lld T %lld seg %lld ldc %lld", who, (long long)B, (long long)K,
               (long long)NF, (long long)F, (long long)T, (long long)seg, (long long)ldc);
  DGEN_REQUIRE(op.farg[0] > 0.f && op.farg[0] < 1e30f, "%s: sample rate %g", who, (double)op.farg[0]);
  DGEN_REQUIRE(op.arg[3] % 4 == 0, "%s: lerp table must be 16-byte aligned", who);
  const int64_t nseg = (T + seg - 1) / seg;
  DGEN_CHECK_CELL(L, op.arg[0], B * F * ldc, "synth.ctrl");
  DGEN_CHECK_CELL(L, op.arg[1], B * T, "synth.f0_frames");
  DGEN_CHECK_CELL(L, op.arg[2], B * T, "synth.uv_frames");
  DGEN_CHECK_CELL(L, op.arg[3], T * 8, "synth.lerp");
  DGEN_CHECK_CELL(L, op.arg[4], nseg * B * K, "synth.checkpoints");
  DGEN_CHECK_CELL(L, op.arg[5], B * T, "synth.y");
  DGEN_CHECK_CELL(L, op.arg[13], T, "synth.noise");
  DGEN_CHECK_CELL(L, op.arg[15], nseg * kSlots, "synth.seg_rows");
  if (L.dry) return 0;
  a.ctrl = cell(L, op.arg[0]);
  a.f0f = cell(L, op.arg[1]);
  a.uvf = cell(L, op.arg[2]);
  a.lerp = cell(L, op.arg[3]);
  a.ckpt = cell(L, op.arg[4]);
  a.noise = cell(L, op.arg[13]);
  a.seg_rows = cell(L, op.arg[15]);
  a.ldc = (int)ldc;
  a.B = (int)B;
  a.K = (int)K;
  a.NF = (int)NF;
  a.F = (int)F;
  a.T = (int)T;
  // phase increments use the host sample rate (u_phasor divides by
  // hostSampleRate, Definitions.swift:96-102); the Nyquist mask uses the
  // graph's rate (DGenConfig.sampleRate, Synth.swift:158-167)
  a.sr = host_rate(L, op.farg[0]);
  a.rsr = 1.0f / a.sr;
  a.nyq = op.farg[0] * 0.5f;
  a.hscale = op.farg[1];
  a.nscale = op.farg[2];
  a.f0lim = fast_f0_limit((int)K);
  return 0;
}

// The narrow LDS layout when the harmonics fit one group and the columns
// (and the row stride) 128.
static bool synth_narrow(const SynthArgs& a) { return a.K <= kMaxK && a.K + 2 + a.NF <= kMaxNC && a.ldc <= kMaxNC; }

int launch_synth_fwd(const Launch& L, const dgen_hip_op& op) {
  SynthArgs a{};
  int rc = synth_args(L, op, a, "synth_fwd");
  if (rc) return rc;
  if (op.arg[12] >= 0) DGEN_CHECK_CELL(L, op.arg[12], 3 * op.arg[6] * op.arg[10], "synth_fwd.aux");
  if (L.dry) return 0;
  const int nseg = (a.T + kSeg - 1) / kSeg;
  const dim3 grid((unsigned)((nseg + kWavesFwd - 1) / kWavesFwd), (unsigned)a.B), block(64 * kWavesFwd);
  float* aux = op.arg[12] >= 0 ? cell(L, op.arg[12]) : nullptr;
  if (synth_narrow(a))
    hipLaunchKernelGGL(k_synth_fwd<SegLds>, grid, block, 0, L.stream, a, cell(L, op.arg[5]), aux);
  else
    hipLaunchKernelGGL(k_synth_fwd<SegLdsWide>, grid, block, 0, L.stream, a, cell(L, op.arg[5]), aux);
  DGEN_LAUNCH_CHECK("k_synth_fwd");
  return 0;
}

int launch_synth_bwd(const Launch& L, const dgen_hip_op& op) {
  SynthArgs a{};
  int rc = synth_args(L, op, a, "synth_bwd");
  if (rc) return rc;
  // [12]=boundary partials ([B][F][6][ldc]) [16]=tape [17]=run table (DGEN_HIP_K_RUN_TABLE) [18]=dctrl
  // [19]=1: [5] (dy) is gathered here from the spectral loss's tile
  // partials [20] ([B][ntiles][kMssAcc]) plus farg[3] times the MSE term of
  // the prediction [21] and target [22] ([B][T]), and stored to [5]
  const int64_t T = op.arg[10], B = op.arg[6], F = op.arg[9], ldc = op.arg[14];
  DGEN_REQUIRE(op.arg[19] == 0 || op.arg[19] == 1, "synth_bwd: gather flag %lld", (long long)op.arg[19]);
  MssGrad mg{};
  const int64_t ntiles = (T + kMssTile - 1) / kMssTile;
  if (op.arg[19] == 1) {
    DGEN_CHECK_CELL(L, op.arg[20], B * ntiles * kMssAcc, "synth_bwd.mss_tiles");
    if (op.farg[3] != 0.f) {
      DGEN_CHECK_CELL(L, op.arg[21], B * T, "synth_bwd.prediction");
      DGEN_CHECK_CELL(L, op.arg[22], B * T, "synth_bwd.target");
    }
  }
  const int64_t nseg = (T + kSeg - 1) / kSeg;
  DGEN_CHECK_CELL(L, op.arg[12], B * F * kRunParts * ldc, "synth_bwd.boundary_partials");
  DGEN_CHECK_CELL(L, op.arg[16], 3 * B * T, "synth_bwd.aux");
  DGEN_CHECK_CELL(L, op.arg[17], (nseg + kRunSegs - 1) / kRunSegs * (kRunRows + 1) * 4, "synth_bwd.run_table");
  DGEN_REQUIRE(op.arg[17] % 4 == 0, "synth_bwd: run table cell must be 16-byte aligned");
  DGEN_REQUIRE(ldc <= kMaxNCWide, "synth_bwd: row stride %lld > %d", (long long)ldc, kMaxNCWide);
  DGEN_CHECK_CELL(L, op.arg[18], B * F * ldc, "synth_bwd.dctrl");
  if (L.dry) return 0;
  if (op.arg[19] == 1) {
    mg.part = cell(L, op.arg[20]);
    mg.ntiles = (int)ntiles;
    mg.w_mse = op.farg[3];
    if (mg.w_mse != 0.f) {
      mg.x = cell(L, op.arg[21]);
      mg.tgt = cell(L, op.arg[22]);
    }
  }
  const dim3 grid((unsigned)((nseg + kRunSegs - 1) / kRunSegs), (unsigned)a.B), block(64 * kRunSegs);
  if (synth_narrow(a))
    hipLaunchKernelGGL(k_synth_bwd<SegLdsBwd>, grid, block, 0, L.stream, a, cell(L, op.arg[5]), cell(L, op.arg[16]),
                       reinterpret_cast<const uint4*>(cell(L, op.arg[17])), cell(L, op.arg[18]), cell(L, op.arg[12]),
                       mg);
  else
    hipLaunchKernelGGL(k_synth_bwd<SegLdsBwdWide>, grid, block, 0, L.stream, a, cell(L, op.arg[5]),
                       cell(L, op.arg[16]), reinterpret_cast<const uint4*>(cell(L, op.arg[17])),
                       cell(L, op.arg[18]), cell(L, op.arg[12]), mg);
  DGEN_LAUNCH_CHECK("k_synth_bwd");
  return 0;
}

int launch_synth_bwd_reduce(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=boundary partials [1]=row_list [2]=dctrl [3]=B [4]=NC [5]=F [6]=T [7]=seg [8]=ldc
  //      [9]=Z or -1 [10]=dZ [11]=K [12]=NF (with Z: the head backward too)
  const int64_t part = op.arg[0], rl = op.arg[1], dc = op.arg[2], B = op.arg[3], NC = op.arg[4], F = op.arg[5],
                T = op.arg[6], seg = op.arg[7], ldc = op.arg[8];
  const int64_t Zc = op.arg[9], dZc = op.arg[10], K = op.arg[11], NF = op.arg[12];
  const bool heads = Zc >= 0;
  DGEN_REQUIRE(B > 0 && B <= 65535 && NC > 0 && ldc >= NC && ldc <= kMaxNCWide && F > 0 && T > 0 && seg == kSeg,
               "synth_bwd_reduce: B %lld NC %lld F %lld T %lld seg %lld ldc %lld", (long long)B, (long long)NC,
               (long long)F, (long long)T, (long long)seg, (long long)ldc);
  DGEN_CHECK_CELL(L, part, B * F * kRunParts * ldc, "synth_bwd_reduce.boundary_partials");
  DGEN_CHECK_CELL(L, rl, F * kRowEntries, "synth_bwd_reduce.row_list");
  DGEN_CHECK_CELL(L, dc, B * F * ldc, "synth_bwd_reduce.dctrl");
  if (heads) {
    DGEN_REQUIRE(K > 0 && NF > 0 && K + 2 + NF == NC, "synth_bwd_reduce: heads K %lld NF %lld NC %lld", (long long)K,
                 (long long)NF, (long long)NC);
    DGEN_CHECK_CELL(L, Zc, B * F * ldc, "synth_bwd_reduce.Z");
    DGEN_CHECK_CELL(L, dZc, B * F * ldc, "synth_bwd_reduce.dZ");
  }
  if (L.dry) return 0;
  const dim3 grid((unsigned)((F + 3) / 4), (unsigned)B), block(256);
  float* zp = heads ? cell(L, Zc) : nullptr;
  float* dzp = heads ? cell(L, dZc) : nullptr;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, block, 0, L.stream, cell(L, part), cell(L, rl), cell(L, dc), (int)B, (int)NC,
                       (int)ldc, (int)F, zp, dzp, (int)K, (int)NF);
  };
  if (ldc <= 128)
    heads ? go(k_synth_bwd_reduce<true, 2>) : go(k_synth_bwd_reduce<false, 2>);
  else
    heads ? go(k_synth_bwd_reduce<true, 8>) : go(k_synth_bwd_reduce<false, 8>);
  DGEN_LAUNCH_CHECK("k_synth_bwd_reduce");
  return 0;
}

}  // namespace dgen
