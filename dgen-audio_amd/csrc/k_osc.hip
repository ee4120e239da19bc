// Deterministic phasor bank -> sum -> one-pole history (config 1).
//
// Signal.phasor(Tensor) lowers to the stateless deterministicPhasor
// (Sources/DGenLazy/SignalTensor.swift:67-80, Sources/DGen/Emit+State.swift:
// 370-387): phase = r - floor(r), r = (f / sr) * n with n the frame index in
// this call, so the oscillator sum is frame-parallel.  The history one-pole
// y[n] = x[n] + pole * y[n-1] (Emit+State.swift:150-224) is a first-order
// linear recurrence, evaluated as a two-pass scan over 256-frame tiles:
//   k_osc_tiles  one thread per frame: the oscillator sum, then the tile's
//                zero-state response by a workgroup scan of the affine maps
//                y -> pole*y + x[n]; writes it and the tile's map (pole^len,
//                zero-state end);
//   k_osc_apply  each workgroup composes the maps of the tiles before it
//                (a workgroup scan over at most kMaxFusedTiles tiles) and adds
//                pole^(i+1) * carry to its zero-state response.
// Longer signals compose the tile maps in a single-workgroup pass
// (k_osc_carries) between the two.  Every output store maps non-finite values
// to 0 (CRenderer.swift:1021-1039).  The scan reassociates the recurrence's
// fp32 sums; the oscillator sum keeps the reference's order over k.
#pragma clang fp contract(off)

#include "internal.h"

namespace dgen {

constexpr int kTile = 256;             // frames per workgroup (one per thread)
constexpr int kMaxFusedTiles = 1024;   // tiles k_osc_apply scans itself
constexpr int kOscLds = 1024;          // oscillators staged in LDS per pass

// Affine map y -> a*y + b; compose(first, second) applies first, then second.
struct Aff {
  float a, b;
};
__device__ __forceinline__ Aff compose(Aff f, Aff s) { return Aff{f.a * s.a, s.a * f.b + s.b}; }

// Inclusive scan of one map per thread over a 256-thread workgroup (four
// waves): shuffles within each wave, then the wave totals through LDS.
__device__ __forceinline__ Aff block_scan(Aff v, Aff* lds_tot) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    Aff u{__shfl_up(v.a, off, 64), __shfl_up(v.b, off, 64)};
    if (lane >= off) v = compose(u, v);
  }
  if (lane == 63) lds_tot[w] = v;
  __syncthreads();
  Aff pre{1.f, 0.f};
  for (int j = 0; j < w; ++j) pre = compose(pre, lds_tot[j]);
  __syncthreads();
  return w ? compose(pre, v) : v;
}

__global__ __launch_bounds__(kTile) void k_osc_tiles(const float* __restrict__ freqs, const float* __restrict__ amps,
                                                     int nosc, float sr, int frames, float pole,
                                                     float* __restrict__ zs, float2* __restrict__ tiles) {
  __shared__ float s_inc[kOscLds], s_amp[kOscLds];
  __shared__ Aff s_tot[kTile / 64];
  const int n = blockIdx.x * kTile + threadIdx.x;
  const float fn = (float)n;
  float acc = 0.f;
  for (int k0 = 0; k0 < nosc; k0 += kOscLds) {
    const int kn = min(kOscLds, nosc - k0);
    __syncthreads();
    for (int k = threadIdx.x; k < kn; k += kTile) {
      s_inc[k] = freqs[k0 + k] / sr;  // phaseIncrement = freq / sampleRate
      s_amp[k] = amps[k0 + k];
    }
    __syncthreads();
    for (int k = 0; k < kn; ++k) {
      const float r = s_inc[k] * fn;
      const float phase = r - floorf(r);
      // sin(phase * 2pi): the transcendental unit takes revolutions
      acc = acc + sin_2pif_hw(phase) * s_amp[k];
    }
  }
  const bool live = n < frames;
  Aff v = block_scan(Aff{live ? pole : 1.f, live ? acc : 0.f}, s_tot);
  if (live) zs[n] = v.b;
  if (threadIdx.x == kTile - 1) tiles[blockIdx.x] = make_float2(v.a, v.b);
}

// Carries of any number of tiles: one workgroup, blocks of 256 tile maps
// scanned in parallel, the running carry composed block by block.
__global__ __launch_bounds__(kTile) void k_osc_carries(const float2* __restrict__ tiles, float* __restrict__ carry,
                                                       int ntiles) {
  __shared__ Aff s_tot[kTile / 64];
  __shared__ Aff s_inc[kTile];
  float run = 0.f;  // y entering the block
  for (int t0 = 0; t0 < ntiles; t0 += kTile) {
    const int t = t0 + threadIdx.x;
    const float2 m = t < ntiles ? tiles[t] : make_float2(1.f, 0.f);
    const Aff inc = block_scan(Aff{m.x, m.y}, s_tot);
    s_inc[threadIdx.x] = inc;
    __syncthreads();
    // carry into tile t: the maps of the block's tiles before t applied to `run`
    const Aff ex = threadIdx.x ? s_inc[threadIdx.x - 1] : Aff{1.f, 0.f};
    if (t < ntiles) carry[t] = ex.a * run + ex.b;
    const Aff blk = s_inc[kTile - 1];
    run = blk.a * run + blk.b;
    __syncthreads();
  }
}

template <bool FUSED>
__global__ __launch_bounds__(kTile) void k_osc_apply(const float* __restrict__ zs, const float2* __restrict__ tiles,
                                                     const float* __restrict__ carry, int frames, float pole,
                                                     float* __restrict__ out) {
  __shared__ Aff s_tot[kTile / 64];
  __shared__ float s_carry;
  const int g = blockIdx.x;
  if constexpr (FUSED) {
    // compose the maps of tiles 0 .. g-1 (g <= kMaxFusedTiles): four per thread
    Aff v{1.f, 0.f};
#pragma unroll
    for (int j = 0; j < kMaxFusedTiles / kTile; ++j) {
      const int t = threadIdx.x * (kMaxFusedTiles / kTile) + j;
      if (t < g) {
        const float2 m = tiles[t];
        v = compose(v, Aff{m.x, m.y});
      }
    }
    v = block_scan(v, s_tot);
    if (threadIdx.x == kTile - 1) s_carry = v.b;  // the composed maps applied to y[-1] = 0
  } else {
    if (threadIdx.x == 0) s_carry = carry[g];
  }
  // pole^(i+1) for this thread's frame: the scan of the per-frame multipliers
  Aff p = block_scan(Aff{pole, 0.f}, s_tot);
  __syncthreads();
  const int n = g * kTile + threadIdx.x;
  if (n >= frames) return;
  const float y = zs[n] + p.a * s_carry;
  out[n] = isfinite(y) ? y : 0.f;
}

// ---- streaming bank: one wave, state carried between runs -----------------
// The frame loop of the reference's C backend, one block of 64 frames at a
// time: lane k (< n_osc) steps oscillator k's phase through the block (the
// stateful u_phasor, or the deterministic phase of the frame index within
// this run), lane i (< 64) sums frame i's oscillators in order, and the
// one-pole runs frame by frame on every lane (the value is uniform; lane i
// keeps frame i's).  The state cell holds the phases and y[n-1] across runs,
// so any split of a run into runs gives the same samples.
constexpr int kStreamBlk = 64;
constexpr int kStreamMaxOsc = 64;

__device__ __forceinline__ float stream_phasor_wrap(float next) {
  const float w = next - floorf(next);
  return w >= 1.0f ? w - 1.0f : w;
}

__global__ __launch_bounds__(64) void k_stream_osc(const float* __restrict__ freqs, const float* __restrict__ amps,
                                                   float* __restrict__ out, int nosc, int frames,
                                                   float* __restrict__ state, int stateful, float sr, float pole,
                                                   int reset) {
  __shared__ float s_ph[kStreamBlk][kStreamMaxOsc + 1];
  __shared__ float s_amp[kStreamMaxOsc];
  __shared__ float s_x[kStreamBlk];
  const int lane = threadIdx.x;
  const bool osc = lane < nosc;
  const float inc = osc ? freqs[lane] / sr : 0.f;  // phaseIncrement = freq / sampleRate
  if (osc) s_amp[lane] = amps[lane];
  float ph = (osc && stateful && !reset) ? state[lane] : 0.f;
  float y = reset ? 0.f : state[nosc];
  for (int f0 = 0; f0 < frames; f0 += kStreamBlk) {
    const int nb = min(kStreamBlk, frames - f0);
    if (osc) {
      if (stateful) {
        for (int i = 0; i < nb; ++i) {
          s_ph[i][lane] = ph;  // pre-increment output
          ph = stream_phasor_wrap(ph + inc);
        }
      } else {
        for (int i = 0; i < nb; ++i) {
          const float r = inc * (float)(f0 + i);
          s_ph[i][lane] = r - floorf(r);
        }
      }
    }
    wave_sync();
    if (lane < nb) {
      float x = 0.f;
      for (int k = 0; k < nosc; ++k) x = x + sin_2pif_hw(s_ph[lane][k]) * s_amp[k];
      s_x[lane] = x;
    }
    wave_sync();
    float mine = 0.f;
    for (int i = 0; i < nb; ++i) {
      y = s_x[i] + pole * y;
      if (i == lane) mine = y;
    }
    if (lane < nb) out[f0 + lane] = isfinite(mine) ? mine : 0.f;
    wave_sync();
  }
  if (osc && stateful) state[lane] = ph;
  if (lane == 0) state[nosc] = y;
}

int launch_stream_osc_bank(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=freqs [1]=amps [2]=out [3]=n_osc (<= 64) [4]=frames (capacity) [5]=state (n_osc + 1)
  //      [6]=stateful (0: deterministic phasor, frame index from 0 in every run; 1: u_phasor state)
  // farg: [0]=sample rate [1]=pole
  const int64_t fr = op.arg[0], am = op.arg[1], out = op.arg[2], nosc = op.arg[3], frames = op.arg[4],
                st = op.arg[5], stateful = op.arg[6];
  DGEN_REQUIRE(nosc > 0 && nosc <= kStreamMaxOsc && frames > 0 && frames <= (1 << 28) && (stateful == 0 || stateful == 1),
               "stream_osc_bank: n_osc %lld frames %lld stateful %lld", (long long)nosc, (long long)frames,
               (long long)stateful);
  DGEN_REQUIRE(op.farg[0] > 0.f && op.farg[0] < 1e30f, "stream_osc_bank: sample rate %g", (double)op.farg[0]);
  DGEN_CHECK_CELL(L, fr, nosc, "stream_osc_bank.freqs");
  DGEN_CHECK_CELL(L, am, nosc, "stream_osc_bank.amps");
  DGEN_CHECK_CELL(L, out, frames, "stream_osc_bank.out");
  DGEN_CHECK_CELL(L, st, nosc + 1, "stream_osc_bank.state");
  if (L.dry) return 0;
  const int64_t n = std::min<int64_t>(frames, L.frames ? (int64_t)L.frames : frames);
  hipLaunchKernelGGL(k_stream_osc, dim3(1), dim3(64), 0, L.stream, cell(L, fr), cell(L, am), cell(L, out), (int)nosc,
                     (int)n, cell(L, st), (int)stateful, host_rate(L, op.farg[0]), op.farg[1], L.reset ? 1 : 0);
  DGEN_LAUNCH_CHECK("k_stream_osc");
  return 0;
}

int launch_osc_bank(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=freqs [1]=amps [2]=out [3]=n_osc [4]=frames [5]=workspace
  //      (frames + 1 + 3*tiles floats, tiles = ceil(frames/256), even cell)
  const int64_t fr = op.arg[0], am = op.arg[1], out = op.arg[2], nosc = op.arg[3], frames = op.arg[4],
                ws = op.arg[5];
  DGEN_REQUIRE(nosc > 0 && nosc <= 65536 && frames > 0 && frames <= (1 << 28),
               "osc_bank: n_osc %lld frames %lld", (long long)nosc, (long long)frames);
  const int64_t tiles_cap = (frames + kTile - 1) / kTile;
  DGEN_CHECK_CELL(L, fr, nosc, "osc_bank.freqs");
  DGEN_CHECK_CELL(L, am, nosc, "osc_bank.amps");
  DGEN_CHECK_CELL(L, out, frames, "osc_bank.out");
  DGEN_CHECK_CELL(L, ws, frames + 1 + 3 * tiles_cap, "osc_bank.workspace");
  DGEN_REQUIRE(ws % 2 == 0, "osc_bank: workspace cell must be 8-byte aligned");
  if (L.dry) return 0;
  // a run of frame_count frames computes the first frame_count outputs
  const int64_t n = std::min<int64_t>(frames, L.frames ? (int64_t)L.frames : frames);
  const int64_t tiles = (n + kTile - 1) / kTile;
  float* zs = cell(L, ws);
  float2* tl = reinterpret_cast<float2*>(cell(L, ws) + ((frames + 1) & ~int64_t(1)));
  float* carry = reinterpret_cast<float*>(tl + tiles_cap);
  const float sr = host_rate(L, op.farg[0]), pole = op.farg[1];
  hipLaunchKernelGGL(k_osc_tiles, dim3((unsigned)tiles), dim3(kTile), 0, L.stream, cell(L, fr), cell(L, am),
                     (int)nosc, sr, (int)n, pole, zs, tl);
  DGEN_LAUNCH_CHECK("k_osc_tiles");
  if (tiles <= kMaxFusedTiles) {
    hipLaunchKernelGGL(k_osc_apply<true>, dim3((unsigned)tiles), dim3(kTile), 0, L.stream, zs, tl, nullptr, (int)n,
                       pole, cell(L, out));
  } else {
    hipLaunchKernelGGL(k_osc_carries, dim3(1), dim3(kTile), 0, L.stream, tl, carry, (int)tiles);
    DGEN_LAUNCH_CHECK("k_osc_carries");
    hipLaunchKernelGGL(k_osc_apply<false>, dim3((unsigned)tiles), dim3(kTile), 0, L.stream, zs, tl, carry, (int)n,
                       pole, cell(L, out));
  }
  DGEN_LAUNCH_CHECK("k_osc_apply");
  return 0;
}

}  // namespace dgen
