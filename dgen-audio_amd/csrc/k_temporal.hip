// Temporal gradient of stateful accumulators (phasor, accum) and the
// swept-phasor bank that exercises it.
//
// Reference: temporalIncrementGradient (Sources/DGen/Gradients.swift:209-261)
// emits three phases (Sources/DGen/Emit+TemporalGradient.swift:15-105): store
// the output gradient and the reset flag per frame, a static reverse scan per
// element (one thread each, over all frames), then a frame-parallel read
// divided by the sample rate for a phasor.  The scan is the reset-aware
// exclusive suffix sum
//   active = reset[n] > 0 ? 0 : carry;  out[n] = active;  carry = g[n] + active
// run from the last frame down.
//
// Here the scan is parallel in time too: it is an affine recurrence in the
// carry, so frames are cut into chunks of kChunk:
//   k_tg_chunk  per (element, chunk): the chunk run from a zero carry; its map
//               carry_out = alpha * carry_in + gamma (alpha = 0 when the
//               chunk holds a reset, else 1)
//   k_tg_carry  per element: the maps composed from the last chunk down ->
//               the carry entering every chunk
//   k_tg_apply  per (element, chunk): the chunk re-run from its carry in the
//               reference's order, writing out[n] (/ sample rate)
// Only the carries between chunks are reassociated.  g, out: [T][E] (a
// wave reads 64 consecutive elements of one frame); reset: [T].
#pragma clang fp contract(off)

#include "internal.h"

namespace dgen {
namespace {

constexpr int kChunk = 256;   // frames per scan chunk
constexpr float kTwoPi = 2.0f * 3.14159265358979323846f;
constexpr int kThreads = 256;

__device__ __forceinline__ bool is_reset(const float* __restrict__ reset, int n) {
  return reset && reset[n] > 0.0f;
}

__global__ __launch_bounds__(kThreads) void k_tg_chunk(const float* __restrict__ g, const float* __restrict__ reset,
                                                       float* __restrict__ gamma, float* __restrict__ alpha, int E,
                                                       int T) {
  const int e = blockIdx.x * kThreads + threadIdx.x, c = blockIdx.y;
  const int n0 = c * kChunk, n1 = min(T, n0 + kChunk);
  float carry = 0.0f;
  bool cut = false;
  for (int n = n1 - 1; n >= n0; --n) {
    const bool rs = is_reset(reset, n);
    cut |= rs;
    const float active = rs ? 0.0f : carry;
    if (e < E) carry = g[(size_t)n * E + e] + active;
  }
  if (e < E) gamma[(size_t)c * E + e] = carry;
  if (e == 0) alpha[c] = cut ? 0.0f : 1.0f;
}

__global__ __launch_bounds__(kThreads) void k_tg_carry(const float* __restrict__ gamma, const float* __restrict__ alpha,
                                                       float* __restrict__ carry_in, int E, int C) {
  const int e = blockIdx.x * kThreads + threadIdx.x;
  if (e >= E) return;
  float k = 0.0f;  // nothing follows the last frame
  for (int c = C - 1; c >= 0; --c) {
    carry_in[(size_t)c * E + e] = k;
    k = alpha[c] * k + gamma[(size_t)c * E + e];
  }
}

__global__ __launch_bounds__(kThreads) void k_tg_apply(const float* __restrict__ g, const float* __restrict__ reset,
                                                       const float* __restrict__ carry_in, float* __restrict__ out,
                                                       int E, int T, float sr, int scale) {
  const int e = blockIdx.x * kThreads + threadIdx.x, c = blockIdx.y;
  if (e >= E) return;
  const int n0 = c * kChunk, n1 = min(T, n0 + kChunk);
  float carry = carry_in[(size_t)c * E + e];
  for (int n = n1 - 1; n >= n0; --n) {
    const float active = is_reset(reset, n) ? 0.0f : carry;
    out[(size_t)n * E + e] = scale ? active / sr : active;
    carry = g[(size_t)n * E + e] + active;
  }
}

// The swept-phasor bank (Tests/DGenLazyTests/TemporalGradientTests.swift:
// 24-60), one lane per thread: f = base + slope[e] * time[n], the stateful
// phasor of f with reset (u_phasor / u_accum order, Definitions.swift:
// 96-102, 215-246; output = the state before the frame's update), and the
// mse loss against `target` of the phase, or with `smooth` of sin(2 pi
// phase) (continuous across the phase's wraps): per-lane loss sums and the
// upstream gradient of every frame.
__global__ __launch_bounds__(kThreads) void k_swept_phasor(const float* __restrict__ slope,
                                                           const float* __restrict__ time,
                                                           const float* __restrict__ reset, float* __restrict__ phase,
                                                           float* __restrict__ gout, float* __restrict__ lossp, int E,
                                                           int T, float sr, float base, float target, int smooth) {
  const int e = blockIdx.x * kThreads + threadIdx.x;
  if (e >= E) return;
  const float s = slope[e];
  float ph = 0.0f;
  // fp64 loss sum: in fp32, small terms added to a running sum near 2e4
  // (ulp 2e-3) round the same way every frame and bias the loss
  double ls = 0.0;
  for (int n = 0; n < T; ++n) {
    const bool rs = is_reset(reset, n);
    const float f = base + s * time[n];
    const float acc = ph;
    const float next = rs ? 0.0f : acc + f / sr;
    float w = next - floorf(next);
    if (w >= 1.0f) w = w - 1.0f;
    ph = rs ? 0.0f : w;
    // sin / cos of 2 pi acc: the transcendental unit takes revolutions
    const float v = smooth ? sin_2pif_hw(acc) : acc;
    const float d = v - target;
    ls = ls + (double)(d * d);
    if (phase) phase[(size_t)n * E + e] = acc;
    gout[(size_t)n * E + e] = smooth ? 2.0f * d * (cos_2pif_hw(acc) * kTwoPi) : 2.0f * d;
  }
  lossp[e] = (float)ls;
}

}  // namespace

int launch_temporal_grad_scan(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=g ([T][E]) [1]=reset ([T]) or -1 [2]=out ([T][E]) [3]=E [4]=T [5]=workspace
  //      (2*C*E + C floats, C = ceil(T/256)) [6]=divide by the sample rate (phasor: 1)
  // farg: [0]=sample rate
  const int64_t g = op.arg[0], rs = op.arg[1], out = op.arg[2], E = op.arg[3], T = op.arg[4], ws = op.arg[5],
                scale = op.arg[6];
  DGEN_REQUIRE(E > 0 && E <= (1 << 24) && T > 0 && T < (1ll << 30) && E * T < (1ll << 40) &&
                   (scale == 0 || scale == 1),
               "temporal_grad_scan: E %lld T %lld scale %lld", (long long)E, (long long)T, (long long)scale);
  DGEN_REQUIRE(!scale || (op.farg[0] > 0.f && op.farg[0] < 1e30f), "temporal_grad_scan: sample rate %g",
               (double)op.farg[0]);
  const int64_t C = (T + kChunk - 1) / kChunk;
  DGEN_REQUIRE(C <= 65535, "temporal_grad_scan: %lld chunks", (long long)C);
  DGEN_CHECK_CELL(L, g, E * T, "temporal_grad_scan.g");
  if (rs >= 0) DGEN_CHECK_CELL(L, rs, T, "temporal_grad_scan.reset");
  DGEN_CHECK_CELL(L, out, E * T, "temporal_grad_scan.out");
  DGEN_CHECK_CELL(L, ws, 2 * C * E + C, "temporal_grad_scan.workspace");
  if (L.dry) return 0;
  float* gamma = cell(L, ws);
  float* kin = gamma + C * E;
  float* alpha = kin + C * E;
  const float* r = rs >= 0 ? cell(L, rs) : nullptr;
  const unsigned eb = (unsigned)((E + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(k_tg_chunk, dim3(eb, (unsigned)C), dim3(kThreads), 0, L.stream, cell(L, g), r, gamma, alpha,
                     (int)E, (int)T);
  DGEN_LAUNCH_CHECK("k_tg_chunk");
  hipLaunchKernelGGL(k_tg_carry, dim3(eb), dim3(kThreads), 0, L.stream, gamma, alpha, kin, (int)E, (int)C);
  DGEN_LAUNCH_CHECK("k_tg_carry");
  hipLaunchKernelGGL(k_tg_apply, dim3(eb, (unsigned)C), dim3(kThreads), 0, L.stream, cell(L, g), r, kin,
                     cell(L, out), (int)E, (int)T, host_rate(L, op.farg[0]), (int)scale);
  DGEN_LAUNCH_CHECK("k_tg_apply");
  return 0;
}

int launch_swept_phasor(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=slope ([E]) [1]=time ([T]) [2]=reset ([T]) or -1 [3]=phase ([T][E]) or -1 [4]=upstream ([T][E])
  //      [5]=loss partials ([E]) [6]=E [7]=T [8]=smooth (loss on sin(2 pi phase))
  // farg: [0]=sample rate [1]=base frequency [2]=target
  const int64_t sl = op.arg[0], tm = op.arg[1], rs = op.arg[2], ph = op.arg[3], gu = op.arg[4], lp = op.arg[5],
                E = op.arg[6], T = op.arg[7], smooth = op.arg[8];
  DGEN_REQUIRE(E > 0 && E <= (1 << 24) && T > 0 && T < (1ll << 30) && E * T < (1ll << 40),
               "swept_phasor: E %lld T %lld", (long long)E, (long long)T);
  DGEN_REQUIRE(op.farg[0] > 0.f && op.farg[0] < 1e30f, "swept_phasor: sample rate %g", (double)op.farg[0]);
  DGEN_CHECK_CELL(L, sl, E, "swept_phasor.slope");
  DGEN_CHECK_CELL(L, tm, T, "swept_phasor.time");
  if (rs >= 0) DGEN_CHECK_CELL(L, rs, T, "swept_phasor.reset");
  if (ph >= 0) DGEN_CHECK_CELL(L, ph, E * T, "swept_phasor.phase");
  DGEN_CHECK_CELL(L, gu, E * T, "swept_phasor.upstream");
  DGEN_CHECK_CELL(L, lp, E, "swept_phasor.loss_partials");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_swept_phasor, dim3((unsigned)((E + kThreads - 1) / kThreads)), dim3(kThreads), 0, L.stream,
                     cell(L, sl), cell(L, tm), rs >= 0 ? cell(L, rs) : nullptr, ph >= 0 ? cell(L, ph) : nullptr,
                     cell(L, gu), cell(L, lp), (int)E, (int)T, host_rate(L, op.farg[0]), op.farg[1], op.farg[2],
                     smooth ? 1 : 0);
  DGEN_LAUNCH_CHECK("k_swept_phasor");
  return 0;
}

}  // namespace dgen
