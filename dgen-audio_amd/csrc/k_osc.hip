// Deterministic phasor bank -> sum -> one-pole history (config 1).
//
// Signal.phasor(Tensor) lowers to the stateless deterministicPhasor
// (Sources/DGenLazy/SignalTensor.swift:67-80, Sources/DGen/Emit+State.swift:
// 370-387): phase = r - floor(r), r = (f / sr) * n, evaluated per frame, so
// the oscillator sum is frame-parallel.  The history one-pole
// y[n] = x[n] + pole * y[n-1] (Emit+State.swift:150-224) is a linear
// recurrence; it is evaluated as a three-phase chunked scan: zero-state
// chunk ends in parallel, a short sequential pass over chunk carries, then
// every chunk re-runs its recurrence from the exact carry.  Within a chunk
// the operation order is the reference's; only the carries are re-associated.
#pragma clang fp contract(off)

#include "internal.h"

namespace dgen {

constexpr float kTwoPi = 2.0f * 3.14159265358979323846f;
constexpr int kChunk = 256;

__global__ void k_osc_sum(const float* __restrict__ freqs, const float* __restrict__ amps, int nosc, float sr,
                          int frames, float* __restrict__ x) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= frames) return;
  const float fn = (float)n;
  float acc = 0.f;
  for (int k = 0; k < nosc; ++k) {
    const float inc = freqs[k] / sr;
    const float r = inc * fn;
    const float phase = r - floorf(r);
    acc = acc + sinf(phase * kTwoPi) * amps[k];
  }
  x[n] = acc;
}

__global__ void k_onepole_ends(const float* __restrict__ x, float* __restrict__ ends, int frames, float pole) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const int n0 = c * kChunk;
  if (n0 >= frames) return;
  const int n1 = min(frames, n0 + kChunk);
  float z = 0.f;
  for (int n = n0; n < n1; ++n) z = x[n] + pole * z;
  ends[c] = z;
}

__global__ void k_onepole_carries(const float* __restrict__ ends, float* __restrict__ carry, int chunks, int frames,
                                  float pole) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  float y = 0.f;
  for (int c = 0; c < chunks; ++c) {
    carry[c] = y;  // y[n0 - 1]
    const int len = min(kChunk, frames - c * kChunk);
    float pl = 1.f;
    for (int i = 0; i < len; ++i) pl = pl * pole;
    y = ends[c] + pl * y;
  }
}

__global__ void k_onepole_apply(const float* __restrict__ x, const float* __restrict__ carry, float* __restrict__ out,
                                int frames, float pole) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const int n0 = c * kChunk;
  if (n0 >= frames) return;
  const int n1 = min(frames, n0 + kChunk);
  float y = carry[c];
  for (int n = n0; n < n1; ++n) {
    y = x[n] + pole * y;
    out[n] = isfinite(y) ? y : 0.f;
  }
}

int launch_osc_bank(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=freqs [1]=amps [2]=out [3]=n_osc [4]=frames [5]=workspace (frames + 2*chunks floats)
  const int64_t fr = op.arg[0], am = op.arg[1], out = op.arg[2], nosc = op.arg[3], frames = op.arg[4],
                ws = op.arg[5];
  DGEN_REQUIRE(nosc > 0 && nosc <= 4096 && frames > 0 && frames <= (1 << 28), "osc_bank: n_osc %lld frames %lld",
               (long long)nosc, (long long)frames);
  const int64_t chunks = (frames + kChunk - 1) / kChunk;
  DGEN_CHECK_CELL(L, fr, nosc, "osc_bank.freqs");
  DGEN_CHECK_CELL(L, am, nosc, "osc_bank.amps");
  DGEN_CHECK_CELL(L, out, frames, "osc_bank.out");
  DGEN_CHECK_CELL(L, ws, frames + 2 * chunks, "osc_bank.workspace");
  if (L.dry) return 0;
  float* x = cell(L, ws);
  float* ends = x + frames;
  float* carry = ends + chunks;
  const float sr = op.farg[0], pole = op.farg[1];
  hipLaunchKernelGGL(k_osc_sum, dim3((unsigned)((frames + 255) / 256)), dim3(256), 0, L.stream, cell(L, fr),
                     cell(L, am), (int)nosc, sr, (int)frames, x);
  DGEN_LAUNCH_CHECK("k_osc_sum");
  hipLaunchKernelGGL(k_onepole_ends, dim3((unsigned)((chunks + 63) / 64)), dim3(64), 0, L.stream, x, ends,
                     (int)frames, pole);
  DGEN_LAUNCH_CHECK("k_onepole_ends");
  hipLaunchKernelGGL(k_onepole_carries, dim3(1), dim3(64), 0, L.stream, ends, carry, (int)chunks, (int)frames, pole);
  DGEN_LAUNCH_CHECK("k_onepole_carries");
  hipLaunchKernelGGL(k_onepole_apply, dim3((unsigned)((chunks + 63) / 64)), dim3(64), 0, L.stream, x, carry,
                     cell(L, out), (int)frames, pole);
  DGEN_LAUNCH_CHECK("k_onepole_apply");
  return 0;
}

}  // namespace dgen
