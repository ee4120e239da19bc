// Internal interface between the runtime (runtime.cpp) and the kernel
// families (*.hip).  Each kernel class has one launcher that validates its
// operands against the arena and, unless `dry`, enqueues its kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>

#include "../../include/dgen_hip.h"

namespace dgen {

// A generic UOp block as loaded for a context (uop_render.cpp renders it,
// the runtime compiles and loads it): the kernel and what its launch needs.
struct BlockInfo {
  hipFunction_t fn = nullptr;
  int dispatch = 0, n = 0, frame_order = 0;
  int64_t max_cell = -1;  // largest cell addressed directly
};

struct Launch {
  hipStream_t stream = nullptr;
  float* arena = nullptr;       // device arena base
  uint64_t arena_floats = 0;    // arena size in floats
  uint32_t frames = 0;          // frame_count of this run
  int device = 0;
  int cu_count = 256;
  bool dry = false;             // validate only
  float host_sr = 0.f;          // host sample rate of this run; 0: each op's own
  bool reset = false;           // streaming classes start from zero state (else the state cells)
  const BlockInfo* blocks = nullptr;  // the context's generic UOp blocks
  size_t n_blocks = 0;
};

// Sample rate a phase increment divides by: the run's host sample rate when
// one is set (u_phasor divides by hostSampleRate, Definitions.swift:96-102,
// which the C backend takes from DGenProcessContextV1.sample_rate), else the
// rate the op was rendered with.
inline float host_rate(const Launch& L, float rendered) { return L.host_sr > 0.f ? L.host_sr : rendered; }

// Thread-local last-error text; returns `code` for tail calls.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Cell-range check: [off, off+n) inside the arena and off >= 0.
int check_cell(const Launch& L, int64_t off, uint64_t n, const char* what);
inline float* cell(const Launch& L, int64_t off) { return L.arena + off; }

#define DGEN_CHECK_CELL(L, off, n, what)                      \
  do {                                                        \
    int _rc = ::dgen::check_cell((L), (off), (uint64_t)(n), (what)); \
    if (_rc) return _rc;                                      \
  } while (0)

#define DGEN_REQUIRE(cond, ...)                                  \
  do {                                                           \
    if (!(cond)) return ::dgen::fail(DGEN_HIP_E_INVALID, __VA_ARGS__); \
  } while (0)

#define DGEN_HIP_TRY(expr)                                                              \
  do {                                                                                  \
    hipError_t _e = (expr);                                                             \
    if (_e != hipSuccess)                                                               \
      return ::dgen::fail(DGEN_HIP_E_DEVICE, "%s failed: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

// Launch-error check after a kernel launch.
#define DGEN_LAUNCH_CHECK(name)                                                         \
  do {                                                                                  \
    hipError_t _e = hipGetLastError();                                                  \
    if (_e != hipSuccess)                                                               \
      return ::dgen::fail(DGEN_HIP_E_DEVICE, "launch of %s failed: %s", name, hipGetErrorString(_e)); \
  } while (0)

using Launcher = int (*)(const Launch&, const dgen_hip_op&);

// Workgroup barrier that orders LDS only: waits for the wave's own LDS
// operations, not for its outstanding global memory operations (HIP's
// __syncthreads() also waits for those, which exposes prefetch latency).
// Kernels use it only where no global-memory ordering between threads of
// the workgroup is needed.
// Spectral-loss tiles: a workgroup owns kMssTile output samples and keeps the
// gradient of [a - kMssHalo, a + kMssTile) (kMssHalo = largest N - 1); the
// tile partials are [B][ntiles][kMssAcc].  The synth backward adds them up
// per sample when it reads the prediction's gradient.
constexpr int kMssTile = 4096;
constexpr int kMssHalo = 2047;
constexpr int kMssAcc = kMssTile + kMssHalo;

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Orders one wave's LDS accesses around this point for every lane of the
// wave: a wave's LDS instructions execute in issue order, so only the
// compiler has to be kept from moving accesses across it (no hardware
// barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier, or the wave-level ordering above when every thread
// that shares the LDS data lies in the calling wave.
template <bool WAVE>
__device__ __forceinline__ void lds_sync() {
  if constexpr (WAVE) wave_sync();
  else lds_barrier();
}

// tanh within a few ulp at a fraction of the libm cost: for |x| < 0.55 the
// odd Taylor series to x^15 (truncation below 5e-8 relative; the series
// converges for |x| < pi/2), otherwise 1 - 2/(e^{2|x|} + 1) on the hardware
// exp2 and reciprocal (no cancellation there: 2/(e^{2|x|}+1) <= 0.5).
__device__ __forceinline__ float fast_tanh(float x) {
  const float ax = fabsf(x), x2 = x * x;
  float p = fmaf(x2, -929569.0f / 638512875.0f, 21844.0f / 6081075.0f);
  p = fmaf(x2, p, -1382.0f / 155925.0f);
  p = fmaf(x2, p, 62.0f / 2835.0f);
  p = fmaf(x2, p, -17.0f / 315.0f);
  p = fmaf(x2, p, 2.0f / 15.0f);
  p = fmaf(x2, p, -1.0f / 3.0f);
  const float small = fmaf(x * x2, p, x);
  const float e = __builtin_amdgcn_exp2f(ax * 2.8853900817779268f);  // e^{2|x|}
  const float big = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
  return ax < 0.55f ? small : copysignf(big, x);
}

int launch_accum_table(const Launch&, const dgen_hip_op&);
int launch_dense_small(const Launch&, const dgen_hip_op&);
int launch_dense_small_wgrad(const Launch&, const dgen_hip_op&);
int launch_gemm(const Launch&, const dgen_hip_op&);
int launch_split_bf16(const Launch&, const dgen_hip_op&);
int launch_colsum(const Launch&, const dgen_hip_op&);
int launch_heads_fwd(const Launch&, const dgen_hip_op&);
int launch_heads_bwd(const Launch&, const dgen_hip_op&);
int launch_phasor_carry(const Launch&, const dgen_hip_op&);
int launch_synth_fwd(const Launch&, const dgen_hip_op&);
int launch_synth_bwd(const Launch&, const dgen_hip_op&);
int launch_synth_bwd_reduce(const Launch&, const dgen_hip_op&);
int launch_spectral_loss(const Launch&, const dgen_hip_op&);
int launch_spectral_gather(const Launch&, const dgen_hip_op&);
int launch_adam(const Launch&, const dgen_hip_op&);
int launch_osc_bank(const Launch&, const dgen_hip_op&);
int launch_noise_table(const Launch&, const dgen_hip_op&);
int launch_row_schedule(const Launch&, const dgen_hip_op&);
int launch_run_table(const Launch&, const dgen_hip_op&);
int launch_fft_tables(const Launch&, const dgen_hip_op&);
int launch_lerp_frames(const Launch&, const dgen_hip_op&);
int launch_biquad_chunk(const Launch&, const dgen_hip_op&);
int launch_biquad_carry(const Launch&, const dgen_hip_op&);
int launch_biquad_fwd(const Launch&, const dgen_hip_op&);
int launch_biquad_adj_chunk(const Launch&, const dgen_hip_op&);
int launch_biquad_bwd(const Launch&, const dgen_hip_op&);
int launch_stft_fwd(const Launch&, const dgen_hip_op&);
int launch_stft_bwd(const Launch&, const dgen_hip_op&);
int launch_membrane_fwd(const Launch&, const dgen_hip_op&);
int launch_membrane_bwd(const Launch&, const dgen_hip_op&);
int launch_stream_osc_bank(const Launch&, const dgen_hip_op&);
int launch_stream_biquad(const Launch&, const dgen_hip_op&);
int launch_temporal_grad_scan(const Launch&, const dgen_hip_op&);
int launch_swept_phasor(const Launch&, const dgen_hip_op&);
int launch_svf_chunk(const Launch&, const dgen_hip_op&);
int launch_svf_fwd(const Launch&, const dgen_hip_op&);
int launch_svf_seq(const Launch&, const dgen_hip_op&);
int launch_svf_adj_chunk(const Launch&, const dgen_hip_op&);
int launch_svf_bwd(const Launch&, const dgen_hip_op&);

// Generic UOp blocks (uop_render.cpp): the HIP C++ source of a block list,
// and the largest cell a block addresses directly (-1: none).
}  // namespace dgen
#include <string>
namespace dgen {
int render_blocks(const dgen_hip_block* blocks, uint32_t n, std::string& source);
int64_t block_max_cell(const dgen_hip_block& b);
int launch_uop_block(const Launch&, const dgen_hip_op&);

// (segment, slot) entries listed per control row by the static row schedule
// (a row is read by at most this many synth segments: 3 at a control hop of
// 64 frames, ~9 at 256).
constexpr int kRowEntries = 16;

// Sum over the 64 lanes of a wave (butterfly; every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
// sin and cos of the reference's expression phase * 2pi_f32: the graphs
// multiply a phase in revolutions by the fp32 constant 2pi_f32 =
// 6.28318548... (2pi (1 + 2.78e-8)) and take sinf of the product
// (CRenderer.swift:825-827).  The hardware units take revolutions and
// evaluate sin(2 pi p), a function whose phase runs 2.78e-8 slow: a
// systematic, phase-proportional error (up to 1.75e-7 rad) that puts
// coherent error lines into the spectrum, where a random rounding error of
// the same size would not.  The forms below evaluate the reference's
// function itself.
//
// kTwoPiF32Excess = 2pi_f32 - 2pi (rounded to fp32).
constexpr float kTwoPiF32Excess = 0x1.777a5cp-23f;
// sin(p * 2pi_f32) for p in [0, 1) on the hardware units, to their
// accuracy (max abs error 1.4e-7 against the exact value over a 2^24-point
// grid): sin(2 pi p + e p) ~ sin(2 pi p) + e p cos(2 pi p), e the
// constant's excess.  Two transcendental operations and one FMA.
__device__ __forceinline__ float sin_2pif_hw(float p) {
  return fmaf(p * kTwoPiF32Excess, __builtin_amdgcn_cosf(p), __builtin_amdgcn_sinf(p));
}
// cos(p * 2pi_f32) likewise: cos(2 pi p) - e p sin(2 pi p).
__device__ __forceinline__ float cos_2pif_hw(float p) {
  return fmaf(-p * kTwoPiF32Excess, __builtin_amdgcn_sinf(p), __builtin_amdgcn_cosf(p));
}

// e^x and ln x on the hardware exp2 / log2 (v_exp_f32, v_log_f32, ~1 ulp);
// the argument scaling adds ~|x| 6e-8 relative to e^x.
__device__ __forceinline__ float hw_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float hw_ln(float x) { return __builtin_amdgcn_logf(x) * 0.69314718055994531f; }
// softplus(x) = max(x,0) + log(1 + exp(-|x|))  (Model.swift:153-157)
__device__ __forceinline__ float softplus(float x) { return fmaxf(x, 0.f) + hw_ln(1.f + hw_exp(-fabsf(x))); }
// d softplus through the reference AD rules: [x>=0] - sign(x) e^{-|x|}/(1+e^{-|x|})
__device__ __forceinline__ float softplus_grad(float x) {
  const float e = hw_exp(-fabsf(x));
  const float sg = x > 0.f ? 1.f : (x < 0.f ? -1.f : 0.f);
  return (x >= 0.f ? 1.f : 0.f) - sg * (e * __builtin_amdgcn_rcpf(1.f + e));
}

}  // namespace dgen
