// Latency probe for the phase chain's floor on this part (not part of the
// library): cycles per frame of phase = fract(phase + inc), the carry's two
// dependent VALU instructions a frame (Emit+State.swift:322-369), for one
// wave per workgroup and 32 workgroups, under what the carry kernel adds
// around it one piece at a time.
//
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       dgen-audio_amd/csrc/probe_chain.cpp -o probe_chain && ./probe_chain
//
// Modes:
//   0  increments in registers (the dependent-instruction floor)
//   1  a dependent add alone
//   2  increments streamed from LDS, 8 ds_read_b128 per half segment one
//      half ahead (the carry's straight run)
//   3  2 + a barrier every 3 segments with three producer waves writing
//      16 ds_write_b128 each per interval
//   4  3 + the phase stored to global memory at every segment start
#include <hip/hip_runtime.h>

#include <cstdio>
#include <vector>

namespace {
constexpr int kLd = 68;       // k-major row stride of the increment ring (floats)
constexpr int kBufs = 9;      // ring segments
constexpr int kFramesReg = 64000;

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));            \
      return 1;                                                               \
    }                                                                         \
  } while (0)

// modes 0 and 1: one wave, increments in registers, kFramesReg frames
template <int MODE>
__global__ __launch_bounds__(64) void k_reg(const float* in, float* out, unsigned long long* cyc) {
  float v[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) v[i] = in[i * 64 + threadIdx.x];
  float ph = 0.0f;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < kFramesReg / 64; ++it) {
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      if constexpr (MODE == 0) ph = __builtin_amdgcn_fractf(ph + v[i]);
      else ph = ph + v[i];
    }
  }
  asm volatile("" : "+v"(ph));
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  out[blockIdx.x * 64 + threadIdx.x] = ph;
  if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}

// modes 2..4: the chain wave (wave 0) steps 3 segments per interval from
// the LDS ring; waves 1..3 act as producers in modes 3 and 4
template <int MODE>
__global__ __launch_bounds__(256) void k_lds(const float* in, float* out, unsigned long long* cyc, int nint) {
  __shared__ __align__(16) float s_inc[kBufs][64 * kLd];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int i = threadIdx.x; i < kBufs * 64 * kLd; i += blockDim.x) s_inc[0][i] = in[i % 4096];
  __syncthreads();
  float ph = 0.0f;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  if (wave == 0) {
    __builtin_amdgcn_s_setprio(3);
    float va[64], vb[64];
    auto ld = [&](int s, int h, float* d) {
      asm volatile("" ::: "memory");
      const float4* src = reinterpret_cast<const float4*>(&s_inc[s % kBufs][lane * kLd]) + 8 * h;
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
      for (int i = 0; i < 32; ++i) ph = __builtin_amdgcn_fractf(ph + v[i]);
      __builtin_amdgcn_sched_barrier(0);
    };
    auto ck = [&](int s) {
      if constexpr (MODE >= 4) out[4096 + (size_t)s * 64 + lane] = ph;
    };
    ld(0, 0, va);
    ld(0, 1, va + 32);
    for (int it = 0; it < nint; ++it) {
      const int s0 = 3 * it;
      float* X = va;
      float* Y = va + 32;
      float* Z = vb;
      ck(s0);
      ld(s0 + 1, 0, Z); st(X); ld(s0 + 1, 1, X); st(Y);
      ck(s0 + 1);
      ld(s0 + 2, 0, Y); st(Z); ld(s0 + 2, 1, Z); st(X);
      ck(s0 + 2);
      ld(s0 + 3, 0, X); st(Y); ld(s0 + 3, 1, Y); st(Z);
      if constexpr (MODE >= 3) asm volatile("s_barrier" ::: "memory");
    }
  } else if constexpr (MODE >= 3) {
    float acc = (float)lane;
    for (int it = 0; it < nint; ++it) {
      // a segment two intervals ahead: never one the chain is reading
      float4* dst = reinterpret_cast<float4*>(&s_inc[(3 * it + 6 + wave - 1) % kBufs][lane * kLd]);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        dst[q] = make_float4(acc, acc * 0.5f, acc * 0.25f, acc + (float)q);
        acc = fmaf(acc, 0.999f, 1e-3f);
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    ph = acc;
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  out[blockIdx.x * 256 + threadIdx.x] = ph;
  if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}
}  // namespace

int main() {
  constexpr int G = 32, nint = 333;  // 333 intervals of 3 segments: 63936 frames
  float *in = nullptr, *out = nullptr;
  unsigned long long* cyc = nullptr;
  CHECK(hipMalloc(&in, 4096 * sizeof(float)));
  CHECK(hipMalloc(&out, (4096 + 3 * nint * 64 + G * 256) * sizeof(float)));
  CHECK(hipMalloc(&cyc, G * sizeof(unsigned long long)));
  std::vector<float> h(4096);
  for (int i = 0; i < 4096; ++i) h[i] = 0.0123f * (float)(i % 97) + 0.001f;
  CHECK(hipMemcpy(in, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
  auto report = [&](const char* name, double frames) -> int {
    unsigned long long c[G];
    CHECK(hipMemcpy(c, cyc, sizeof(c), hipMemcpyDeviceToHost));
    double m = 0;
    for (int i = 0; i < G; ++i) m += (double)c[i];
    std::printf("%-62s %6.2f cycles per frame\n", name, m / G / frames);
    return 0;
  };
  for (int rep = 0; rep < 2; ++rep) hipLaunchKernelGGL(k_reg<0>, dim3(G), dim3(64), 0, 0, in, out, cyc);
  CHECK(hipDeviceSynchronize());
  if (report("0 add+fract, increments in registers", kFramesReg)) return 1;
  for (int rep = 0; rep < 2; ++rep) hipLaunchKernelGGL(k_reg<1>, dim3(G), dim3(64), 0, 0, in, out, cyc);
  CHECK(hipDeviceSynchronize());
  if (report("1 add alone", kFramesReg)) return 1;
  for (int rep = 0; rep < 2; ++rep) hipLaunchKernelGGL(k_lds<2>, dim3(G), dim3(256), 0, 0, in, out, cyc, nint);
  CHECK(hipDeviceSynchronize());
  if (report("2 increments streamed from LDS", 192.0 * nint)) return 1;
  for (int rep = 0; rep < 2; ++rep) hipLaunchKernelGGL(k_lds<3>, dim3(G), dim3(256), 0, 0, in, out, cyc, nint);
  CHECK(hipDeviceSynchronize());
  if (report("3 + interval barriers, three LDS-writing producer waves", 192.0 * nint)) return 1;
  for (int rep = 0; rep < 2; ++rep) hipLaunchKernelGGL(k_lds<4>, dim3(G), dim3(256), 0, 0, in, out, cyc, nint);
  CHECK(hipDeviceSynchronize());
  if (report("4 + a phase store to global memory per segment", 192.0 * nint)) return 1;
  CHECK(hipFree(in));
  CHECK(hipFree(out));
  CHECK(hipFree(cyc));
  return 0;
}
