// Two-cell ZDF state-variable filter bank (low-pass) and its BPTT adjoint.
//
// Reference: the hand-rolled Cytomic/TPT SVF of the MonologueVoice filter,
// Tests/DGenLazyTests/SVFBPTTScratchTests.swift:21-34 (history cells ic1,
// ic2 with pass-through writes, saturation s = ic / (1 + |kSat ic|)), driven
// as at :56-63: fc = (fBase [* m] + envelope).clip(20, 20000),
// g = tan((pi * fc) / sr), kDamp = 1 / res.  Per lane and frame:
//   a1 = 1 / (1 + g (g + kd)), a2 = g a1, v3 = x - s2, v1 = a1 s1 + a2 v3,
//   ic1 <- 2 v1 - s1, v1p = (ic1 + s1) / 2, v2 = s2 + g v1p,
//   ic2 <- 2 v2 - s2, y = (ic2 + s2) / 2.
// The reference runs it as one sequential frame loop per lane and, for the
// gradient, a reverse loop over stored per-frame values
// (BPTTEmission.swift:133-160).
//
// Here, with kSat the constant 0 (a linear recurrence in (ic1, ic2)), time
// is parallel like the biquad bank: frames cut into chunks of L,
//   k_svf_chunk      per (lane, chunk): the chunk's zero-state result and its
//                    responses to the two unit states, in fp64 on the fp32
//                    coefficients (an affine 2x2 map per chunk)
//   DGEN_HIP_K_BIQUAD_CARRY composes the maps per lane -> every chunk's state
//   k_svf_fwd        each chunk re-run in fp32 from its state: y, the cells
//                    entering every frame, per-chunk loss partials
// With a learnable kSat the forward is not affine and runs one lane per
// thread over all frames (k_svf_seq, the reference's schedule).  The adjoint
// of the cells IS affine in both cases (its Jacobians read the stored
// cells), so the backward is always chunked:
//   k_svf_adj_chunk  per (lane, chunk), reverse: zero-carry adjoint and unit
//                    responses (fp64; for the linear bank k_svf_fwd can form
//                    them instead), then the carry kernel in reverse
//   k_svf_bwd        each chunk's adjoint replayed in fp32 from its carry,
//                    chained through the coefficient nodes to per-chunk
//                    gradient partials [C][P][B] (base, res[, kSat]) and
//                    optionally d loss / d x.
// Every frame computes in the reference graph's node order with IEEE fp32
// (no contraction), like the CPU restatement it is checked against.
//
// Layout: x, y, target [T][B]; cells [2][T][B] (ic1 plane, ic2 plane);
// params [P][B] = base | res (| kSat), P = 2 linear, 3 saturating; m and the
// envelope are per-frame signals shared by all lanes ([T], optional).
#pragma clang fp contract(off)

#include <type_traits>

#include "dev_math.h"
#include "internal.h"

namespace dgen {
namespace {

constexpr int kThreads = 256;   // lanes per workgroup of the chunked kernels
constexpr int kSeqThreads = 64;  // lanes per workgroup of the sequential forward
constexpr int kG = 8;           // frames per prefetch group
constexpr float kPi = 3.14159265358979323846f;

struct Ctl {
  const float* m;    // [T] cutoff scale or null (1)
  const float* env;  // [T] cutoff offset or null (0)
};

struct SvfK {
  float g, a1, a2, u, Q;
  bool pass;  // the clip passes the cutoff's gradient
};

// clip = max(min(v, 20000), 20) (Functions.swift:780-782); min passes its
// input's gradient where v <= hi, max where min(v, hi) >= lo
// (Gradients.swift:386-410).
__device__ __forceinline__ SvfK svf_coef(float raw, float kd, float sr, float rsr) {
  SvfK K;
  const float lo = raw <= 20000.0f ? raw : 20000.0f;
  const float fc = lo >= 20.0f ? lo : 20.0f;
  K.pass = raw <= 20000.0f && lo >= 20.0f;
  K.u = div_rn(kPi * fc, sr, rsr);
  K.g = tanf(K.u);
  K.Q = 1.0f + K.g * (K.g + kd);
  K.a1 = rcp_rn(K.Q);
  K.a2 = K.g * K.a1;
  return K;
}

__device__ __forceinline__ float raw_cutoff(float base, float m, float e, const Ctl& ctl) {
  const float v = base * m;
  return ctl.env ? v + e : v;
}

// One frame of the fp32 program: cells (c1, c2) -> next; returns y.
// (the saturation's quotients: reciprocal + one correction, like 1/Q)
template <bool SAT>
__device__ __forceinline__ float sat_div(float c, float ks) {
  if constexpr (!SAT) {
    return c;
  } else {
    const float d = 1.0f + fabsf(ks * c);
    return div_rn(c, d, rcp_rn(d));
  }
}

template <bool SAT>
__device__ __forceinline__ float svf_step(const SvfK& K, float ks, float x, float& c1, float& c2) {
  const float s1 = sat_div<SAT>(c1, ks);
  const float s2 = sat_div<SAT>(c2, ks);
  const float v3 = x - s2;
  const float v1 = K.a1 * s1 + K.a2 * v3;
  const float ic1 = 2.0f * v1 - s1;
  const float v1p = (ic1 + s1) * 0.5f;
  const float v2 = s2 + K.g * v1p;
  const float ic2 = 2.0f * v2 - s2;
  c1 = ic1;
  c2 = ic2;
  return (ic2 + s2) * 0.5f;
}

// Streams frames [n0, n1) forwards (REV: n1-1 down to n0): f(n, v, m, e)
// with v[s] = src[s][n][k], m = m[n] (1) and e = env[n] (0).  The next
// group's loads are issued before the current group is processed.
template <int NS, bool REV, class F>
__device__ __forceinline__ void walk(const float* const (&src)[NS], const Ctl& ctl, int B, int k, int n0, int n1,
                                     F&& f) {
  const int cnt = n1 - n0;
  if (cnt <= 0) return;
  auto frame = [&](int i) { return REV ? n1 - 1 - i : n0 + i; };
  float cv[kG][NS], cm[kG], ce[kG];
  auto load = [&](int i, float (&v)[kG][NS], float (&mv)[kG], float (&ev)[kG]) {
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      const int n = frame(min(i + j, cnt - 1));
#pragma unroll
      for (int s = 0; s < NS; ++s) v[j][s] = src[s][(size_t)n * B + k];
      mv[j] = ctl.m ? ctl.m[n] : 1.0f;
      ev[j] = ctl.env ? ctl.env[n] : 0.0f;
    }
  };
  load(0, cv, cm, ce);
  int i = 0;
  for (; i + kG <= cnt; i += kG) {
    float nv[kG][NS], nm[kG], ne[kG];
    load(i + kG, nv, nm, ne);
#pragma unroll
    for (int j = 0; j < kG; ++j) f(frame(i + j), cv[j], cm[j], ce[j]);
#pragma unroll
    for (int j = 0; j < kG; ++j) {
#pragma unroll
      for (int s = 0; s < NS; ++s) cv[j][s] = nv[j][s];
      cm[j] = nm[j];
      ce[j] = ne[j];
    }
  }
#pragma unroll
  for (int j = 0; j < kG; ++j)
    if (i + j < cnt) f(frame(i + j), cv[j], cm[j], ce[j]);
}

struct Lane {
  int k, c, n0, n1;
  float base, res, kd, ks, rsr;
};

__device__ __forceinline__ bool lane_chunk(const float* __restrict__ prm, int B, int T, int L, float sr, bool sat,
                                           Lane& l) {
  l.k = blockIdx.y * kThreads + threadIdx.x;
  if (l.k >= B) return false;
  l.c = blockIdx.x;
  l.n0 = l.c * L;
  l.n1 = min(T, l.n0 + L);
  l.base = prm[l.k];
  l.res = prm[B + l.k];
  l.kd = 1.0f / l.res;
  l.ks = sat ? prm[2 * B + l.k] : 0.0f;
  l.rsr = rcp_rn(sr);
  return true;
}

// ------------------------------------------------------------ forward scan
__global__ __launch_bounds__(kThreads) void k_svf_chunk(const float* __restrict__ x, Ctl ctl,
                                                        const float* __restrict__ prm, double* __restrict__ summ,
                                                        int B, int T, int L, float sr) {
  Lane l;
  if (!lane_chunk(prm, B, T, L, sr, false, l)) return;
  double p1 = 0.0, p2 = 0.0, u1 = 1.0, u2 = 0.0, w1 = 0.0, w2 = 1.0;
  auto adv = [](double a1, double a2, double g, double xx, double& c1, double& c2) {
    const double v3 = xx - c2;
    const double v1 = a1 * c1 + a2 * v3;
    const double ic1 = 2.0 * v1 - c1;
    const double v1p = (ic1 + c1) * 0.5;
    const double v2 = c2 + g * v1p;
    c1 = ic1;
    c2 = 2.0 * v2 - c2;
  };
  const float* const src[1] = {x};
  walk<1, false>(src, ctl, B, l.k, l.n0, l.n1, [&](int, const float* v, float m, float e) {
    const SvfK K = svf_coef(raw_cutoff(l.base, m, e, ctl), l.kd, sr, l.rsr);
    const double a1 = K.a1, a2 = K.a2, g = K.g;
    adv(a1, a2, g, v[0], p1, p2);
    adv(a1, a2, g, 0.0, u1, u2);
    adv(a1, a2, g, 0.0, w1, w2);
  });
  double* o = summ + (size_t)l.c * 6 * B + l.k;
  o[0] = p1;
  o[(size_t)B] = p2;
  o[(size_t)2 * B] = u1;
  o[(size_t)3 * B] = u2;
  o[(size_t)4 * B] = w1;
  o[(size_t)5 * B] = w2;
}

// ADJ (with LOSS): the chunk's adjoint summary as well, the map that
// k_svf_adj_chunk<false> forms running backwards, accumulated forwards here.
// With kSat = 0 one frame takes the cells' adjoint (l1, l2) to A_n (l1, l2)
// + b_n e_n, e_n = 2 (y_n - tgt_n), where (from the reverse of svf_step)
// A_n = [[2 a1 - 1, 2 a1 g], [-2 a2, 1 - 2 a2 g]] and b_n = (a1 g, 1 - a2 g).
// Over frames n0..n1-1 (taken from n1-1 down) the state leaving is M l + z
// with M = A_n0 ... A_n1-1 and z = sum_n P_n b_n e_n, P_n = A_n0 ... A_n-1:
// prefix products, carried in fp64.  Summary [6][B] = (z, M e1, M e2).
template <bool LOSS, bool ADJ = false>
__global__ __launch_bounds__(kThreads) void k_svf_fwd(const float* __restrict__ x, Ctl ctl,
                                                      const float* __restrict__ prm, const float* __restrict__ init,
                                                      float* __restrict__ y, float* __restrict__ cells,
                                                      const float* __restrict__ tgt, float* __restrict__ lossp, int B,
                                                      int T, int L, float sr, double* __restrict__ asumm) {
  static_assert(!ADJ || LOSS, "the adjoint summary needs the target");
  Lane l;
  if (!lane_chunk(prm, B, T, L, sr, false, l)) return;
  const int k = l.k;
  float c1 = init[(size_t)l.c * 2 * B + k], c2 = init[((size_t)l.c * 2 + 1) * B + k];
  float ls = 0.0f;
  double p11 = 1.0, p12 = 0.0, p21 = 0.0, p22 = 1.0, z1 = 0.0, z2 = 0.0;
  const size_t plane = (size_t)T * B;
  auto step = [&](int n, const float* v, float m, float e) {
    const SvfK K = svf_coef(raw_cutoff(l.base, m, e, ctl), l.kd, sr, l.rsr);
    const size_t i = (size_t)n * B + k;
    if (cells) {
      cells[i] = c1;
      cells[plane + i] = c2;
    }
    const float out = svf_step<false>(K, 0.0f, v[0], c1, c2);
    y[i] = out;
    if constexpr (LOSS) {
      const float d = out - v[1];
      ls += d * d;
    }
    if constexpr (ADJ) {
      const double a1 = K.a1, a2 = K.a2, g = K.g;
      const double ee = 2.0 * ((double)out - (double)v[1]);
      const double b1 = a1 * g, b2 = 1.0 - a2 * g;
      z1 += ee * (p11 * b1 + p12 * b2);
      z2 += ee * (p21 * b1 + p22 * b2);
      const double A11 = 2.0 * a1 - 1.0, A12 = 2.0 * a1 * g, A21 = -2.0 * a2, A22 = 1.0 - 2.0 * a2 * g;
      const double n11 = p11 * A11 + p12 * A21, n12 = p11 * A12 + p12 * A22;
      const double n21 = p21 * A11 + p22 * A21, n22 = p21 * A12 + p22 * A22;
      p11 = n11;
      p12 = n12;
      p21 = n21;
      p22 = n22;
    }
  };
  if constexpr (LOSS) {
    const float* const src[2] = {x, tgt};
    walk<2, false>(src, ctl, B, k, l.n0, l.n1, step);
    lossp[(size_t)l.c * B + k] = ls;
    if constexpr (ADJ) {
      double* o = asumm + (size_t)l.c * 6 * B + k;
      o[0] = z1;
      o[(size_t)B] = z2;
      o[(size_t)2 * B] = p11;
      o[(size_t)3 * B] = p21;
      o[(size_t)4 * B] = p12;
      o[(size_t)5 * B] = p22;
    }
  } else {
    const float* const src[1] = {x};
    walk<1, false>(src, ctl, B, k, l.n0, l.n1, step);
  }
}

// g = tan(pi fc / sr) of every (frame, lane) into a tape [T][B]: it does not
// depend on the cells, so the saturating forward's sequential loop reads it
// instead of evaluating tan (a1 and a2 follow from g in a few operations off
// the loop's dependency chain).  One load per frame: the sequential loop is
// bound by its outstanding memory operations, not by arithmetic.
__global__ __launch_bounds__(kThreads) void k_svf_coef(Ctl ctl, const float* __restrict__ prm,
                                                       float* __restrict__ tape, int B, int T, int L, float sr) {
  Lane l;
  if (!lane_chunk(prm, B, T, L, sr, false, l)) return;
  for (int n = l.n0; n < l.n1; ++n) {
    const SvfK K = svf_coef(raw_cutoff(l.base, ctl.m ? ctl.m[n] : 1.0f, ctl.env ? ctl.env[n] : 0.0f, ctl), l.kd,
                            sr, l.rsr);
    tape[(size_t)n * B + l.k] = K.g;
  }
}

// Saturating forward: one lane per thread over all frames, from the state
// cell ([2][B], or zero) and back into it; loss partials per L-frame chunk.
// TAPE: coefficients from k_svf_coef's tape, else evaluated in the loop.
// sanitize: out stores map non-finite values to 0 (CRenderer.swift:1021-1039).
template <bool LOSS, bool TAPE>
__global__ __launch_bounds__(kSeqThreads) void k_svf_seq(const float* __restrict__ x, Ctl ctl,
                                                         const float* __restrict__ prm, const float* __restrict__ tape,
                                                         float* __restrict__ state, int reset, float* __restrict__ y,
                                                         float* __restrict__ cells, const float* __restrict__ tgt,
                                                         float* __restrict__ lossp, int B, int T, int L, float sr,
                                                         int sanitize) {
  const int k = blockIdx.x * kSeqThreads + threadIdx.x;
  if (k >= B) return;
  const float base = prm[k], kd = 1.0f / prm[B + k], ks = prm[2 * B + k], rsr = rcp_rn(sr);
  float c1 = 0.0f, c2 = 0.0f;
  if (state && !reset) {
    c1 = state[k];
    c2 = state[B + k];
  }
  const size_t plane = (size_t)T * B;
  const int C = (T + L - 1) / L;
  constexpr int NS = 1 + (LOSS ? 1 : 0) + (TAPE ? 1 : 0);
  const float* src[NS];
  src[0] = x;
  if constexpr (LOSS) src[1] = tgt;
  if constexpr (TAPE) src[NS - 1] = tape;
  const float* const(&csrc)[NS] = src;
  const Ctl none{nullptr, nullptr};
  for (int c = 0; c < C; ++c) {
    float ls = 0.0f;
    auto step = [&](int n, const float* v, float m, float e) {
      SvfK K;
      if constexpr (TAPE) {
        K.g = v[NS - 1];
        K.Q = 1.0f + K.g * (K.g + kd);
        K.a1 = rcp_rn(K.Q);
        K.a2 = K.g * K.a1;
      } else {
        K = svf_coef(raw_cutoff(base, m, e, ctl), kd, sr, rsr);
      }
      const size_t i = (size_t)n * B + k;
      if (cells) {
        cells[i] = c1;
        cells[plane + i] = c2;
      }
      const float out = svf_step<true>(K, ks, v[0], c1, c2);
      y[i] = sanitize && !isfinite(out) ? 0.0f : out;
      if constexpr (LOSS) {
        const float d = out - v[1];
        ls += d * d;
      }
    };
    const int n0 = c * L, n1 = min(T, n0 + L);
    walk<NS, false>(csrc, TAPE ? none : ctl, B, k, n0, n1, step);
    if constexpr (LOSS) lossp[(size_t)c * B + k] = ls;
  }
  if (state) {
    state[k] = c1;
    state[B + k] = c2;
  }
}

// The saturating forward of a training step, staged through LDS.  Each
// wave's 64 lanes step 32-frame tiles: a tile's x, target and coefficient
// rows arrive by 16-byte load-to-LDS copies issued one tile ahead (each
// instruction brings four frames of the wave's 64 lanes), the frame loop
// reads and writes only LDS, and the tile's cells and y leave as 16-byte
// stores.  Per frame the wave issues a fraction of one global memory
// instruction instead of six, so the loop is bound by its own dependent
// chain instead of by outstanding memory operations.  The arithmetic is
// k_svf_seq's (tape coefficients, the saturating step, loss partials per
// L frames), so the results are the same bit for bit.  Needs B a multiple
// of 64 and T and L multiples of 32.
constexpr int kTileF = 32;
__global__ __launch_bounds__(64) void k_svf_seq_tiled(const float* __restrict__ x, const float* __restrict__ prm,
                                                      const float* __restrict__ tape, float* __restrict__ state,
                                                      float* __restrict__ y, float* __restrict__ cells,
                                                      const float* __restrict__ tgt, float* __restrict__ lossp, int B,
                                                      int T, int L, int sanitize) {
  // inputs, double buffered: [array: x, target, g][frame][lane]; outputs
  // [array: c1, c2, y][frame][lane].  (Reading a1 and a2 from two more tape
  // planes instead of computing them from g measured no faster: the loop is
  // bound by the latency of its ~23 dependent operations per frame.)
  constexpr int NI = 3;
  __shared__ __align__(16) float in0[NI][kTileF][64];
  __shared__ __align__(16) float in1[NI][kTileF][64];
  __shared__ __align__(16) float out[3][kTileF][64];
  const int lane = threadIdx.x, k0 = blockIdx.x * 64, k = k0 + lane;
  const float kd = 1.0f / prm[B + k], ks = prm[2 * B + k];
  float c1 = 0.0f, c2 = 0.0f;
  if (state) {
    c1 = state[k];
    c2 = state[B + k];
  }
  const size_t plane = (size_t)T * B;
  // lane l copies/stores frame 4i + l/16 of an instruction's four, lanes
  // k0 + 4(l%16) .. +3 of it
  const int fq = lane >> 4, kq = k0 + 4 * (lane & 15);
  const float* const srcs[NI] = {x, tgt, tape};
  // (the buffers are named, not passed by reference: a generic pointer to
  // them here made the compiler emit an illegal aperture compare)
  auto issue = [&](auto bi, int n0) {
#pragma unroll
    for (int a = 0; a < NI; ++a)
#pragma unroll
      for (int i = 0; i < kTileF / 4; ++i) {
        const void* src = srcs[a] + (size_t)(n0 + 4 * i + fq) * B + kq;
        if constexpr (decltype(bi)::value == 0)
          __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)&in0[a][4 * i][0], 16, 0, 0);
        else
          __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)&in1[a][4 * i][0], 16, 0, 0);
      }
  };
  float ls = 0.0f;
  auto tile = [&](const float (&buf)[NI][kTileF][64], int n0) {
#pragma unroll 4
    for (int f = 0; f < kTileF; ++f) {
      SvfK K;
      K.g = buf[2][f][lane];
      K.Q = 1.0f + K.g * (K.g + kd);
      K.a1 = rcp_rn(K.Q);
      K.a2 = K.g * K.a1;
      out[0][f][lane] = c1;
      out[1][f][lane] = c2;
      const float o = svf_step<true>(K, ks, buf[0][f][lane], c1, c2);
      out[2][f][lane] = sanitize && !isfinite(o) ? 0.0f : o;
      const float d = o - buf[1][f][lane];
      ls += d * d;
    }
    // the wave's own LDS writes land before its reads below (in order)
    wave_sync();
    float* const dsts[3] = {cells, cells + plane, y};
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int i = 0; i < kTileF / 4; ++i) {
        const float4 v = *reinterpret_cast<const float4*>(&out[a][4 * i + fq][4 * (lane & 15)]);
        *reinterpret_cast<float4*>(dsts[a] + (size_t)(n0 + 4 * i + fq) * B + kq) = v;
      }
    // a chunk's partial is complete at its last tile; the last chunk ends
    // at T, which need not be a multiple of L
    if ((n0 + kTileF) % L == 0 || n0 + kTileF == T) {
      lossp[(size_t)((n0 + kTileF - 1) / L) * B + k] = ls;
      ls = 0.0f;
    }
  };
  const int ntile = T / kTileF;
  const std::integral_constant<int, 0> b0;
  const std::integral_constant<int, 1> b1;
  issue(b0, 0);
  for (int t = 0; t < ntile; t += 2) {
    // tile t from in0 (its copies landed), tile t+1's copies into in1
    if (t + 1 < ntile) issue(b1, (t + 1) * kTileF);
    tile(in0, t * kTileF);
    if (t + 1 >= ntile) break;
    if (t + 2 < ntile) issue(b0, (t + 2) * kTileF);
    tile(in1, (t + 1) * kTileF);
  }
  if (state) {
    state[k] = c1;
    state[B + k] = c2;
  }
}

// ------------------------------------------------------------ adjoint scan
// d s / d c for s = c / (1 + |ks c|): 1/D - (c/D^2) sgn(ks c) ks (1 when linear).
__device__ __forceinline__ float sgn(float v) { return v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f); }

template <bool SAT>
__global__ __launch_bounds__(kThreads) void k_svf_adj_chunk(Ctl ctl, const float* __restrict__ prm,
                                                            const float* __restrict__ y,
                                                            const float* __restrict__ tgt,
                                                            const float* __restrict__ cells,
                                                            double* __restrict__ summ, int B, int T, int L, float sr) {
  Lane l;
  if (!lane_chunk(prm, B, T, L, sr, SAT, l)) return;
  double l1 = 0.0, l2 = 0.0, u1 = 1.0, u2 = 0.0, w1 = 0.0, w2 = 1.0;
  // the cells' adjoint through one frame (the reverse of svf_step)
  auto back = [](double a1, double a2, double g, double J1, double J2, double e, double& L1, double& L2) {
    const double ic2_b = 0.5 * e + L2;
    const double v2_b = 2.0 * ic2_b;
    double s2_b = (0.5 * e - ic2_b) + v2_b;
    const double v1p_b = v2_b * g;
    const double ic1_b = L1 + 0.5 * v1p_b;
    double s1_b = 0.5 * v1p_b - ic1_b;
    const double v1_b = 2.0 * ic1_b;
    s1_b += v1_b * a1;
    s2_b -= v1_b * a2;
    L1 = s1_b * J1;
    L2 = s2_b * J2;
  };
  auto frame = [&](const float* v, float m, float e) {
    const SvfK K = svf_coef(raw_cutoff(l.base, m, e, ctl), l.kd, sr, l.rsr);
    double J1 = 1.0, J2 = 1.0;
    if constexpr (SAT) {
      // ds/dc = 1/D - (c/D^2) sgn(ks c) ks = (D - |ks c|)/D^2 = 1/D^2
      const float r1 = rcp_rn(1.0f + fabsf(l.ks * v[2])), r2 = rcp_rn(1.0f + fabsf(l.ks * v[3]));
      J1 = (double)r1 * (double)r1;
      J2 = (double)r2 * (double)r2;
    }
    const double a1 = K.a1, a2 = K.a2, g = K.g;
    const double ee = 2.0 * ((double)v[0] - (double)v[1]);
    back(a1, a2, g, J1, J2, ee, l1, l2);
    back(a1, a2, g, J1, J2, 0.0, u1, u2);
    back(a1, a2, g, J1, J2, 0.0, w1, w2);
  };
  const size_t plane = (size_t)T * B;
  if constexpr (SAT) {
    const float* const src[4] = {y, tgt, cells, cells + plane};
    walk<4, true>(src, ctl, B, l.k, l.n0, l.n1, [&](int, const float* v, float m, float e) { frame(v, m, e); });
  } else {
    const float* const src[2] = {y, tgt};
    walk<2, true>(src, ctl, B, l.k, l.n0, l.n1, [&](int, const float* v, float m, float e) { frame(v, m, e); });
  }
  double* o = summ + (size_t)l.c * 6 * B + l.k;
  o[0] = l1;
  o[(size_t)B] = l2;
  o[(size_t)2 * B] = u1;
  o[(size_t)3 * B] = u2;
  o[(size_t)4 * B] = w1;
  o[(size_t)5 * B] = w2;
}

// Each chunk's adjoint replayed from its carry in fp32 (node order of the
// CPU restatement), with the chain rule through the coefficient nodes:
// a2 = g a1, a1 = 1/Q, Q = 1 + g (g + kd), g = tan(u) (d/du = 1/(cos u)^2),
// u = (pi fc) / sr, fc = clip(base m + env), kd = 1/res.
// gpart[c][0][k] = d/d base, [1] = d/d res, [2] = d/d kSat (saturating).
template <bool SAT>
__global__ __launch_bounds__(kThreads) void k_svf_bwd(const float* __restrict__ x, Ctl ctl,
                                                      const float* __restrict__ prm, const float* __restrict__ y,
                                                      const float* __restrict__ tgt, const float* __restrict__ cells,
                                                      const float* __restrict__ ainit, float* __restrict__ gpart,
                                                      float* __restrict__ xbar, int B, int T, int L, float sr) {
  Lane l;
  if (!lane_chunk(prm, B, T, L, sr, SAT, l)) return;
  const int k = l.k;
  float L1 = ainit[(size_t)l.c * 2 * B + k], L2 = ainit[((size_t)l.c * 2 + 1) * B + k];
  float gb = 0.0f, gkd = 0.0f, gks = 0.0f;
  const float ks = l.ks;
  const size_t plane = (size_t)T * B;
  const float* const src[5] = {x, y, tgt, cells, cells + plane};
  walk<5, true>(src, ctl, B, k, l.n0, l.n1, [&](int n, const float* v, float m, float e) {
    const SvfK K = svf_coef(raw_cutoff(l.base, m, e, ctl), l.kd, sr, l.rsr);
    const float c1 = v[3], c2 = v[4];
    const float D1 = 1.0f + fabsf(ks * c1), D2 = 1.0f + fabsf(ks * c2);
    const float s1 = sat_div<SAT>(c1, ks), s2 = sat_div<SAT>(c2, ks);
    const float v3 = v[0] - s2;
    const float v1 = K.a1 * s1 + K.a2 * v3;
    const float ic1 = 2.0f * v1 - s1;
    const float v1p = (ic1 + s1) * 0.5f;
    const float ee = 2.0f * (v[1] - v[2]);
    const float ic2_b = 0.5f * ee + L2;
    float s2_b = 0.5f * ee - ic2_b;
    const float v2_b = 2.0f * ic2_b;
    s2_b += v2_b;
    float g_b = v2_b * v1p;
    const float v1p_b = v2_b * K.g;
    const float ic1_b = L1 + 0.5f * v1p_b;
    float s1_b = 0.5f * v1p_b - ic1_b;
    const float v1_b = 2.0f * ic1_b;
    float a1_b = v1_b * s1;
    s1_b += v1_b * K.a1;
    const float a2_b = v1_b * v3;
    const float v3_b = v1_b * K.a2;
    if (xbar) xbar[(size_t)n * B + k] = v3_b;
    s2_b -= v3_b;
    if constexpr (SAT) {
      // ds/dc = 1/D^2, ds/dks = -(c/D^2) sgn(ks c) c = -s |c| sgn(ks) / D
      const float r1 = rcp_rn(D1), r2 = rcp_rn(D2);
      const float q1 = (c1 * (r1 * r1)) * sgn(ks * c1), q2 = (c2 * (r2 * r2)) * sgn(ks * c2);
      L1 = s1_b * (r1 * r1);
      L2 = s2_b * (r2 * r2);
      gks += -(s1_b * q1 * c1) - s2_b * q2 * c2;
    } else {
      L1 = s1_b;
      L2 = s2_b;
    }
    g_b += a2_b * K.a1;
    a1_b += a2_b * K.g;
    const float Q_b = -a1_b / (K.Q * K.Q);
    g_b += Q_b * ((K.g + l.kd) + K.g);
    gkd += Q_b * K.g;
    const float cu = cosf(K.u);
    const float u_b = g_b * (1.0f / (cu * cu));
    const float fc_b = div_rn(u_b, sr, l.rsr) * kPi;
    if (K.pass) gb += fc_b * m;
  });
  const int P = SAT ? 3 : 2;
  gpart[((size_t)l.c * P) * B + k] = gb;
  gpart[((size_t)l.c * P + 1) * B + k] = gkd * (-1.0f / (l.res * l.res));
  if constexpr (SAT) gpart[((size_t)l.c * P + 2) * B + k] = gks;
}

struct SvfShape {
  int64_t B, T, L, C;
};

int svf_shape(int64_t B, int64_t T, int64_t L, SvfShape& s, const char* who) {
  DGEN_REQUIRE(B > 0 && B <= (1 << 20) && T > 0 && T < (1ll << 30) && L > 0 && L <= (1 << 20),
               "%s: B %lld T %lld L %lld", who, (long long)B, (long long)T, (long long)L);
  DGEN_REQUIRE(B * T < (1ll << 40), "%s: B*T too large", who);
  s = SvfShape{B, T, L, (T + L - 1) / L};
  DGEN_REQUIRE(s.C <= 65535, "%s: %lld chunks exceeds the grid limit (raise the chunk length)", who,
               (long long)s.C);
  return 0;
}

dim3 svf_grid(const SvfShape& s) { return dim3((unsigned)s.C, (unsigned)((s.B + kThreads - 1) / kThreads)); }

double* dcell(const Launch& L, int64_t off) { return reinterpret_cast<double*>(cell(L, off)); }

int svf_ctl(const Launch& L, int64_t m, int64_t env, int64_t T, const char* who, Ctl& ctl) {
  if (m >= 0) DGEN_CHECK_CELL(L, m, T, who);
  if (env >= 0) DGEN_CHECK_CELL(L, env, T, who);
  ctl.m = m >= 0 ? cell(L, m) : nullptr;
  ctl.env = env >= 0 ? cell(L, env) : nullptr;
  return 0;
}

int svf_rate(const Launch& L, float rendered, const char* who, float& sr) {
  sr = host_rate(L, rendered);
  DGEN_REQUIRE(sr > 0.f && sr < 1e30f, "%s: sample rate %g", who, (double)sr);
  return 0;
}

}  // namespace

int launch_svf_chunk(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=x [1]=mod or -1 [2]=env or -1 [3]=params ([2][B]) [4]=summary ([C][6][B] fp64) [5]=B [6]=T [7]=L
  const int64_t x = op.arg[0], prm = op.arg[3], summ = op.arg[4];
  SvfShape s;
  if (int rc = svf_shape(op.arg[5], op.arg[6], op.arg[7], s, "svf_chunk")) return rc;
  Ctl ctl{};
  if (int rc = svf_ctl(L, op.arg[1], op.arg[2], s.T, "svf_chunk.mod/env", ctl)) return rc;
  float sr;
  if (int rc = svf_rate(L, op.farg[0], "svf_chunk", sr)) return rc;
  DGEN_CHECK_CELL(L, x, s.B * s.T, "svf_chunk.x");
  DGEN_CHECK_CELL(L, prm, 2 * s.B, "svf_chunk.params");
  DGEN_CHECK_CELL(L, summ, 12 * s.C * s.B, "svf_chunk.summary");
  DGEN_REQUIRE(summ % 2 == 0, "svf_chunk: summary cell must be 8-byte aligned");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_svf_chunk, svf_grid(s), dim3(kThreads), 0, L.stream, cell(L, x), ctl, cell(L, prm),
                     dcell(L, summ), (int)s.B, (int)s.T, (int)s.L, sr);
  DGEN_LAUNCH_CHECK("k_svf_chunk");
  return 0;
}

int launch_svf_fwd(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=x [1]=mod [2]=env [3]=params ([2][B]) [4]=init ([C][2][B]) [5]=y [6]=cells ([2][T][B]) or -1
  //      [7]=target or -1 [8]=loss partials ([C][B]) or -1 [9]=B [10]=T [11]=L
  //      [12]=adjoint summary ([C][6][B] fp64) when [13]=1
  const int64_t x = op.arg[0], prm = op.arg[3], init = op.arg[4], y = op.arg[5], cl = op.arg[6], tgt = op.arg[7],
                lossp = op.arg[8];
  SvfShape s;
  if (int rc = svf_shape(op.arg[9], op.arg[10], op.arg[11], s, "svf_fwd")) return rc;
  Ctl ctl{};
  if (int rc = svf_ctl(L, op.arg[1], op.arg[2], s.T, "svf_fwd.mod/env", ctl)) return rc;
  float sr;
  if (int rc = svf_rate(L, op.farg[0], "svf_fwd", sr)) return rc;
  DGEN_CHECK_CELL(L, x, s.B * s.T, "svf_fwd.x");
  DGEN_CHECK_CELL(L, prm, 2 * s.B, "svf_fwd.params");
  DGEN_CHECK_CELL(L, init, 2 * s.C * s.B, "svf_fwd.init");
  DGEN_CHECK_CELL(L, y, s.B * s.T, "svf_fwd.y");
  if (cl >= 0) DGEN_CHECK_CELL(L, cl, 2 * s.B * s.T, "svf_fwd.cells");
  DGEN_REQUIRE((tgt >= 0) == (lossp >= 0), "svf_fwd: target and loss partials go together");
  if (tgt >= 0) {
    DGEN_CHECK_CELL(L, tgt, s.B * s.T, "svf_fwd.target");
    DGEN_CHECK_CELL(L, lossp, s.C * s.B, "svf_fwd.loss_partials");
  }
  const bool adj = op.arg[13] == 1;
  const int64_t asumm = op.arg[12];
  if (adj) {
    DGEN_REQUIRE(tgt >= 0, "svf_fwd: the adjoint summary needs the target");
    DGEN_REQUIRE(asumm % 2 == 0, "svf_fwd: summary cell must be 8-byte aligned");
    DGEN_CHECK_CELL(L, asumm, 12 * s.C * s.B, "svf_fwd.adjoint_summary");
  }
  if (L.dry) return 0;
  float* cp = cl >= 0 ? cell(L, cl) : nullptr;
  if (adj)
    hipLaunchKernelGGL((k_svf_fwd<true, true>), svf_grid(s), dim3(kThreads), 0, L.stream, cell(L, x), ctl,
                       cell(L, prm), cell(L, init), cell(L, y), cp, cell(L, tgt), cell(L, lossp), (int)s.B, (int)s.T,
                       (int)s.L, sr, dcell(L, asumm));
  else if (tgt >= 0)
    hipLaunchKernelGGL(k_svf_fwd<true>, svf_grid(s), dim3(kThreads), 0, L.stream, cell(L, x), ctl, cell(L, prm),
                       cell(L, init), cell(L, y), cp, cell(L, tgt), cell(L, lossp), (int)s.B, (int)s.T, (int)s.L, sr,
                       nullptr);
  else
    hipLaunchKernelGGL(k_svf_fwd<false>, svf_grid(s), dim3(kThreads), 0, L.stream, cell(L, x), ctl, cell(L, prm),
                       cell(L, init), cell(L, y), cp, nullptr, nullptr, (int)s.B, (int)s.T, (int)s.L, sr, nullptr);
  DGEN_LAUNCH_CHECK("k_svf_fwd");
  return 0;
}

int launch_svf_seq(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=x [1]=mod [2]=env [3]=params ([3][B]) [4]=state ([2][B]) or -1 [5]=y [6]=cells or -1
  //      [7]=target or -1 [8]=loss partials ([C][B]) or -1 [9]=B [10]=T [11]=L [12]=sanitize
  //      [13]=coefficient tape ([T][B]) or -1
  // As DGEN_HIP_K_STREAM_SVF: state required, no cells or loss, and a run
  // processes the first frame_count frames.
  const int64_t x = op.arg[0], prm = op.arg[3], st = op.arg[4], y = op.arg[5], cl = op.arg[6], tgt = op.arg[7],
                lossp = op.arg[8];
  const bool stream = op.kernel == DGEN_HIP_K_STREAM_SVF;
  SvfShape s;
  if (int rc = svf_shape(op.arg[9], op.arg[10], op.arg[11], s, "svf_seq")) return rc;
  const int64_t T = stream ? std::min<int64_t>(s.T, L.frames) : s.T;
  const int64_t tape = op.arg[13];
  DGEN_REQUIRE(!stream || (st >= 0 && cl < 0 && tgt < 0 && tape < 0),
               "stream_svf: needs a state cell, stores no cells, loss or coefficient tape");
  Ctl ctl{};
  if (int rc = svf_ctl(L, op.arg[1], op.arg[2], s.T, "svf_seq.mod/env", ctl)) return rc;
  float sr;
  if (int rc = svf_rate(L, op.farg[0], "svf_seq", sr)) return rc;
  DGEN_CHECK_CELL(L, x, s.B * s.T, "svf_seq.x");
  DGEN_CHECK_CELL(L, prm, 3 * s.B, "svf_seq.params");
  if (st >= 0) DGEN_CHECK_CELL(L, st, 2 * s.B, "svf_seq.state");
  DGEN_CHECK_CELL(L, y, s.B * s.T, "svf_seq.y");
  if (cl >= 0) DGEN_CHECK_CELL(L, cl, 2 * s.B * s.T, "svf_seq.cells");
  DGEN_REQUIRE((tgt >= 0) == (lossp >= 0), "svf_seq: target and loss partials go together");
  if (tgt >= 0) {
    DGEN_CHECK_CELL(L, tgt, s.B * s.T, "svf_seq.target");
    DGEN_CHECK_CELL(L, lossp, s.C * s.B, "svf_seq.loss_partials");
  }
  if (tape >= 0) DGEN_CHECK_CELL(L, tape, s.B * s.T, "svf_seq.coefficient_tape");
  if (L.dry) return 0;
  const dim3 grid((unsigned)((s.B + kSeqThreads - 1) / kSeqThreads));
  float* sp = st >= 0 ? cell(L, st) : nullptr;
  float* cp = cl >= 0 ? cell(L, cl) : nullptr;
  const int reset = stream && L.reset ? 1 : 0, san = op.arg[12] ? 1 : 0;
  float* tp = tape >= 0 ? cell(L, tape) : nullptr;
  if (tp) {
    hipLaunchKernelGGL(k_svf_coef, svf_grid(s), dim3(kThreads), 0, L.stream, ctl, cell(L, prm), tp, (int)s.B,
                       (int)s.T, (int)s.L, sr);
    DGEN_LAUNCH_CHECK("k_svf_coef");
  }
  float* tg = tgt >= 0 ? cell(L, tgt) : nullptr;
  float* lp = lossp >= 0 ? cell(L, lossp) : nullptr;
  if (tgt >= 0 && tp && cp && !stream && s.B % 64 == 0 && T % kTileF == 0 && s.L % kTileF == 0) {
    // the training forward through LDS tiles (the same arithmetic)
    hipLaunchKernelGGL(k_svf_seq_tiled, dim3((unsigned)(s.B / 64)), dim3(64), 0, L.stream, cell(L, x), cell(L, prm),
                       tp, sp, cell(L, y), cp, tg, lp, (int)s.B, (int)T, (int)s.L, san);
    DGEN_LAUNCH_CHECK("k_svf_seq_tiled");
    return 0;
  }
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kSeqThreads), 0, L.stream, cell(L, x), ctl, cell(L, prm), tp, sp, reset,
                       cell(L, y), cp, tg, lp, (int)s.B, (int)T, (int)s.L, sr, san);
  };
  if (tgt >= 0)
    tp ? go(k_svf_seq<true, true>) : go(k_svf_seq<true, false>);
  else
    tp ? go(k_svf_seq<false, true>) : go(k_svf_seq<false, false>);
  DGEN_LAUNCH_CHECK("k_svf_seq");
  return 0;
}

int launch_svf_adj_chunk(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=mod [1]=env [2]=params ([P][B]) [3]=y [4]=target [5]=cells (saturating) or -1 [6]=summary
  //      [7]=B [8]=T [9]=L [10]=saturating
  const int64_t prm = op.arg[2], y = op.arg[3], tgt = op.arg[4], cl = op.arg[5], summ = op.arg[6], sat = op.arg[10];
  SvfShape s;
  if (int rc = svf_shape(op.arg[7], op.arg[8], op.arg[9], s, "svf_adj_chunk")) return rc;
  DGEN_REQUIRE(sat == 0 || sat == 1, "svf_adj_chunk: saturating %lld", (long long)sat);
  Ctl ctl{};
  if (int rc = svf_ctl(L, op.arg[0], op.arg[1], s.T, "svf_adj_chunk.mod/env", ctl)) return rc;
  float sr;
  if (int rc = svf_rate(L, op.farg[0], "svf_adj_chunk", sr)) return rc;
  DGEN_CHECK_CELL(L, prm, (2 + sat) * s.B, "svf_adj_chunk.params");
  DGEN_CHECK_CELL(L, y, s.B * s.T, "svf_adj_chunk.y");
  DGEN_CHECK_CELL(L, tgt, s.B * s.T, "svf_adj_chunk.target");
  DGEN_REQUIRE(!sat || cl >= 0, "svf_adj_chunk: the saturating adjoint reads the stored cells");
  if (cl >= 0) DGEN_CHECK_CELL(L, cl, 2 * s.B * s.T, "svf_adj_chunk.cells");
  DGEN_CHECK_CELL(L, summ, 12 * s.C * s.B, "svf_adj_chunk.summary");
  DGEN_REQUIRE(summ % 2 == 0, "svf_adj_chunk: summary cell must be 8-byte aligned");
  if (L.dry) return 0;
  if (sat)
    hipLaunchKernelGGL(k_svf_adj_chunk<true>, svf_grid(s), dim3(kThreads), 0, L.stream, ctl, cell(L, prm),
                       cell(L, y), cell(L, tgt), cell(L, cl), dcell(L, summ), (int)s.B, (int)s.T, (int)s.L, sr);
  else
    hipLaunchKernelGGL(k_svf_adj_chunk<false>, svf_grid(s), dim3(kThreads), 0, L.stream, ctl, cell(L, prm),
                       cell(L, y), cell(L, tgt), nullptr, dcell(L, summ), (int)s.B, (int)s.T, (int)s.L, sr);
  DGEN_LAUNCH_CHECK("k_svf_adj_chunk");
  return 0;
}

int launch_svf_bwd(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=x [1]=mod [2]=env [3]=params ([P][B]) [4]=y [5]=target [6]=cells [7]=adjoint init ([C][2][B])
  //      [8]=grad partials ([C][P][B]) [9]=xbar ([T][B]) or -1 [10]=B [11]=T [12]=L [13]=saturating
  const int64_t x = op.arg[0], prm = op.arg[3], y = op.arg[4], tgt = op.arg[5], cl = op.arg[6], ainit = op.arg[7],
                gpart = op.arg[8], xb = op.arg[9], sat = op.arg[13];
  SvfShape s;
  if (int rc = svf_shape(op.arg[10], op.arg[11], op.arg[12], s, "svf_bwd")) return rc;
  DGEN_REQUIRE(sat == 0 || sat == 1, "svf_bwd: saturating %lld", (long long)sat);
  Ctl ctl{};
  if (int rc = svf_ctl(L, op.arg[1], op.arg[2], s.T, "svf_bwd.mod/env", ctl)) return rc;
  float sr;
  if (int rc = svf_rate(L, op.farg[0], "svf_bwd", sr)) return rc;
  const int64_t P = 2 + sat;
  DGEN_CHECK_CELL(L, x, s.B * s.T, "svf_bwd.x");
  DGEN_CHECK_CELL(L, prm, P * s.B, "svf_bwd.params");
  DGEN_CHECK_CELL(L, y, s.B * s.T, "svf_bwd.y");
  DGEN_CHECK_CELL(L, tgt, s.B * s.T, "svf_bwd.target");
  DGEN_CHECK_CELL(L, cl, 2 * s.B * s.T, "svf_bwd.cells");
  DGEN_CHECK_CELL(L, ainit, 2 * s.C * s.B, "svf_bwd.adjoint_init");
  DGEN_CHECK_CELL(L, gpart, P * s.C * s.B, "svf_bwd.grad_partials");
  if (xb >= 0) DGEN_CHECK_CELL(L, xb, s.B * s.T, "svf_bwd.xbar");
  if (L.dry) return 0;
  float* xp = xb >= 0 ? cell(L, xb) : nullptr;
  if (sat)
    hipLaunchKernelGGL(k_svf_bwd<true>, svf_grid(s), dim3(kThreads), 0, L.stream, cell(L, x), ctl, cell(L, prm),
                       cell(L, y), cell(L, tgt), cell(L, cl), cell(L, ainit), cell(L, gpart), xp, (int)s.B, (int)s.T,
                       (int)s.L, sr);
  else
    hipLaunchKernelGGL(k_svf_bwd<false>, svf_grid(s), dim3(kThreads), 0, L.stream, cell(L, x), ctl, cell(L, prm),
                       cell(L, y), cell(L, tgt), cell(L, cl), cell(L, ainit), cell(L, gpart), xp, (int)s.B, (int)s.T,
                       (int)s.L, sr);
  DGEN_LAUNCH_CHECK("k_svf_bwd");
  return 0;
}

}  // namespace dgen
