// Tensor biquad bank (RBJ low-pass, Direct Form I, coefficients recomputed
// every sample) and its BPTT adjoint.
//
// Reference: the biquad graph Sources/DGen/HigherOps.swift:401-570 (tensor
// form SignalTensor.biquad, Sources/DGenLazy/Functions.swift:1196-1217), run
// as one sequential frame loop per lane (StatefulTensorParallelPolicy.swift:
// 21-74) and, for the gradient, a reverse-time loop over stored per-frame
// values (BPTTEmission.swift:133-160).
//
// Here time is parallel too.  The recurrence y[n] = F[n] - a1[n] y[n-1] -
// a2[n] y[n-2] is affine in the state (y[n-1], y[n-2]), so the frames are cut
// into chunks of L and one thread owns one (lane, chunk):
//   k_bq_chunk      the chunk's zero-state response and its responses to the
//                   two unit initial states (an affine 2x2 map per chunk)
//   k_bq_carry      per lane, the chunk maps composed in order (a two-level
//                   scan through LDS) -> every chunk's exact initial state
// The summaries and the carry are evaluated in fp64 on the fp32 coefficient
// sequence: at low cutoffs the two unit responses are large (~1/w0) and
// nearly opposite, so an fp32 composition would cancel ~7 bits at every chunk
// boundary.  Each chunk then starts from the exact state of the same fp32
// program rounded to fp32, and runs the reference's fp32 Direct Form I.
//   k_bq_fwd        each chunk re-run from its initial state: y, and the
//                   per-chunk partial sums of the loss sum (y - tgt)^2
// The adjoint lambda[n] = g[n] - a1[n+1] lambda[n+1] - a2[n+2] lambda[n+2],
// g = 2 (y - tgt), is the same kind of recurrence run backwards, with the
// carries (v1, v2) = what is owed to lambda[n-1] and lambda[n-2]:
//   chunk summaries (k_bq_adj_chunk, or formed by k_bq_fwd's replay),
//   k_bq_carry (reverse), k_bq_bwd -> per-chunk gradient partials [C][2][B],
//   summed per lane by the deterministic column sum.
//
// Layout: x, y, tgt are [T][B] (frame-major, lane-minor: a wave reads 256
// contiguous bytes per frame); parameters are [2][B] = base | Q; the cutoff
// of lane k at frame n is base[k] * m[n] (m: the shared modulation signal).
#include <mutex>

#include "dev_math.h"
#include "internal.h"

namespace dgen {
namespace {

constexpr int kThreads = 256;  // lanes per workgroup (one chunk)
constexpr int kG = 8;          // frames per prefetch group
constexpr int kCarryLanes = 8;  // lanes per carry workgroup
constexpr int kCarryGroups = 32;  // chunk groups per lane in the carry scan

// 2*pi/44100 as the Float constant the reference hardcodes
// (HigherOps.swift:446-447), whatever the sample rate.
constexpr float kW0PerHz = 0.00014247585730565955f;

struct Coef {
  float c, s, alpha, r, P, D;  // cos w, sin w, div18, recip24, div11, add10
  float b0, b1, a1, a2;        // b2 == b0 for the low-pass
};

// RBJ low-pass, mode 0 and gain 1, in the reference graph's node order
// (HigherOps.swift:443-556): mult7 = |fc| * w0/Hz; add10 = 1 - cos;
// div11 = add10 / 2; div18 = (sin * 0.5) / |Q|; recip24 = 1 / (div18 + 1);
// b0 = b2 = div11 * recip24, b1 = add10 * recip24, a1 = (-2 cos) * recip24,
// a2 = (1 - div18) * recip24.  q = |Q|, rq = RN(1/q).
__device__ __forceinline__ Coef coef(float fc, float q, float rq) {
  Coef k;
  const float w = fabsf(fc) * kW0PerHz;
  sincosf(w, &k.s, &k.c);
  k.D = 1.0f - k.c;
  k.P = k.D * 0.5f;
  k.alpha = div_rn(k.s * 0.5f, q, rq);
  k.r = rcp_rn(k.alpha + 1.0f);
  k.b0 = k.P * k.r;
  k.b1 = k.D * k.r;
  k.a2 = (1.0f - k.alpha) * k.r;
  k.a1 = (-2.0f * k.c) * k.r;
  return k;
}

// Streams frames [n0, n1) forward: f(n, v, m) with v[s] = src[s][n][k] and
// m = mod[n] (1 when unmodulated).  The next group's loads are issued before
// the current group is processed; indices are clamped into [n0, n1).
template <int NS, bool MOD, class F>
__device__ __forceinline__ void walk_fwd(const float* const (&src)[NS], const float* __restrict__ mod, int B, int k,
                                         int n0, int n1, F&& f) {
  float cv[kG][NS], cm[kG];
  auto load = [&](int n, float (&v)[kG][NS], float (&mv)[kG]) {
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      const int nn = min(n + j, n1 - 1);
#pragma unroll
      for (int s = 0; s < NS; ++s) v[j][s] = src[s][(size_t)nn * B + k];
      mv[j] = MOD ? mod[nn] : 1.0f;
    }
  };
  load(n0, cv, cm);
  int n = n0;
  for (; n + kG <= n1; n += kG) {
    float nv[kG][NS], nm[kG];
    load(n + kG, nv, nm);
#pragma unroll
    for (int j = 0; j < kG; ++j) f(n + j, cv[j], cm[j]);
#pragma unroll
    for (int j = 0; j < kG; ++j) {
#pragma unroll
      for (int s = 0; s < NS; ++s) cv[j][s] = nv[j][s];
      cm[j] = nm[j];
    }
  }
#pragma unroll
  for (int j = 0; j < kG; ++j)
    if (n + j < n1) f(n + j, cv[j], cm[j]);
}

// Streams frames hi-1, hi-2, ..., lo backwards (lo may be negative: frames
// before 0 read as 0, modulation as 1), prefetching like walk_fwd.
template <int NS, bool MOD, class F>
__device__ __forceinline__ void walk_rev(const float* const (&src)[NS], const float* __restrict__ mod, int B, int k,
                                         int hi, int lo, F&& f) {
  float cv[kG][NS], cm[kG];
  auto load = [&](int n, float (&v)[kG][NS], float (&mv)[kG]) {
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      const int nn = max(n - j, lo);
      const int nc = max(nn, 0);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float t = src[s][(size_t)nc * B + k];
        v[j][s] = nn >= 0 ? t : 0.0f;
      }
      mv[j] = MOD ? (nn >= 0 ? mod[nc] : 1.0f) : 1.0f;
    }
  };
  load(hi - 1, cv, cm);
  int n = hi - 1;
  for (; n - kG + 1 >= lo; n -= kG) {
    float nv[kG][NS], nm[kG];
    load(n - kG, nv, nm);
#pragma unroll
    for (int j = 0; j < kG; ++j) f(n - j, cv[j], cm[j]);
#pragma unroll
    for (int j = 0; j < kG; ++j) {
#pragma unroll
      for (int s = 0; s < NS; ++s) cv[j][s] = nv[j][s];
      cm[j] = nm[j];
    }
  }
#pragma unroll
  for (int j = 0; j < kG; ++j)
    if (n - j >= lo) f(n - j, cv[j], cm[j]);
}

__device__ __forceinline__ float sign_of(float v) { return v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f); }

struct LaneChunk {
  int k, c, n0, n1;
  float base, q, rq, qsign;
};

__device__ __forceinline__ bool lane_chunk(const float* __restrict__ prm, int B, int T, int L, LaneChunk& lc) {
  lc.k = blockIdx.y * kThreads + threadIdx.x;
  if (lc.k >= B) return false;
  lc.c = blockIdx.x;
  lc.n0 = lc.c * L;
  lc.n1 = min(T, lc.n0 + L);
  lc.base = prm[lc.k];
  const float Q = prm[B + lc.k];
  lc.q = fabsf(Q);
  lc.rq = 1.0f / lc.q;
  lc.qsign = sign_of(Q);
  return true;
}

// ------------------------------------------------------------ forward scan
template <bool MOD>
__global__ __launch_bounds__(kThreads) void k_bq_chunk(const float* __restrict__ x, const float* __restrict__ mod,
                                                       const float* __restrict__ prm, double* __restrict__ summ,
                                                       int B, int T, int L) {
  LaneChunk lc;
  if (!lane_chunk(prm, B, T, L, lc)) return;
  const int k = lc.k;
  double x1 = lc.n0 >= 1 ? x[(size_t)(lc.n0 - 1) * B + k] : 0.0f;
  double x2 = lc.n0 >= 2 ? x[(size_t)(lc.n0 - 2) * B + k] : 0.0f;
  double p1 = 0.0, p2 = 0.0, u1 = 1.0, u2 = 0.0, w1 = 0.0, w2 = 1.0;
  const float* const src[1] = {x};
  walk_fwd<1, MOD>(src, mod, B, k, lc.n0, lc.n1, [&](int, const float* v, float m) {
    const Coef K = coef(lc.base * m, lc.q, lc.rq);
    const double b0 = K.b0, b1 = K.b1, a1 = K.a1, a2 = K.a2;
    const double x0 = v[0];
    const double p = ((x2 * b0 + x1 * b1) + x0 * b0) - (p2 * a2 + p1 * a1);
    const double u = -(u2 * a2 + u1 * a1);
    const double w = -(w2 * a2 + w1 * a1);
    p2 = p1;
    p1 = p;
    u2 = u1;
    u1 = u;
    w2 = w1;
    w1 = w;
    x2 = x1;
    x1 = x0;
  });
  double* o = summ + (size_t)lc.c * 6 * B + k;
  o[0] = p1;
  o[(size_t)B] = p2;
  o[(size_t)2 * B] = u1;
  o[(size_t)3 * B] = u2;
  o[(size_t)4 * B] = w1;
  o[(size_t)5 * B] = w2;
}

// Affine map Y -> p + [u w] Y on the 2-vector Y = (Y1, Y2).
struct Map {
  double p1, p2, u1, u2, w1, w2;
};
__device__ __forceinline__ Map load_map(const double* __restrict__ summ, int B, int c, int k) {
  const double* s = summ + (size_t)c * 6 * B + k;
  return Map{s[0], s[(size_t)B], s[(size_t)2 * B], s[(size_t)3 * B], s[(size_t)4 * B], s[(size_t)5 * B]};
}
// then(a, b): apply a, then b.
__device__ __forceinline__ Map then(const Map& a, const Map& b) {
  return Map{b.p1 + b.u1 * a.p1 + b.w1 * a.p2, b.p2 + b.u2 * a.p1 + b.w2 * a.p2,
             b.u1 * a.u1 + b.w1 * a.u2,        b.u2 * a.u1 + b.w2 * a.u2,
             b.u1 * a.w1 + b.w1 * a.w2,        b.u2 * a.w1 + b.w2 * a.w2};
}

// Initial state of every chunk: init[c] = (Y1, Y2) entering chunk c in the
// scan's order (ascending c, or descending for the adjoint), from zero state
// before the first.  Workgroup = kCarryLanes lanes x kCarryGroups groups of
// consecutive chunks: (1) each thread composes its group's maps, (2) one
// thread per lane scans the group maps in LDS, (3) each thread replays its
// group from the group's initial state, writing every chunk's.
__global__ __launch_bounds__(kCarryLanes* kCarryGroups) void k_bq_carry(const double* __restrict__ summ,
                                                                         float* __restrict__ init, int B, int C,
                                                                         int reverse) {
  __shared__ Map s_map[kCarryGroups][kCarryLanes];
  __shared__ double s_y[kCarryGroups][kCarryLanes][2];
  const int l = threadIdx.x % kCarryLanes, g = threadIdx.x / kCarryLanes;
  const int k = blockIdx.x * kCarryLanes + l;
  const bool live = k < B;
  const int per = (C + kCarryGroups - 1) / kCarryGroups;
  const int i0 = min(C, g * per), i1 = min(C, i0 + per);  // positions in scan order
  auto chunk_at = [&](int i) { return reverse ? C - 1 - i : i; };
  Map acc{0.0, 0.0, 1.0, 0.0, 0.0, 1.0};
  if (live) {
    int i = i0;
    for (; i + 4 <= i1; i += 4) {
      Map m[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) m[j] = load_map(summ, B, chunk_at(i + j), k);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = then(acc, m[j]);
    }
    for (; i < i1; ++i) acc = then(acc, load_map(summ, B, chunk_at(i), k));
  }
  s_map[g][l] = acc;
  __syncthreads();
  if (g == 0) {
    double Y1 = 0.0, Y2 = 0.0;
    for (int h = 0; h < kCarryGroups; ++h) {
      s_y[h][l][0] = Y1;
      s_y[h][l][1] = Y2;
      const Map& mp = s_map[h][l];
      const double n1 = mp.p1 + mp.u1 * Y1 + mp.w1 * Y2;
      const double n2 = mp.p2 + mp.u2 * Y1 + mp.w2 * Y2;
      Y1 = n1;
      Y2 = n2;
    }
  }
  __syncthreads();
  if (!live) return;
  double Y1 = s_y[g][l][0], Y2 = s_y[g][l][1];
  int i = i0;
  for (; i + 4 <= i1; i += 4) {
    Map m[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) m[j] = load_map(summ, B, chunk_at(i + j), k);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = chunk_at(i + j);
      init[(size_t)c * 2 * B + k] = (float)Y1;
      init[((size_t)c * 2 + 1) * B + k] = (float)Y2;
      const double n1 = m[j].p1 + m[j].u1 * Y1 + m[j].w1 * Y2;
      const double n2 = m[j].p2 + m[j].u2 * Y1 + m[j].w2 * Y2;
      Y1 = n1;
      Y2 = n2;
    }
  }
  for (; i < i1; ++i) {
    const int c = chunk_at(i);
    const Map mp = load_map(summ, B, c, k);
    init[(size_t)c * 2 * B + k] = (float)Y1;
    init[((size_t)c * 2 + 1) * B + k] = (float)Y2;
    const double n1 = mp.p1 + mp.u1 * Y1 + mp.w1 * Y2;
    const double n2 = mp.p2 + mp.u2 * Y1 + mp.w2 * Y2;
    Y1 = n1;
    Y2 = n2;
  }
}

// ADJ (with LOSS): the chunk's adjoint summary as well, the map that
// k_bq_adj_chunk forms by running the chunk backwards, accumulated forwards
// here from the values the replay has in hand.  Per frame the adjoint state
// (v1, v2) goes to A_n (v1, v2) + b_n g_n with A_n = [[-a1, 1], [-a2, 0]],
// b_n = (-a1, -a2) and g_n = 2 (y_n - tgt_n), so over the chunk (frames
// n0..n1-1, taken from n1-1 down) the state leaving is M (v1, v2) + z with
// M = A_n0 A_n0+1 ... A_n1-1 and z = sum_n P_n b_n g_n, P_n = A_n0 ... A_n-1:
// both are prefix products, and P_n b_n is the first column of P_n+1.  The
// summary [6][B] per chunk is (z, M e1, M e2) in fp64, as k_bq_adj_chunk's
// (v, u, w), so the separate backward pass over y and the target is not run.
template <bool MOD, bool LOSS, bool ADJ = false>
__global__ __launch_bounds__(kThreads) void k_bq_fwd(const float* __restrict__ x, const float* __restrict__ mod,
                                                     const float* __restrict__ prm, const float* __restrict__ init,
                                                     float* __restrict__ y, const float* __restrict__ tgt,
                                                     float* __restrict__ lossp, int B, int T, int L,
                                                     double* __restrict__ asumm) {
  static_assert(!ADJ || LOSS, "the adjoint summary needs the target");
  LaneChunk lc;
  if (!lane_chunk(prm, B, T, L, lc)) return;
  const int k = lc.k;
  float y1 = init[(size_t)lc.c * 2 * B + k], y2 = init[((size_t)lc.c * 2 + 1) * B + k];
  float x1 = lc.n0 >= 1 ? x[(size_t)(lc.n0 - 1) * B + k] : 0.0f;
  float x2 = lc.n0 >= 2 ? x[(size_t)(lc.n0 - 2) * B + k] : 0.0f;
  float ls = 0.0f;
  // adjoint prefix product P = [[p11, p12], [p21, p22]] and sum z
  double p11 = 1.0, p12 = 0.0, p21 = 0.0, p22 = 1.0, z1 = 0.0, z2 = 0.0;
  auto step = [&](int n, const float* v, float m) {
    const Coef K = coef(lc.base * m, lc.q, lc.rq);
    const float x0 = v[0];
    const float out = ((x2 * K.b0 + x1 * K.b1) + x0 * K.b0) - (y2 * K.a2 + y1 * K.a1);
    y[(size_t)n * B + k] = out;
    if constexpr (LOSS) {
      const float d = out - v[1];
      ls += d * d;
    }
    if constexpr (ADJ) {
      const double a1 = K.a1, a2 = K.a2;
      const double g = 2.0 * ((double)out - (double)v[1]);
      const double q1 = -a1 * p11 - a2 * p12, q2 = -a1 * p21 - a2 * p22;
      p12 = p11;
      p22 = p21;
      p11 = q1;
      p21 = q2;
      z1 += g * q1;
      z2 += g * q2;
    }
    y2 = y1;
    y1 = out;
    x2 = x1;
    x1 = x0;
  };
  if constexpr (LOSS) {
    const float* const src[2] = {x, tgt};
    walk_fwd<2, MOD>(src, mod, B, k, lc.n0, lc.n1, step);
    lossp[(size_t)lc.c * B + k] = ls;
    if constexpr (ADJ) {
      double* o = asumm + (size_t)lc.c * 6 * B + k;
      o[0] = z1;
      o[(size_t)B] = z2;
      o[(size_t)2 * B] = p11;
      o[(size_t)3 * B] = p21;
      o[(size_t)4 * B] = p12;
      o[(size_t)5 * B] = p22;
    }
  } else {
    const float* const src[1] = {x};
    walk_fwd<1, MOD>(src, mod, B, k, lc.n0, lc.n1, step);
  }
}

// ------------------------------------------------------------ adjoint scan
template <bool MOD>
__global__ __launch_bounds__(kThreads) void k_bq_adj_chunk(const float* __restrict__ mod, const float* __restrict__ prm,
                                                           const float* __restrict__ y,
                                                           const float* __restrict__ tgt, double* __restrict__ summ,
                                                           int B, int T, int L) {
  LaneChunk lc;
  if (!lane_chunk(prm, B, T, L, lc)) return;
  const int k = lc.k;
  double v1 = 0.0, v2 = 0.0, u1 = 1.0, u2 = 0.0, w1 = 0.0, w2 = 1.0;
  const float* const src[2] = {y, tgt};
  walk_rev<2, MOD>(src, mod, B, k, lc.n1, lc.n0, [&](int, const float* v, float m) {
    const Coef K = coef(lc.base * m, lc.q, lc.rq);
    const double a1 = K.a1, a2 = K.a2;
    const double lam = 2.0 * ((double)v[0] - (double)v[1]) + v1;
    v1 = v2 - a1 * lam;
    v2 = -a2 * lam;
    const double lu = u1;
    u1 = u2 - a1 * lu;
    u2 = -a2 * lu;
    const double lw = w1;
    w1 = w2 - a1 * lw;
    w2 = -a2 * lw;
  });
  double* o = summ + (size_t)lc.c * 6 * B + k;
  o[0] = v1;
  o[(size_t)B] = v2;
  o[(size_t)2 * B] = u1;
  o[(size_t)3 * B] = u2;
  o[(size_t)4 * B] = w1;
  o[(size_t)5 * B] = w2;
}

// Gradient partials of one (lane, chunk): the chain rule of the adjoint
// through the coefficient nodes (b0 = b2 = P r, b1 = D r, a1 = -2c r,
// a2 = (1 - alpha) r, r = 1/(1 + alpha), alpha = s/(2q), w = |base m| w0).
// gpart[c][0][k] = d/d base_k, gpart[c][1][k] = d/d Q_k over the chunk.
template <bool MOD>
__global__ __launch_bounds__(kThreads) void k_bq_bwd(const float* __restrict__ x, const float* __restrict__ mod,
                                                     const float* __restrict__ prm, const float* __restrict__ y,
                                                     const float* __restrict__ tgt, const float* __restrict__ ainit,
                                                     float* __restrict__ gpart, int B, int T, int L) {
  LaneChunk lc;
  if (!lane_chunk(prm, B, T, L, lc)) return;
  const int k = lc.k;
  float v1 = ainit[(size_t)lc.c * 2 * B + k], v2 = ainit[((size_t)lc.c * 2 + 1) * B + k];
  // shift registers: values at frames j+2 (a) and j+1 (b) while frame j streams in
  auto at = [&](const float* p, int n) { return n >= 0 ? p[(size_t)n * B + k] : 0.0f; };
  float xa = at(x, lc.n1 - 1), xb = at(x, lc.n1 - 2);
  float ya = at(y, lc.n1 - 1), yb = at(y, lc.n1 - 2);
  float ta = at(tgt, lc.n1 - 1), tb = at(tgt, lc.n1 - 2);
  float ma = MOD ? mod[lc.n1 - 1] : 1.0f;
  float mb = MOD ? (lc.n1 >= 2 ? mod[lc.n1 - 2] : 1.0f) : 1.0f;
  float Sw = 0.0f, Sq = 0.0f;
  const float* const src[3] = {x, y, tgt};
  walk_rev<3, MOD>(src, mod, B, k, lc.n1 - 2, lc.n0 - 2, [&](int, const float* v, float m) {
    // frame n = j + 2: x0 = x[n], x1 = x[n-1], x2 = x[n-2] (likewise y)
    const float x0 = xa, x1 = xb, x2 = v[0];
    const float y0 = ya, y1 = yb, y2 = v[1];
    const float fc = lc.base * ma;
    const Coef K = coef(fc, lc.q, lc.rq);
    const float lam = 2.0f * (y0 - ta) + v1;
    v1 = v2 - K.a1 * lam;
    v2 = -K.a2 * lam;
    const float gb02 = lam * (x0 + x2), gb1 = lam * x1, ga1 = -lam * y1, ga2 = -lam * y2;
    const float dr = gb02 * K.P + gb1 * K.D + ga1 * (-2.0f * K.c) + ga2 * (1.0f - K.alpha);
    const float dP = gb02 * K.r;
    const float dD = gb1 * K.r + 0.5f * dP;
    const float dc = -dD - 2.0f * K.r * ga1;
    const float dal = -ga2 * K.r - dr * K.r * K.r;
    const float ds = 0.5f * lc.rq * dal;
    const float dw = -K.s * dc + K.c * ds;
    Sw += dw * (MOD ? ma : 1.0f) * sign_of(fc);
    Sq += dal * K.alpha;
    xa = xb;
    xb = v[0];
    ya = yb;
    yb = v[1];
    ta = tb;
    tb = v[2];
    ma = mb;
    mb = m;
  });
  gpart[(size_t)lc.c * 2 * B + k] = Sw * kW0PerHz;
  gpart[((size_t)lc.c * 2 + 1) * B + k] = -Sq * lc.rq * lc.qsign;
}

struct BqShape {
  int64_t B, T, L, C;
};

int bq_shape(int64_t B, int64_t T, int64_t L, BqShape& s, const char* who) {
  DGEN_REQUIRE(B > 0 && B <= (1 << 20) && T > 0 && T < (1ll << 30) && L > 0 && L <= (1 << 20),
               "%s: B %lld T %lld L %lld", who, (long long)B, (long long)T, (long long)L);
  DGEN_REQUIRE(B * T < (1ll << 40), "%s: B*T too large", who);
  s = BqShape{B, T, L, (T + L - 1) / L};
  DGEN_REQUIRE(s.C <= 65535, "%s: %lld chunks exceeds the grid limit (raise the chunk length)", who,
               (long long)s.C);
  return 0;
}

double* dcell(const Launch& L, int64_t off) { return reinterpret_cast<double*>(cell(L, off)); }

dim3 bq_grid(const BqShape& s) { return dim3((unsigned)s.C, (unsigned)((s.B + kThreads - 1) / kThreads)); }

// Enqueue the three passes of the forward on raw device pointers (shared by
// the schedule's launchers and the no-allocation entry point).
void bq_enqueue_chunk(hipStream_t st, const float* x, const float* mod, const float* prm, double* summ,
                      const BqShape& s) {
  if (mod)
    hipLaunchKernelGGL(k_bq_chunk<true>, bq_grid(s), dim3(kThreads), 0, st, x, mod, prm, summ, (int)s.B, (int)s.T,
                       (int)s.L);
  else
    hipLaunchKernelGGL(k_bq_chunk<false>, bq_grid(s), dim3(kThreads), 0, st, x, nullptr, prm, summ, (int)s.B,
                       (int)s.T, (int)s.L);
}
void bq_enqueue_carry(hipStream_t st, const double* summ, float* init, int64_t B, int64_t C, int rev) {
  hipLaunchKernelGGL(k_bq_carry, dim3((unsigned)((B + kCarryLanes - 1) / kCarryLanes)),
                     dim3(kCarryLanes * kCarryGroups), 0, st, summ, init, (int)B, (int)C, rev);
}
void bq_enqueue_fwd(hipStream_t st, const float* x, const float* m, const float* prm, const float* init, float* y,
                    const float* t, float* lp, const BqShape& s, double* asumm = nullptr) {
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, bq_grid(s), dim3(kThreads), 0, st, x, m, prm, init, y, t, lp, (int)s.B, (int)s.T,
                       (int)s.L, asumm);
  };
  if (m && t && asumm) go(k_bq_fwd<true, true, true>);
  else if (t && asumm) go(k_bq_fwd<false, true, true>);
  else if (m && t) go(k_bq_fwd<true, true>);
  else if (m) go(k_bq_fwd<true, false>);
  else if (t) go(k_bq_fwd<false, true>);
  else go(k_bq_fwd<false, false>);
}

}  // namespace

int launch_biquad_chunk(const Launch& L, const dgen_hip_op& op) {
  const int64_t x = op.arg[0], mod = op.arg[1], prm = op.arg[2], summ = op.arg[3];
  BqShape s;
  if (int rc = bq_shape(op.arg[4], op.arg[5], op.arg[6], s, "biquad_chunk")) return rc;
  DGEN_CHECK_CELL(L, x, s.B * s.T, "biquad_chunk.x");
  if (mod >= 0) DGEN_CHECK_CELL(L, mod, s.T, "biquad_chunk.mod");
  DGEN_CHECK_CELL(L, prm, 2 * s.B, "biquad_chunk.params");
  DGEN_CHECK_CELL(L, summ, 12 * s.C * s.B, "biquad_chunk.summary");
  DGEN_REQUIRE(summ % 2 == 0, "biquad_chunk: summary cell must be 8-byte aligned");
  if (L.dry) return 0;
  bq_enqueue_chunk(L.stream, cell(L, x), mod >= 0 ? cell(L, mod) : nullptr, cell(L, prm), dcell(L, summ), s);
  DGEN_LAUNCH_CHECK("k_bq_chunk");
  return 0;
}

int launch_biquad_carry(const Launch& L, const dgen_hip_op& op) {
  const int64_t summ = op.arg[0], init = op.arg[1], B = op.arg[2], C = op.arg[3], rev = op.arg[4];
  DGEN_REQUIRE(B > 0 && B <= (1 << 20) && C > 0 && C <= 65535 && (rev == 0 || rev == 1),
               "biquad_carry: B %lld C %lld reverse %lld", (long long)B, (long long)C, (long long)rev);
  DGEN_CHECK_CELL(L, summ, 12 * C * B, "biquad_carry.summary");
  DGEN_REQUIRE(summ % 2 == 0, "biquad_carry: summary cell must be 8-byte aligned");
  DGEN_CHECK_CELL(L, init, 2 * C * B, "biquad_carry.init");
  if (L.dry) return 0;
  bq_enqueue_carry(L.stream, dcell(L, summ), cell(L, init), B, C, (int)rev);
  DGEN_LAUNCH_CHECK("k_bq_carry");
  return 0;
}

int launch_biquad_fwd(const Launch& L, const dgen_hip_op& op) {
  const int64_t x = op.arg[0], mod = op.arg[1], prm = op.arg[2], init = op.arg[3], y = op.arg[4];
  const int64_t tgt = op.arg[8], lossp = op.arg[9];
  BqShape s;
  if (int rc = bq_shape(op.arg[5], op.arg[6], op.arg[7], s, "biquad_fwd")) return rc;
  DGEN_CHECK_CELL(L, x, s.B * s.T, "biquad_fwd.x");
  if (mod >= 0) DGEN_CHECK_CELL(L, mod, s.T, "biquad_fwd.mod");
  DGEN_CHECK_CELL(L, prm, 2 * s.B, "biquad_fwd.params");
  DGEN_CHECK_CELL(L, init, 2 * s.C * s.B, "biquad_fwd.init");
  DGEN_CHECK_CELL(L, y, s.B * s.T, "biquad_fwd.y");
  DGEN_REQUIRE((tgt >= 0) == (lossp >= 0), "biquad_fwd: target and loss partials go together");
  if (tgt >= 0) {
    DGEN_CHECK_CELL(L, tgt, s.B * s.T, "biquad_fwd.target");
    DGEN_CHECK_CELL(L, lossp, s.C * s.B, "biquad_fwd.loss_partials");
  }
  // arg[11] = 1: the adjoint chunk summaries too, into arg[10]
  const bool adj = op.arg[11] == 1;
  const int64_t asumm = op.arg[10];
  DGEN_REQUIRE(op.arg[11] == 0 || adj, "biquad_fwd: arg[11] %lld (0, or 1 with adjoint summaries)",
               (long long)op.arg[11]);
  if (adj) {
    DGEN_REQUIRE(tgt >= 0, "biquad_fwd: adjoint summaries need the target");
    DGEN_REQUIRE(asumm % 2 == 0, "biquad_fwd: summary cell must be 8-byte aligned");
    DGEN_CHECK_CELL(L, asumm, 12 * s.C * s.B, "biquad_fwd.adjoint_summary");
  }
  if (L.dry) return 0;
  bq_enqueue_fwd(L.stream, cell(L, x), mod >= 0 ? cell(L, mod) : nullptr, cell(L, prm), cell(L, init), cell(L, y),
                 tgt >= 0 ? cell(L, tgt) : nullptr, lossp >= 0 ? cell(L, lossp) : nullptr, s,
                 adj ? dcell(L, asumm) : nullptr);
  DGEN_LAUNCH_CHECK("k_bq_fwd");
  return 0;
}

int launch_biquad_adj_chunk(const Launch& L, const dgen_hip_op& op) {
  const int64_t mod = op.arg[0], prm = op.arg[1], y = op.arg[2], tgt = op.arg[3], summ = op.arg[4];
  BqShape s;
  if (int rc = bq_shape(op.arg[5], op.arg[6], op.arg[7], s, "biquad_adj_chunk")) return rc;
  if (mod >= 0) DGEN_CHECK_CELL(L, mod, s.T, "biquad_adj_chunk.mod");
  DGEN_CHECK_CELL(L, prm, 2 * s.B, "biquad_adj_chunk.params");
  DGEN_CHECK_CELL(L, y, s.B * s.T, "biquad_adj_chunk.y");
  DGEN_CHECK_CELL(L, tgt, s.B * s.T, "biquad_adj_chunk.target");
  DGEN_CHECK_CELL(L, summ, 12 * s.C * s.B, "biquad_adj_chunk.summary");
  DGEN_REQUIRE(summ % 2 == 0, "biquad_adj_chunk: summary cell must be 8-byte aligned");
  if (L.dry) return 0;
  if (mod >= 0)
    hipLaunchKernelGGL(k_bq_adj_chunk<true>, bq_grid(s), dim3(kThreads), 0, L.stream, cell(L, mod), cell(L, prm),
                       cell(L, y), cell(L, tgt), dcell(L, summ), (int)s.B, (int)s.T, (int)s.L);
  else
    hipLaunchKernelGGL(k_bq_adj_chunk<false>, bq_grid(s), dim3(kThreads), 0, L.stream, nullptr, cell(L, prm),
                       cell(L, y), cell(L, tgt), dcell(L, summ), (int)s.B, (int)s.T, (int)s.L);
  DGEN_LAUNCH_CHECK("k_bq_adj_chunk");
  return 0;
}

int launch_biquad_bwd(const Launch& L, const dgen_hip_op& op) {
  const int64_t x = op.arg[0], mod = op.arg[1], prm = op.arg[2], y = op.arg[3], tgt = op.arg[4],
                ainit = op.arg[5], gpart = op.arg[6];
  BqShape s;
  if (int rc = bq_shape(op.arg[7], op.arg[8], op.arg[9], s, "biquad_bwd")) return rc;
  DGEN_CHECK_CELL(L, x, s.B * s.T, "biquad_bwd.x");
  if (mod >= 0) DGEN_CHECK_CELL(L, mod, s.T, "biquad_bwd.mod");
  DGEN_CHECK_CELL(L, prm, 2 * s.B, "biquad_bwd.params");
  DGEN_CHECK_CELL(L, y, s.B * s.T, "biquad_bwd.y");
  DGEN_CHECK_CELL(L, tgt, s.B * s.T, "biquad_bwd.target");
  DGEN_CHECK_CELL(L, ainit, 2 * s.C * s.B, "biquad_bwd.adjoint_init");
  DGEN_CHECK_CELL(L, gpart, 2 * s.C * s.B, "biquad_bwd.grad_partials");
  if (L.dry) return 0;
  if (mod >= 0)
    hipLaunchKernelGGL(k_bq_bwd<true>, bq_grid(s), dim3(kThreads), 0, L.stream, cell(L, x), cell(L, mod),
                       cell(L, prm), cell(L, y), cell(L, tgt), cell(L, ainit), cell(L, gpart), (int)s.B, (int)s.T,
                       (int)s.L);
  else
    hipLaunchKernelGGL(k_bq_bwd<false>, bq_grid(s), dim3(kThreads), 0, L.stream, cell(L, x), nullptr, cell(L, prm),
                       cell(L, y), cell(L, tgt), cell(L, ainit), cell(L, gpart), (int)s.B, (int)s.T, (int)s.L);
  DGEN_LAUNCH_CHECK("k_bq_bwd");
  return 0;
}

// ---- streaming bank: one thread per lane, history carried between runs ----
// The reference's per-lane frame loop (StatefulTensorParallelPolicy.swift:
// 21-74): lane k steps Direct Form I frame by frame in registers from the
// history cells state[4][B] (x[n-1], x[n-2], y[n-1], y[n-2]) and writes them
// back, so any split of a run into runs gives the same samples; frames are
// read and written [frame][lane] (a wave's 64 lanes are 256 contiguous
// bytes).  Out stores map non-finite values to 0 (CRenderer.swift:1021-1039).
template <bool MOD>
__global__ __launch_bounds__(kThreads) void k_stream_bq(const float* __restrict__ x, const float* __restrict__ mod,
                                                        const float* __restrict__ prm, float* __restrict__ state,
                                                        float* __restrict__ y, int B, int T, int reset) {
  const int k = blockIdx.x * kThreads + threadIdx.x;
  if (k >= B) return;
  const float base = prm[k], q = fabsf(prm[B + k]), rq = 1.0f / q;
  float x1 = 0.f, x2 = 0.f, y1 = 0.f, y2 = 0.f;
  if (!reset) {
    x1 = state[k];
    x2 = state[B + k];
    y1 = state[2 * B + k];
    y2 = state[3 * B + k];
  }
  const float* const src[1] = {x};
  walk_fwd<1, MOD>(src, mod, B, k, 0, T, [&](int n, const float* v, float m) {
    const Coef K = coef(base * m, q, rq);
    const float x0 = v[0];
    const float out = ((x2 * K.b0 + x1 * K.b1) + x0 * K.b0) - (y2 * K.a2 + y1 * K.a1);
    y[(size_t)n * B + k] = isfinite(out) ? out : 0.f;
    y2 = y1;
    y1 = out;
    x2 = x1;
    x1 = x0;
  });
  state[k] = x1;
  state[B + k] = x2;
  state[2 * B + k] = y1;
  state[3 * B + k] = y2;
}

int launch_stream_biquad(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=x ([frames][B]) [1]=mod ([frames]) or -1 [2]=params ([2][B]) [3]=state ([4][B]) [4]=y ([frames][B])
  //      [5]=B [6]=frames (capacity)
  const int64_t x = op.arg[0], mod = op.arg[1], prm = op.arg[2], st = op.arg[3], y = op.arg[4], B = op.arg[5],
                T = op.arg[6];
  DGEN_REQUIRE(B > 0 && B <= (1 << 20) && T > 0 && T < (1ll << 30) && B * T < (1ll << 40),
               "stream_biquad: B %lld frames %lld", (long long)B, (long long)T);
  DGEN_CHECK_CELL(L, x, B * T, "stream_biquad.x");
  if (mod >= 0) DGEN_CHECK_CELL(L, mod, T, "stream_biquad.mod");
  DGEN_CHECK_CELL(L, prm, 2 * B, "stream_biquad.params");
  DGEN_CHECK_CELL(L, st, 4 * B, "stream_biquad.state");
  DGEN_CHECK_CELL(L, y, B * T, "stream_biquad.y");
  if (L.dry) return 0;
  const int64_t n = std::min<int64_t>(T, L.frames ? (int64_t)L.frames : T);
  const dim3 grid((unsigned)((B + kThreads - 1) / kThreads));
  if (mod >= 0)
    hipLaunchKernelGGL(k_stream_bq<true>, grid, dim3(kThreads), 0, L.stream, cell(L, x), cell(L, mod), cell(L, prm),
                       cell(L, st), cell(L, y), (int)B, (int)n, L.reset ? 1 : 0);
  else
    hipLaunchKernelGGL(k_stream_bq<false>, grid, dim3(kThreads), 0, L.stream, cell(L, x), nullptr, cell(L, prm),
                       cell(L, st), cell(L, y), (int)B, (int)n, L.reset ? 1 : 0);
  DGEN_LAUNCH_CHECK("k_stream_bq");
  return 0;
}

// ---- the bank forward without allocation -----------------------------------
// The chunk summaries ([C][6][B] fp64) and chunk initial states ([C][2][B]
// fp32) of dgen_hip_biquad_forward_noalloc live in this fixed device array
// (each GPU the library runs on holds its own copy until the process ends).
// Host code never passes the array's name to a kernel: it is a host-side
// stand-in, not a device address.  Each device's address comes from
// hipGetSymbolAddress on that call's first use of the device, with the
// device current.
constexpr int64_t kNoAllocScratchBytes = 16ll << 20;
static __device__ __align__(256) double scratch[kNoAllocScratchBytes / sizeof(double)];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int scratch_on(int device, void** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(DGEN_HIP_E_DEVICE, "biquad_forward_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", device,
                  hipGetErrorString(e));
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return 0;
}
}  // namespace

}  // namespace dgen

extern "C" int dgen_hip_biquad_forward_noalloc(int device, const float* x, const float* mod, const float* params,
                                               float* y, uint32_t B, uint32_t T, uint32_t chunk, void* stream) {
  using namespace dgen;
  if (!x || !params || !y) return fail(DGEN_HIP_E_INVALID, "biquad_forward_noalloc: null x, params or y");
  const uint32_t L = chunk ? chunk : 256;
  BqShape s;
  if (int rc = bq_shape(B, T, L, s, "biquad_forward_noalloc")) return rc;
  const int64_t need = (int64_t)sizeof(double) * 6 * s.C * s.B + (int64_t)sizeof(float) * 2 * s.C * s.B;
  if (need > kNoAllocScratchBytes)
    return fail(DGEN_HIP_E_RANGE,
                "biquad_forward_noalloc: B=%u lanes x %lld chunks need %lld bytes of scratch; the fixed scratch holds "
                "%lld (lanes x ceil(T/chunk) <= %lld; raise the chunk length or split the bank)",
                B, (long long)s.C, (long long)need, (long long)kNoAllocScratchBytes,
                (long long)(kNoAllocScratchBytes / 56));
  int n = 0, prev = 0;
  DGEN_HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n || device >= kMaxScratchDevices)
    return fail(DGEN_HIP_E_INVALID, "biquad_forward_noalloc: device %d of %d", device, n);
  DGEN_HIP_TRY(hipGetDevice(&prev));
  DGEN_HIP_TRY(hipSetDevice(device));
  void* base = nullptr;
  int rc = scratch_on(device, &base);
  if (!rc) {
    double* summ = static_cast<double*>(base);
    float* init = reinterpret_cast<float*>(summ + 6 * s.C * s.B);
    hipStream_t st = static_cast<hipStream_t>(stream);
    bq_enqueue_chunk(st, x, mod, params, summ, s);
    bq_enqueue_carry(st, summ, init, s.B, s.C, 0);
    bq_enqueue_fwd(st, x, mod, params, init, y, nullptr, nullptr, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      rc = fail(DGEN_HIP_E_DEVICE, "biquad_forward_noalloc: launch failed: %s", hipGetErrorString(e));
  }
  (void)hipSetDevice(prev);
  return rc;
}
