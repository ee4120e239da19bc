// 2D membrane (damped wave equation with the 3x3 zero-padded Laplacian),
// forward and discrete adjoint.
//
// Reference: the TensorHistory idiom of Examples/BendingMetal/main.swift:
// 96-169 (state read, pad + conv2d Laplacian, update, history writes, pickup
// of the new state); conv2d "same" semantics Sources/DGen/Emit+Tensor.swift:
// 173-205; tensor history Sources/DGen/Tensor.swift:1253-1320.  The
// reference runs this as a sequential frame loop over the whole grid per
// frame (FeedbackAnalysis.swift:354-362) and has no adjoint for conv2d.
//
// State store S (in HBM, one field per frame): S[0] = u_{-1}, S[1] = u_0,
// S[n+1] = u_n, so the backward reads every forward state instead of
// recomputing it (4801 fields of 1 MB at 512^2 x 4800).
//
// Temporal blocking: a workgroup owns a kTile x kTile tile and keeps a
// kSide x kSide region (the tile plus a kHalo ring) of the two live fields
// in LDS.  One launch advances ks <= kHalo steps: step s is valid on a band
// that shrinks by one cell per step, so after ks steps the owned tile is
// exact and no workgroup needs another's data until the next launch.  The
// update is in place: u_{n+1}[i] overwrites u_{n-1}[i] (only that cell
// reads it), so one workgroup barrier per step suffices.
//
// Adjoint (L is symmetric): lambda_n = g_n + (2-d) lambda_{n+1}
// + c2 L lambda_{n+1} - (1-d) lambda_{n+2}, g_n = 2 (out[n-1] - tgt[n-1]) at
// the pickup; the same blocked stencil backwards in time, with the
// gradient terms dL/dc2 = sum <L lambda_n, u_{n-1}> and
// dL/dd = sum <lambda_n, u_{n-2} - u_{n-1}> accumulated over the owned cells
// from the stored states.
#include "internal.h"

namespace dgen {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 32;
constexpr int kHalo = 16;
constexpr int kSide = kTile + 2 * kHalo;  // 64
constexpr int kCells = kSide * kSide / kThreads;  // 16 cells per thread
static_assert(kSide == 64, "thread mapping assumes a 64-wide region");

struct MemArgs {
  float* S;           // state store [(T + 2)][R][C]
  const float* prm;   // (c2, d)
  float* out;         // pickup [T]
  const float* tgt;   // target pickup [T] (backward)
  float* lam;         // adjoint boundary fields: 2 sets x (lambda_{m+1}, lambda_{m+2}) x [R][C]
  double* gpart;      // [tiles][2] gradient partials (fp64: the terms cancel heavily)
  int R, C, T, py, px;
};

// Cell j of thread t: column t & 63, row (t >> 6) + 4 j.
__device__ __forceinline__ int cell_row(int j) { return (threadIdx.x >> 6) + 4 * j; }
__device__ __forceinline__ int cell_col() { return threadIdx.x & 63; }

__device__ __forceinline__ float lap5(const float* f, int i) {
  return (((f[i - kSide] + f[i - 1]) + f[i] * -4.0f) + f[i + 1]) + f[i + kSide];
}

// Loads the region of fields a (-> A) and b (-> B) around the tile; cells
// outside the grid are zero (the conv2d zero padding) and stay zero.
__device__ __forceinline__ void load_region(const MemArgs& a, const float* fa, const float* fb, float* A, float* B,
                                            int ry0, int rx0) {
  const int c = cell_col(), gx = rx0 + c;
  const bool cin = gx >= 0 && gx < a.C;
#pragma unroll
  for (int j = 0; j < kCells; ++j) {
    const int r = cell_row(j), gy = ry0 + r;
    const bool in = cin && gy >= 0 && gy < a.R;
    const size_t gi = in ? (size_t)gy * a.C + gx : 0;
    A[r * kSide + c] = (in && fa) ? fa[gi] : 0.0f;
    B[r * kSide + c] = (in && fb) ? fb[gi] : 0.0f;
  }
}

// Forward: frames n0 .. n0+ks-1 (u_{n0+1} .. u_{n0+ks}).
__global__ __launch_bounds__(kThreads) void k_mem_fwd(MemArgs a, int n0, int ks) {
  __shared__ float f[2][kSide * kSide];
  const int y0 = blockIdx.y * kTile, x0 = blockIdx.x * kTile;
  const int ry0 = y0 - kHalo, rx0 = x0 - kHalo;
  const size_t G = (size_t)a.R * a.C;
  const float c2 = a.prm[0], d = a.prm[1];
  float* cur = f[0];
  float* prv = f[1];
  load_region(a, a.S + (size_t)(n0 + 1) * G, a.S + (size_t)n0 * G, cur, prv, ry0, rx0);
  const int c = cell_col(), gx = rx0 + c;
  const bool cin = gx >= 0 && gx < a.C;
  __syncthreads();
  for (int s = 0; s < ks; ++s) {
    const int lo = kHalo + 1 - ks + s, hi = kHalo + kTile - 1 + ks - s;
    if (cin && c >= lo && c < hi) {
#pragma unroll
      for (int j = 0; j < kCells; ++j) {
        const int r = cell_row(j), gy = ry0 + r;
        if (r < lo || r >= hi || gy < 0 || gy >= a.R) continue;
        const int i = r * kSide + c;
        const float u = cur[i], u1 = prv[i];
        const float b = u * 2.0f - u1;
        const float cc = lap5(cur, i) * c2;
        const float g = (u - u1) * d;
        prv[i] = (b + cc) - g;
      }
    }
    lds_barrier();
    float* t = cur;
    cur = prv;
    prv = t;
    // owned cells of u_{n0+s+1} -> S[n0+s+2]; the pickup -> out[n0+s]
    if (cin && c >= kHalo && c < kHalo + kTile) {
      float* dst = a.S + (size_t)(n0 + s + 2) * G;
#pragma unroll
      for (int j = 0; j < kCells; ++j) {
        const int r = cell_row(j), gy = ry0 + r;
        if (r < kHalo || r >= kHalo + kTile || gy >= a.R) continue;
        const float v = cur[r * kSide + c];
        dst[(size_t)gy * a.C + gx] = v;
        if (gy == a.py && gx == a.px) a.out[n0 + s] = v;
      }
    }
  }
}

// Backward: adjoint steps n = m_hi .. m_hi-ks+1 (n >= 0), from
// (lambda_{m_hi+1}, lambda_{m_hi+2}) in lam set `src` (zero when src < 0) to
// set `dst`.  Step n computes lambda_n and, from the same stencil pass, the
// gradient terms of lambda_{n+1} (L symmetric: <lambda, L u> = <L lambda, u>):
//   dc2 += L(lambda_{n+1}) u_n,  dd += lambda_{n+1} (u_{n-1} - u_n)
// over the owned cells, whose two state values are prefetched a step ahead.
// The schedule runs n down to 0 so that lambda_1's terms are included.
__global__ __launch_bounds__(kThreads) void k_mem_bwd(MemArgs a, int m_hi, int ks, int src, int dst, int first) {
  __shared__ float f[2][kSide * kSide];
  __shared__ double red[2][kThreads / 64];
  constexpr int kOwn = kTile / 4;  // owned cells per owning thread: rows j = 4 .. 11
  const int y0 = blockIdx.y * kTile, x0 = blockIdx.x * kTile;
  const int ry0 = y0 - kHalo, rx0 = x0 - kHalo;
  const size_t G = (size_t)a.R * a.C;
  const float c2 = a.prm[0], d = a.prm[1];
  const float ad = 2.0f - d, bd = 1.0f - d;
  float* cur = f[0];  // lambda_{n+1}
  float* prv = f[1];  // lambda_{n+2}
  const float* ls = src >= 0 ? a.lam + (size_t)src * 2 * G : nullptr;
  load_region(a, ls, ls ? ls + G : nullptr, cur, prv, ry0, rx0);
  const int c = cell_col(), gx = rx0 + c;
  const bool cin = gx >= 0 && gx < a.C;
  const bool own_col = cin && c >= kHalo && c < kHalo + kTile;
  // owned cell q = row (t >> 6) + 4 (q + 4): grid index, or -1 outside the grid
  size_t gi[kOwn];
  bool gin[kOwn];
#pragma unroll
  for (int q = 0; q < kOwn; ++q) {
    const int gy = ry0 + cell_row(q + 4);
    gin[q] = own_col && gy < a.R;
    gi[q] = gin[q] ? (size_t)gy * a.C + gx : 0;
  }
  float ua[kOwn], ub[kOwn];  // u_n, u_{n-1} at the owned cells for the current step
  auto fetch = [&](int n, float* va, float* vb) {
    const float* sa = a.S + (size_t)(n + 1) * G;
    const float* sb = a.S + (size_t)n * G;
#pragma unroll
    for (int q = 0; q < kOwn; ++q) {
      va[q] = gin[q] ? sa[gi[q]] : 0.0f;
      vb[q] = gin[q] ? sb[gi[q]] : 0.0f;
    }
  };
  fetch(m_hi, ua, ub);
  double gc = 0.0, gd = 0.0;
  __syncthreads();
  for (int s = 0; s < ks; ++s) {
    const int n = m_hi - s;
    float na[kOwn], nb[kOwn];
    if (s + 1 < ks) fetch(n - 1, na, nb);
    const int lo = kHalo + 1 - ks + s, hi = kHalo + kTile - 1 + ks - s;
    const float src_val = n >= 1 ? 2.0f * (a.out[n - 1] - a.tgt[n - 1]) : 0.0f;
    if (cin && c >= lo && c < hi) {
#pragma unroll
      for (int j = 0; j < kCells; ++j) {
        const int r = cell_row(j), gy = ry0 + r;
        if (r < lo || r >= hi || gy < 0 || gy >= a.R) continue;
        const int i = r * kSide + c;
        const float lap = lap5(cur, i);
        float lam = (ad * cur[i] + c2 * lap) - bd * prv[i];
        if (gy == a.py && gx == a.px) lam += src_val;
        if (j >= 4 && j < 4 + kOwn && own_col) {
          gc += (double)(lap * ua[j - 4]);
          gd += (double)(cur[i] * (ub[j - 4] - ua[j - 4]));
        }
        prv[i] = lam;
      }
    }
    lds_barrier();
    float* t = cur;
    cur = prv;
    prv = t;
    if (s + 1 < ks) {
#pragma unroll
      for (int q = 0; q < kOwn; ++q) {
        ua[q] = na[q];
        ub[q] = nb[q];
      }
    }
  }
  // boundary adjoint fields of this launch: (lambda_{m_lo}, lambda_{m_lo+1}) -> set dst
  if (own_col) {
    float* o = a.lam + (size_t)dst * 2 * G;
#pragma unroll
    for (int q = 0; q < kOwn; ++q) {
      if (!gin[q]) continue;
      const int i = cell_row(q + 4) * kSide + c;
      o[gi[q]] = cur[i];
      o[G + gi[q]] = prv[i];
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    gc += __shfl_xor(gc, off, 64);
    gd += __shfl_xor(gd, off, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x >> 6] = gc;
    red[1][threadIdx.x >> 6] = gd;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double sc = 0.0, sd = 0.0;
    for (int w = 0; w < kThreads / 64; ++w) {
      sc += red[0][w];
      sd += red[1][w];
    }
    double* gp = a.gpart + 2 * (blockIdx.y * gridDim.x + blockIdx.x);
    gp[0] = first ? sc : gp[0] + sc;
    gp[1] = first ? sd : gp[1] + sd;
  }
}

// S[0] = S[1] = u0 (u_{-1} = u_0).
__global__ void k_mem_init(const float* __restrict__ u0, float* __restrict__ S, size_t G) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < G; i += (size_t)gridDim.x * blockDim.x) {
    const float v = u0[i];
    S[i] = v;
    S[G + i] = v;
  }
}

// grads[q] = sum over tiles of the fp64 partials, in tile order.
__global__ void k_mem_grad_final(const double* __restrict__ gpart, float* __restrict__ grads, int tiles) {
  if (threadIdx.x < 2) {
    double t = 0.0;
    for (int i = 0; i < tiles; ++i) t += gpart[2 * i + threadIdx.x];
    grads[threadIdx.x] = (float)t;
  }
}

// lt[n] = (out[n] - tgt[n])^2
__global__ void k_mem_loss_terms(const float* __restrict__ out, const float* __restrict__ tgt, float* __restrict__ lt,
                                 int T) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n < T) {
    const float e = out[n] - tgt[n];
    lt[n] = e * e;
  }
}

int mem_shape(int64_t R, int64_t C, int64_t T, int64_t py, int64_t px, int64_t ks, const char* who) {
  DGEN_REQUIRE(R > 0 && C > 0 && R <= 16384 && C <= 16384 && T > 0 && T < (1 << 28),
               "%s: grid %lld x %lld, T %lld", who, (long long)R, (long long)C, (long long)T);
  DGEN_REQUIRE(py >= 0 && py < R && px >= 0 && px < C, "%s: pickup (%lld, %lld) outside the grid", who,
               (long long)py, (long long)px);
  DGEN_REQUIRE(ks >= 1 && ks <= kHalo, "%s: steps per launch %lld not in [1, %d]", who, (long long)ks, kHalo);
  return 0;
}

}  // namespace

int launch_membrane_fwd(const Launch& L, const dgen_hip_op& op) {
  const int64_t S = op.arg[0], u0 = op.arg[1], prm = op.arg[2], out = op.arg[3];
  const int64_t R = op.arg[4], C = op.arg[5], T = op.arg[6], py = op.arg[7], px = op.arg[8], ks = op.arg[9];
  if (int rc = mem_shape(R, C, T, py, px, ks, "membrane_fwd")) return rc;
  const int64_t G = R * C;
  DGEN_CHECK_CELL(L, S, (T + 2) * G, "membrane_fwd.states");
  DGEN_CHECK_CELL(L, u0, G, "membrane_fwd.u0");
  DGEN_CHECK_CELL(L, prm, 2, "membrane_fwd.params");
  DGEN_CHECK_CELL(L, out, T, "membrane_fwd.pickup");
  if (L.dry) return 0;
  MemArgs a{};
  a.S = cell(L, S);
  a.prm = cell(L, prm);
  a.out = cell(L, out);
  a.R = (int)R;
  a.C = (int)C;
  a.T = (int)T;
  a.py = (int)py;
  a.px = (int)px;
  const unsigned ib = (unsigned)std::min<int64_t>((G + 255) / 256, (int64_t)L.cu_count * 8);
  hipLaunchKernelGGL(k_mem_init, dim3(ib), dim3(256), 0, L.stream, cell(L, u0), a.S, (size_t)G);
  DGEN_LAUNCH_CHECK("k_mem_init");
  const dim3 grid((unsigned)((C + kTile - 1) / kTile), (unsigned)((R + kTile - 1) / kTile));
  for (int64_t n0 = 0; n0 < T; n0 += ks) {
    hipLaunchKernelGGL(k_mem_fwd, grid, dim3(kThreads), 0, L.stream, a, (int)n0, (int)std::min<int64_t>(ks, T - n0));
    DGEN_LAUNCH_CHECK("k_mem_fwd");
  }
  return 0;
}

int launch_membrane_bwd(const Launch& L, const dgen_hip_op& op) {
  const int64_t S = op.arg[0], prm = op.arg[1], out = op.arg[2], tgt = op.arg[3], lam = op.arg[4], gpart = op.arg[5],
                lt = op.arg[6], grads = op.arg[13];
  const int64_t R = op.arg[7], C = op.arg[8], T = op.arg[9], py = op.arg[10], px = op.arg[11], ks = op.arg[12];
  if (int rc = mem_shape(R, C, T, py, px, ks, "membrane_bwd")) return rc;
  const int64_t G = R * C;
  const int64_t tiles = ((R + kTile - 1) / kTile) * ((C + kTile - 1) / kTile);
  DGEN_CHECK_CELL(L, S, (T + 2) * G, "membrane_bwd.states");
  DGEN_CHECK_CELL(L, prm, 2, "membrane_bwd.params");
  DGEN_CHECK_CELL(L, out, T, "membrane_bwd.pickup");
  DGEN_CHECK_CELL(L, tgt, T, "membrane_bwd.target");
  DGEN_CHECK_CELL(L, lam, 4 * G, "membrane_bwd.adjoint_fields");
  DGEN_CHECK_CELL(L, gpart, 4 * tiles, "membrane_bwd.grad_partials");
  DGEN_REQUIRE(gpart % 2 == 0, "membrane_bwd: grad partials cell must be 8-byte aligned");
  DGEN_CHECK_CELL(L, grads, 2, "membrane_bwd.grads");
  DGEN_CHECK_CELL(L, lt, T, "membrane_bwd.loss_terms");
  if (L.dry) return 0;
  MemArgs a{};
  a.S = cell(L, S);
  a.prm = cell(L, prm);
  a.out = cell(L, out);
  a.tgt = cell(L, tgt);
  a.lam = cell(L, lam);
  a.gpart = reinterpret_cast<double*>(cell(L, gpart));
  a.R = (int)R;
  a.C = (int)C;
  a.T = (int)T;
  a.py = (int)py;
  a.px = (int)px;
  hipLaunchKernelGGL(k_mem_loss_terms, dim3((unsigned)((T + 255) / 256)), dim3(256), 0, L.stream, a.out, a.tgt,
                     cell(L, lt), (int)T);
  DGEN_LAUNCH_CHECK("k_mem_loss_terms");
  const dim3 grid((unsigned)((C + kTile - 1) / kTile), (unsigned)((R + kTile - 1) / kTile));
  int src = -1, dst = 0;
  bool first = true;
  for (int64_t m_hi = T; m_hi >= 0; m_hi -= ks) {
    const int n = (int)std::min<int64_t>(ks, m_hi + 1);
    hipLaunchKernelGGL(k_mem_bwd, grid, dim3(kThreads), 0, L.stream, a, (int)m_hi, n, src, dst, first ? 1 : 0);
    DGEN_LAUNCH_CHECK("k_mem_bwd");
    src = dst;
    dst ^= 1;
    first = false;
  }
  hipLaunchKernelGGL(k_mem_grad_final, dim3(1), dim3(64), 0, L.stream, a.gpart, cell(L, grads), (int)tiles);
  DGEN_LAUNCH_CHECK("k_mem_grad_final");
  return 0;
}

}  // namespace dgen
