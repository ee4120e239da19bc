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
// Temporal blocking: a workgroup owns a kTile x kTile tile and advances a
// kSide x kSide region around it (the tile plus a kHalo ring where the grid
// allows) of the two live fields.  One launch advances ks <= kHalo steps:
// values next to a region edge that lies inside the grid go wrong (their
// outside neighbours read as zero) but the error front moves one cell per
// step, so after ks steps the owned tile is still exact and no workgroup
// needs another's data until the next launch.  On grids of at least kSide
// cells each way the region is placed inside the grid: a region edge that is
// a grid edge then reads the exact zero padding and no cell needs a mask.
// Smaller grids centre the region on the tile and zero the cells outside the
// grid by a per-row mask.
//
// Register strips: the region is 64 columns wide, one per wavefront lane;
// wave w holds rows kRows*w .. kRows*w + kRows - 1 of its lane's column for
// both live fields in registers.  Vertical neighbours come from the thread's
// own registers (the strip's first and last rows from the waves above and
// below, through a small double-buffered LDS edge table: one barrier per
// step); horizontal neighbours from the adjacent lanes by DPP wave shifts.
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

constexpr int kTile = 32;
constexpr int kHalo = 16;
constexpr int kSide = kTile + 2 * kHalo;  // 64: one wavefront lane per region column
constexpr int kRows = 4;                  // region rows per thread (four waves per SIMD)
constexpr int kWaves = kSide / kRows;
constexpr int kThreads = 64 * kWaves;
static_assert(kSide == 64, "one region column per wavefront lane");

struct MemArgs {
  float* S;           // state store [(T + 2)][R][C]
  const float* prm;   // (c2, d)
  float* out;         // pickup [T]
  const float* tgt;   // target pickup [T] (backward)
  float* lam;         // adjoint boundary fields: 2 sets x (lambda_{m+1}, lambda_{m+2}) x [R][C]
  double* gpart;      // [tiles][kWaves][2] gradient partials (fp64: the terms cancel heavily)
  int R, C, T, py, px;
  int tiles_x;        // tiles per grid row
};

// Tile of this workgroup.  Workgroups go to the eight XCDs in turn, so when
// the tile count allows, block b takes tile (b % 8) * (tiles / 8) + b / 8:
// each XCD then advances a contiguous band of tiles and the overlapping
// regions of neighbouring tiles meet in that XCD's L2.
__device__ __forceinline__ int tile_index() {
  const int b = blockIdx.x, n = gridDim.x;
  return (n % 8 == 0) ? (b % 8) * (n / 8) + b / 8 : b;
}

// Value of lane c - 1 (0 at lane 0) and of lane c + 1 (0 at lane 63):
// DPP wave_shr:1 / wave_shl:1.
__device__ __forceinline__ float from_left(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x138, 0xf, 0xf, false));
}
__device__ __forceinline__ float from_right(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x130, 0xf, 0xf, false));
}

// Where this thread's strip lies in the grid (INSIDE: the region is placed
// inside the grid).  Row offsets are uniform per wave; with the column's byte
// offset they address a field as base + row + column.
template <bool INSIDE>
struct Strip {
  int lane, w;
  int gx, gy0;    // grid column; grid row of strip row 0
  int R, C;
  int oq0, oq1;   // owned strip rows [oq0, oq1) (uniform per wave)
  bool own_lane;  // the lane's column is owned
  int prow;       // strip row of the pickup cell in this lane, or -1
  int pw;         // strip row of the pickup row if the pickup lies in this strip's rows and the region's columns, else -1
  unsigned colb;  // 4 * column, clamped into the grid
  unsigned ownb;  // 4 * column, clamped into the owned columns

  int tile;       // tile index (row-major)

  __device__ Strip(const MemArgs& a) : R(a.R), C(a.C) {
    lane = threadIdx.x & 63;
    w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    tile = tile_index();
    const int tx0 = (tile % a.tiles_x) * kTile, ty0 = (tile / a.tiles_x) * kTile;
    const int tx1 = min(tx0 + kTile, a.C), ty1 = min(ty0 + kTile, a.R);
    int rx0 = tx0 - kHalo, ry0 = ty0 - kHalo;
    if constexpr (INSIDE) {
      rx0 = min(max(rx0, 0), a.C - kSide);
      ry0 = min(max(ry0, 0), a.R - kSide);
    }
    gx = rx0 + lane;
    gy0 = ry0 + kRows * w;
    oq0 = min(max(ty0 - gy0, 0), kRows);
    oq1 = min(max(ty1 - gy0, 0), kRows);
    own_lane = gx >= tx0 && gx < tx1;
    const int pq = a.py - gy0;
    prow = (gx == a.px && pq >= 0 && pq < kRows) ? pq : -1;
    pw = (a.px - rx0 >= 0 && a.px - rx0 < 64 && pq >= 0 && pq < kRows) ? pq : -1;
    colb = 4u * (unsigned)min(max(gx, 0), a.C - 1);
    ownb = 4u * (unsigned)min(max(gx, tx0), tx1 - 1);
  }
  __device__ bool own_rows() const { return oq0 < oq1; }
  __device__ bool all_rows_owned() const { return oq0 == 0 && oq1 == kRows; }
  // bit q set for owned strip rows
  __device__ unsigned own_mask() const { return ((1u << oq1) - 1u) & ~((1u << oq0) - 1u); }
  // cell (q, lane) is inside the grid
  __device__ bool in(int q) const {
    if constexpr (INSIDE) return true;
    return gx >= 0 && gx < C && gy0 + q >= 0 && gy0 + q < R;
  }
  // byte offset of strip row q's grid row (clamped into the grid; below 2^30)
  __device__ unsigned rowb(int q) const { return 4u * (unsigned)(min(max(gy0 + q, 0), R - 1) * C); }
};

// A field of R x C cells as a raw buffer: loads and stores address it by a
// per-lane column offset plus a uniform row offset (an SGPR operand), and
// the hardware drops any access past its G cells.
using Field = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ Field field(const float* f, size_t G) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(f), 0, (int)(G * sizeof(float)), 0x00020000);
}
// Cache policy operand: 0 = default, kStream = non-temporal (the gfx940
// family's nt bit) for the forward's state stores: each state is written
// once and read once, much later, by the backward, so its traffic need not
// stay in the caches (non-temporal loads in the backward measured slower).
constexpr int kStream = 2;
template <int POLICY = 0>
__device__ __forceinline__ float fload(Field f, unsigned col, unsigned row) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(f, col, row, POLICY));
}
template <int POLICY = 0>
__device__ __forceinline__ void fstore(float v, Field f, unsigned col, unsigned row) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), f, col, row, POLICY);
}

// Reads strip rows of field f (cells outside the grid read a clamped cell).
template <bool INSIDE>
__device__ __forceinline__ void load_rows(const Strip<INSIDE>& st, Field f, float (&v)[kRows]) {
#pragma unroll
  for (int q = 0; q < kRows; ++q) v[q] = fload(f, st.colb, st.rowb(q));
}

// 1 for cells inside the grid, 0 outside (centred regions only).  The
// kernels scale the Laplacian by it: a cell outside the grid starts at zero
// and its update (2u - u_prev + c2 L u - d (u - u_prev) forward, the same form
// backward) then stays exactly zero.
template <bool INSIDE>
__device__ __forceinline__ void keep_mask(const Strip<INSIDE>& st, float (&keep)[kRows]) {
#pragma unroll
  for (int q = 0; q < kRows; ++q) keep[q] = st.in(q) ? 1.0f : 0.0f;
}

// Publishes the strip's first and last rows of u and returns the row above
// the strip and the row below it (zero at the region edge).
template <bool INSIDE>
__device__ __forceinline__ void exchange_edges(float (*e)[2][64], const Strip<INSIDE>& st, const float (&u)[kRows],
                                               float& up, float& dn) {
  e[st.w][0][st.lane] = u[0];
  e[st.w][1][st.lane] = u[kRows - 1];
  lds_barrier();
  up = st.w > 0 ? e[st.w - 1][1][st.lane] : 0.0f;
  dn = st.w + 1 < kWaves ? e[st.w + 1][0][st.lane] : 0.0f;
}

// 5-point Laplacian at strip row q, in the reference's summation order
// (up, left, centre, right, down).
__device__ __forceinline__ float lap_row(const float (&u)[kRows], float up, float dn, int q) {
  const float n = q == 0 ? up : u[q - 1];
  const float s = q == kRows - 1 ? dn : u[q + 1];
  return (((n + from_left(u[q])) + u[q] * -4.0f) + from_right(u[q])) + s;
}

// Forward: frames n0 .. n0+ks-1 (u_{n0+1} .. u_{n0+ks}).
template <bool INSIDE>
__global__ __launch_bounds__(kThreads) void k_mem_fwd(MemArgs a, int n0, int ks) {
  __shared__ float edge[2][kWaves][2][64];
  const Strip<INSIDE> st(a);
  const size_t G = (size_t)a.R * a.C;
  const float c2 = a.prm[0], d = a.prm[1];
  float keep[kRows];
  if constexpr (!INSIDE) keep_mask(st, keep);
  float u[kRows], v[kRows];  // u_n, u_{n-1}
  load_rows(st, field(a.S + (size_t)(n0 + 1) * G, G), u);
  load_rows(st, field(a.S + (size_t)n0 * G, G), v);
  if constexpr (!INSIDE) {
#pragma unroll
    for (int q = 0; q < kRows; ++q) {
      u[q] *= keep[q];
      v[q] *= keep[q];
    }
  }
  // the owned copy of the pickup cell (copies next to a region edge go wrong)
  const bool pick = st.own_lane && st.prow >= st.oq0 && st.prow < st.oq1;
  // (cur, prv) -> prv = the next state; owned cells -> S[n0+s+2], pickup -> out[n0+s]
  auto step = [&](const float (&cur)[kRows], float (&prv)[kRows], int s) {
    float up, dn;
    exchange_edges(edge[s & 1], st, cur, up, dn);
    auto row = [&](int q) {
      float lap = lap_row(cur, up, dn, q);
      if constexpr (!INSIDE) lap *= keep[q];
      const float b = cur[q] * 2.0f - prv[q];
      const float g = (cur[q] - prv[q]) * d;
      prv[q] = (b + lap * c2) - g;
    };
    // interior rows first: they do not wait for the exchanged edge rows
#pragma unroll
    for (int q = 1; q < kRows - 1; ++q) row(q);
    row(0);
    row(kRows - 1);
    if (st.own_rows()) {
      const Field dst = field(a.S + (size_t)(n0 + s + 2) * G, G);
      if (st.own_lane) {
        if (st.all_rows_owned()) {
#pragma unroll
          for (int q = 0; q < kRows; ++q) fstore<kStream>(prv[q], dst, st.colb, st.rowb(q));
        } else {
          const unsigned m = st.own_mask();
#pragma unroll
          for (int q = 0; q < kRows; ++q)
            if ((m >> q) & 1u) fstore<kStream>(prv[q], dst, st.colb, st.rowb(q));
        }
      }
      if (pick) {
#pragma unroll
        for (int q = 0; q < kRows; ++q)
          if (q == st.prow) a.out[n0 + s] = prv[q];
      }
    }
  };
  int s = 0;
  for (; s + 1 < ks; s += 2) {
    step(u, v, s);
    step(v, u, s + 1);
  }
  if (s < ks) step(u, v, s);
}

// Backward: adjoint steps n = m_hi .. m_hi-ks+1 (n >= 0), from
// (lambda_{m_hi+1}, lambda_{m_hi+2}) in lam set `src` (zeroed by the launcher
// before the first launch) to set `dst`.  Step n computes lambda_n and, from
// the same stencil pass, the gradient terms of lambda_{n+1} (L symmetric:
// <lambda, L u> = <L lambda, u>):
//   dc2 += L(lambda_{n+1}) u_n,  dd += lambda_{n+1} (u_{n-1} - u_n)
// over the owned cells: per cell in fp32 over the launch's steps, then in
// fp64 over cells, workgroup partials and launches.  In the waves that hold
// owned rows, the stored states F_k = S[m_hi + 1 - k] (step s needs
// F_s = u_n and F_{s+1} = u_{n-1}) stream through a ring of four register
// strips, loaded three steps ahead.  Every lane and row of those waves loads
// (from its owned column and grid row, clamped), so that with no branch
// around the loads each wait covers exactly the strip it needs; the sums
// keep only the owned cells.  The source terms of the launch's steps are read
// once into LDS, so that no step waits on a vector load.  The schedule runs
// n down to 0 so that lambda_1's terms are included.
struct BwdShared {
  float edge[2][kWaves][2][64];
  float srcv[kHalo];  // 2 (out[n-1] - tgt[n-1]) of step s, 0 for n = 0
};

template <bool INSIDE, bool OWNED>
__device__ __forceinline__ void bwd_strip(const MemArgs& a, const Strip<INSIDE>& st, BwdShared& sh, int m_hi, int ks,
                                          int src, int dst, double& gc, double& gd) {
  const size_t G = (size_t)a.R * a.C;
  const float c2 = a.prm[0], d = a.prm[1];
  const float ad = 2.0f - d, bd = 1.0f - d;
  float keep[kRows];
  if constexpr (!INSIDE) keep_mask(st, keep);
  float x[kRows], y[kRows];  // lambda_{n+1}, lambda_{n+2}
  const float* ls = a.lam + (size_t)src * 2 * G;
  load_rows(st, field(ls, G), x);
  load_rows(st, field(ls + G, G), y);
  auto fetch = [&](int k, float (&f)[kRows]) {
    const Field F = field(a.S + (size_t)(m_hi + 1 - min(k, ks)) * G, G);
#pragma unroll
    for (int q = 0; q < kRows; ++q) f[q] = fload(F, st.ownb, st.rowb(q));
  };
  float f0[kRows], f1[kRows], f2[kRows], f3[kRows];
  float acc_c[kRows], acc_d[kRows];
  if constexpr (OWNED) {
    fetch(0, f0);
    fetch(1, f1);
    fetch(2, f2);
    fetch(3, f3);
#pragma unroll
    for (int q = 0; q < kRows; ++q) acc_c[q] = acc_d[q] = 0.0f;
  }
  // all loads issued: now zero the adjoint outside the grid
  if constexpr (!INSIDE) {
#pragma unroll
    for (int q = 0; q < kRows; ++q) {
      x[q] *= keep[q];
      y[q] *= keep[q];
    }
  }
  // (lambda_{n+1}, lambda_{n+2}) -> lam2 = lambda_n; fa = u_n, fb = u_{n-1};
  // fa is then refilled with F_{s+4} (F_ks again past the launch's end).
  auto step = [&](const float (&lam1)[kRows], float (&lam2)[kRows], float (&fa)[kRows], const float (&fb)[kRows],
                  int s) {
    float up, dn;
    exchange_edges(sh.edge[s & 1], st, lam1, up, dn);
    float lap[kRows];
    auto row = [&](int q) {
      lap[q] = lap_row(lam1, up, dn, q);
      if constexpr (!INSIDE) lap[q] *= keep[q];
      lam2[q] = (ad * lam1[q] + c2 * lap[q]) - bd * lam2[q];
    };
#pragma unroll
    for (int q = 1; q < kRows - 1; ++q) row(q);
    row(0);
    row(kRows - 1);
    if (st.pw >= 0) {  // uniform: only the wave holding the pickup row
      const float src_lane = st.prow >= 0 ? sh.srcv[s] : 0.0f;
#pragma unroll
      for (int q = 0; q < kRows; ++q) lam2[q] += q == st.pw ? src_lane : 0.0f;
    }
    if constexpr (OWNED) {
#pragma unroll
      for (int q = 0; q < kRows; ++q) {
        acc_c[q] = fmaf(lap[q], fa[q], acc_c[q]);
        acc_d[q] = fmaf(lam1[q], fb[q] - fa[q], acc_d[q]);
      }
      fetch(s + 4, fa);
    }
  };
  // Whole groups of four steps, then the rest: no exit or store inside the
  // pipelined loop, so the waits on the ring stay exact.
  int s = 0;
  for (; s + 4 <= ks; s += 4) {
    step(x, y, f0, f1, s);
    step(y, x, f1, f2, s + 1);
    step(x, y, f2, f3, s + 2);
    step(y, x, f3, f0, s + 3);
  }
  if (s < ks) {
    step(x, y, f0, f1, s);
    if (s + 1 < ks) {
      step(y, x, f1, f2, s + 1);
      if (s + 2 < ks) step(x, y, f2, f3, s + 2);
    }
  }
  if constexpr (OWNED) {
    if (st.own_lane) {
      // boundary fields (lambda_{m_lo}, lambda_{m_lo+1}) of the owned cells -> set dst
      const float* o = a.lam + (size_t)dst * 2 * G;
      const Field o0 = field(o, G), o1 = field(o + G, G);
      const bool odd = (ks & 1) != 0;  // an odd step count leaves the newest field in y
      const unsigned m = st.own_mask();
#pragma unroll
      for (int q = 0; q < kRows; ++q) {
        if (!((m >> q) & 1u)) continue;
        fstore(odd ? y[q] : x[q], o0, st.colb, st.rowb(q));
        fstore(odd ? x[q] : y[q], o1, st.colb, st.rowb(q));
        gc += (double)acc_c[q];
        gd += (double)acc_d[q];
      }
    }
  }
}

// Value of lane i - K within the lane's row of 16 (0 for the first K lanes
// of the row): DPP row_shr:K on both halves of a double.
template <int K>
__device__ __forceinline__ double row_shr(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, 0x110 + K, 0xf, 0xf, true);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), 0x110 + K, 0xf, 0xf, true);
  return __builtin_bit_cast(double, (unsigned long long)(unsigned)lo | ((unsigned long long)(unsigned)hi << 32));
}

__device__ __forceinline__ double lane_value(double v, int lane) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = __builtin_amdgcn_readlane((int)(unsigned)b, lane);
  const unsigned hi = __builtin_amdgcn_readlane((int)(unsigned)(b >> 32), lane);
  return __builtin_bit_cast(double, (unsigned long long)lo | ((unsigned long long)hi << 32));
}

// Sum over the wave in a fixed order (uniform result): shift-and-add within
// each row of 16 lanes leaves the row's sum in its last lane, then the four
// row sums.
__device__ __forceinline__ double wave_sum(double v) {
  v += row_shr<1>(v);
  v += row_shr<2>(v);
  v += row_shr<4>(v);
  v += row_shr<8>(v);
  return (lane_value(v, 15) + lane_value(v, 31)) + (lane_value(v, 47) + lane_value(v, 63));
}

// Each wave holding owned rows sums its cells' fp64 terms over the wave and
// adds them to its slot of the tile's partials (zeroed by the launcher),
// read at the start of the launch: no barrier or LDS for the reduction, and
// a fixed summation order.
template <bool INSIDE>
__global__ __launch_bounds__(kThreads) void k_mem_bwd(MemArgs a, int m_hi, int ks, int src, int dst) {
  __shared__ BwdShared sh;
  if ((int)threadIdx.x < ks) {
    const int n = m_hi - (int)threadIdx.x;
    sh.srcv[threadIdx.x] = n >= 1 ? 2.0f * (a.out[n - 1] - a.tgt[n - 1]) : 0.0f;
  }
  const Strip<INSIDE> st(a);
  double gc = 0.0, gd = 0.0;
  if (st.own_rows()) {
    double* gp = a.gpart + 2 * ((size_t)st.tile * kWaves + st.w);
    const double prev_c = gp[0], prev_d = gp[1];
    bwd_strip<INSIDE, true>(a, st, sh, m_hi, ks, src, dst, gc, gd);
    gc = wave_sum(gc);
    gd = wave_sum(gd);
    if (st.lane == 0) {
      gp[0] = prev_c + gc;
      gp[1] = prev_d + gd;
    }
  } else {
    bwd_strip<INSIDE, false>(a, st, sh, m_hi, ks, src, dst, gc, gd);
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

// f[i] = 0 for i < n.
__global__ void k_mem_zero(float* __restrict__ f, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) f[i] = 0.0f;
}

// grads[q] = sum of the fp64 partials [n][2]: one workgroup of kFinal
// threads, each summing a fixed stride of slots, then a fixed tree.
constexpr int kFinal = 1024;
__global__ __launch_bounds__(kFinal) void k_mem_grad_final(const double* __restrict__ gpart, float* __restrict__ grads,
                                                           int n) {
  __shared__ double red[2][kFinal];
  double c = 0.0, d = 0.0;
  for (int i = threadIdx.x; i < n; i += kFinal) {
    c += gpart[2 * i];
    d += gpart[2 * i + 1];
  }
  red[0][threadIdx.x] = c;
  red[1][threadIdx.x] = d;
  __syncthreads();
  for (int h = kFinal / 2; h >= 1; h >>= 1) {
    if ((int)threadIdx.x < h) {
      red[0][threadIdx.x] += red[0][threadIdx.x + h];
      red[1][threadIdx.x] += red[1][threadIdx.x + h];
    }
    __syncthreads();
  }
  if (threadIdx.x < 2) grads[threadIdx.x] = (float)red[threadIdx.x][0];
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
  a.tiles_x = (int)((C + kTile - 1) / kTile);
  const dim3 grid((unsigned)(a.tiles_x * ((R + kTile - 1) / kTile)));
  const bool inside = R >= kSide && C >= kSide;  // regions placed inside the grid
  for (int64_t n0 = 0; n0 < T; n0 += ks) {
    const int n = (int)std::min<int64_t>(ks, T - n0);
    if (inside)
      hipLaunchKernelGGL(k_mem_fwd<true>, grid, dim3(kThreads), 0, L.stream, a, (int)n0, n);
    else
      hipLaunchKernelGGL(k_mem_fwd<false>, grid, dim3(kThreads), 0, L.stream, a, (int)n0, n);
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
  DGEN_CHECK_CELL(L, gpart, 4 * tiles * kWaves, "membrane_bwd.grad_partials");
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
  a.tiles_x = (int)((C + kTile - 1) / kTile);
  const dim3 grid((unsigned)tiles);
  // (lambda_{T+1}, lambda_{T+2}) = 0: set 1 starts zeroed; so do the gradient slots
  const unsigned zb = (unsigned)std::min<int64_t>((2 * G + 255) / 256, (int64_t)L.cu_count * 8);
  hipLaunchKernelGGL(k_mem_zero, dim3(zb), dim3(256), 0, L.stream, a.lam + 2 * G, (size_t)(2 * G));
  DGEN_LAUNCH_CHECK("k_mem_zero");
  const int64_t nslots = tiles * kWaves;
  hipLaunchKernelGGL(k_mem_zero, dim3(zb), dim3(256), 0, L.stream, reinterpret_cast<float*>(a.gpart),
                     (size_t)(4 * nslots));
  DGEN_LAUNCH_CHECK("k_mem_zero");
  const bool inside = R >= kSide && C >= kSide;  // regions placed inside the grid
  int src = 1, dst = 0;
  for (int64_t m_hi = T; m_hi >= 0; m_hi -= ks) {
    const int n = (int)std::min<int64_t>(ks, m_hi + 1);
    if (inside)
      hipLaunchKernelGGL(k_mem_bwd<true>, grid, dim3(kThreads), 0, L.stream, a, (int)m_hi, n, src, dst);
    else
      hipLaunchKernelGGL(k_mem_bwd<false>, grid, dim3(kThreads), 0, L.stream, a, (int)m_hi, n, src, dst);
    DGEN_LAUNCH_CHECK("k_mem_bwd");
    src = dst;
    dst ^= 1;
  }
  hipLaunchKernelGGL(k_mem_grad_final, dim3(1), dim3(kFinal), 0, L.stream, a.gpart, cell(L, grads), (int)nslots);
  DGEN_LAUNCH_CHECK("k_mem_grad_final");
  return 0;
}

}  // namespace dgen
