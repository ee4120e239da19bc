// Control-network pieces around the GEMMs: the small-fan-in first layer and
// its weight gradient, the decoder head activations and their backward, the
// bias-gradient column sums and the Adam update.
//
// Reference: HarmonicDecoderModel (Examples/HarmonicE2E/Model.swift:96-157),
// Adam.step (Sources/DGenLazy/Optimizers.swift:164-204), AD rules for tanh,
// max, abs, exp, log (Sources/DGen/Gradients.swift:398-490).
//
// Reductions are deterministic: fixed-order per-thread loops and fixed-shape
// two-stage sums, no atomics.
#include "dev_math.h"
#include "internal.h"

namespace dgen {

constexpr int kWave = 64;


// ---------------------------------------------------------------- layer 1
// H[m][j] = tanh(sum_i X[m][i] W[i][j] + b[j]) for a fan-in of a few inputs.
// Each thread writes 4 consecutive outputs of a row (width % 4 == 0), grid-
// strided over rows.
__global__ __launch_bounds__(256) void k_dense_small(const float* __restrict__ X, const float* __restrict__ W,
                                                     const float* __restrict__ b, float* __restrict__ H, int rows,
                                                     int fan, int width) {
  const int qw = width / 4;
  const size_t total = (size_t)rows * qw;
  for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (size_t)gridDim.x * blockDim.x) {
    const int m = (int)(g / qw), j = (int)(g % qw) * 4;
    float4 s = *reinterpret_cast<const float4*>(b + j);
    for (int i = 0; i < fan; ++i) {
      const float x = X[(size_t)m * fan + i];
      const float4 w = *reinterpret_cast<const float4*>(W + (size_t)i * width + j);
      s.x = fmaf(x, w.x, s.x);
      s.y = fmaf(x, w.y, s.y);
      s.z = fmaf(x, w.z, s.z);
      s.w = fmaf(x, w.w, s.w);
    }
    *reinterpret_cast<float4*>(H + (size_t)m * width + j) =
        make_float4(fast_tanh(s.x), fast_tanh(s.y), fast_tanh(s.z), fast_tanh(s.w));
  }
}

int launch_dense_small(const Launch& L, const dgen_hip_op& op) {
  const int64_t X = op.arg[0], W = op.arg[1], b = op.arg[2], H = op.arg[3];
  const int64_t rows = op.arg[4], fan = op.arg[5], width = op.arg[6];
  DGEN_REQUIRE(rows > 0 && rows < (1ll << 31) && fan > 0 && fan <= 64 && width > 0 && width <= 65536,
               "dense_small: rows %lld fan %lld width %lld", (long long)rows, (long long)fan, (long long)width);
  DGEN_CHECK_CELL(L, X, rows * fan, "dense_small.X");
  DGEN_CHECK_CELL(L, W, fan * width, "dense_small.W");
  DGEN_CHECK_CELL(L, b, width, "dense_small.b");
  DGEN_CHECK_CELL(L, H, rows * width, "dense_small.H");
  DGEN_REQUIRE(width % 4 == 0 && W % 4 == 0 && b % 4 == 0 && H % 4 == 0,
               "dense_small: width %lld and the W, b, H cells must be multiples of 4", (long long)width);
  if (L.dry) return 0;
  const int64_t quads = rows * (width / 4);
  const unsigned blocks = (unsigned)std::min<int64_t>((quads + 255) / 256, (int64_t)L.cu_count * 16);
  hipLaunchKernelGGL(k_dense_small, dim3(blocks), dim3(256), 0, L.stream, cell(L, X), cell(L, W), cell(L, b),
                     cell(L, H), (int)rows, (int)fan, (int)width);
  DGEN_LAUNCH_CHECK("k_dense_small");
  return 0;
}

// Deterministic two-stage column reductions over the row (batch) axis:
//   out_q[n] = sum_m w_q(m) * A[m][n],  w_q(m) = X[m][q] for q < nw, 1 for q = nw
// Stage 1: workgroup (column block of 64, row chunk c); its 4 waves stride the
// chunk's rows, lanes read 64 consecutive columns (256-byte rows), and the
// waves' sums are combined in LDS in wave order -> part[c][q][n].
// Stage 2: one workgroup per 64 columns sums the chunk partials in chunk order
// (4 waves over interleaved chunks, then wave order).
constexpr int kColChunks = 128;
constexpr int kMaxW = 4;  // weighted sums besides the plain one

// V4: each lane reads 4 consecutive columns (float4; cols, lda and the base
// are multiples of 4), so a workgroup covers 256 columns; else 64 columns.
template <bool V4>
__global__ __launch_bounds__(256) void k_colsum_partial(const float* __restrict__ A, int lda,
                                                        const float* __restrict__ X, int nw, int rows, int cols,
                                                        int chunk, float* __restrict__ part, int want_plain) {
  constexpr int CW = V4 ? 4 : 1;  // columns per lane
  __shared__ float red[4][kMaxW + 1][64 * CW];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = (blockIdx.x * 64 + lane) * CW;
  const int c = blockIdx.y;
  const int m0 = c * chunk, m1 = min(rows, m0 + chunk);
  float acc[kMaxW + 1][CW];
#pragma unroll
  for (int q = 0; q <= kMaxW; ++q)
#pragma unroll
    for (int e = 0; e < CW; ++e) acc[q][e] = 0.f;
  if (n < cols) {
#pragma unroll 8
    for (int m = m0 + wave; m < m1; m += 4) {
      float v[CW];
      if constexpr (V4) {
        const float4 t = *reinterpret_cast<const float4*>(A + (size_t)m * lda + n);
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
      } else {
        v[0] = A[(size_t)m * lda + n];
      }
#pragma unroll
      for (int q = 0; q < kMaxW; ++q)
        if (q < nw) {
          const float x = X[(size_t)m * nw + q];
#pragma unroll
          for (int e = 0; e < CW; ++e) acc[q][e] += x * v[e];
        }
#pragma unroll
      for (int e = 0; e < CW; ++e) acc[kMaxW][e] += v[e];
    }
  }
#pragma unroll
  for (int q = 0; q <= kMaxW; ++q)
#pragma unroll
    for (int e = 0; e < CW; ++e) red[wave][q][lane * CW + e] = acc[q][e];
  __syncthreads();
  if (wave == 0) {
    const int nq = nw + (want_plain ? 1 : 0);
    for (int q = 0; q < nq; ++q) {
      const int src = q < nw ? q : kMaxW;
#pragma unroll
      for (int e = 0; e < CW; ++e) {
        const int col = n + e;
        if (col >= cols) continue;
        const int li = lane * CW + e;
        const float v = ((red[0][src][li] + red[1][src][li]) + red[2][src][li]) + red[3][src][li];
        part[((size_t)c * nq + q) * cols + col] = v;
      }
    }
  }
}

__global__ __launch_bounds__(256) void k_colsum_final(const float* __restrict__ part, int chunks, int nq, int cols,
                                                      float* __restrict__ out0, int ld_out0,
                                                      float* __restrict__ plain_out, int want_plain) {
  __shared__ float red[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = blockIdx.x * 64 + lane;
  const int q = blockIdx.y;
  float s = 0.f;
  if (n < cols) {
    // loads issued 8 at a time; the adds keep the fixed chunk order
#pragma unroll 8
    for (int c = wave; c < chunks; c += 4) s += part[((size_t)c * nq + q) * cols + n];
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && n < cols) {
    const float v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
    if (want_plain && q == nq - 1)
      plain_out[n] = v;
    else
      out0[(size_t)q * ld_out0 + n] = v;
  }
}

// Row chunks of stage 1: weighted sums do more work per row, so they use
// twice as many (shorter) chunks.
static int colsum_chunks(int64_t rows, int nw = 0) {
  return (int)std::min<int64_t>(nw > 0 ? 2 * kColChunks : kColChunks, std::max<int64_t>(1, rows / 32));
}

// out_q (q < nw) rows of out0 (stride ld_out0) and the plain sum into plain_out.
static int colsum_launch(const Launch& L, const float* A, int lda, const float* X, int nw, int rows, int cols,
                         float* ws, float* out0, int ld_out0, float* plain_out) {
  const int chunks = colsum_chunks(rows, nw);
  const int chunk = (rows + chunks - 1) / chunks;
  const int want_plain = plain_out != nullptr;
  const int nq = nw + want_plain;
  const bool v4 = cols % 4 == 0 && lda % 4 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  if (v4)
    hipLaunchKernelGGL(k_colsum_partial<true>, dim3((unsigned)((cols + 255) / 256), (unsigned)chunks), dim3(256), 0,
                       L.stream, A, lda, X, nw, rows, cols, chunk, ws, want_plain);
  else
    hipLaunchKernelGGL(k_colsum_partial<false>, dim3((unsigned)((cols + 63) / 64), (unsigned)chunks), dim3(256), 0,
                       L.stream, A, lda, X, nw, rows, cols, chunk, ws, want_plain);
  DGEN_LAUNCH_CHECK("k_colsum_partial");
  hipLaunchKernelGGL(k_colsum_final, dim3((unsigned)((cols + 63) / 64), (unsigned)nq), dim3(256), 0, L.stream, ws,
                     chunks, nq, cols, out0, ld_out0, plain_out, want_plain);
  DGEN_LAUNCH_CHECK("k_colsum_final");
  return 0;
}

int launch_colsum(const Launch& L, const dgen_hip_op& op) {
  const int64_t A = op.arg[0], out = op.arg[1], rows = op.arg[2], cols = op.arg[3], lda = op.arg[4], ws = op.arg[5];
  DGEN_REQUIRE(rows > 0 && rows < (1ll << 31) && cols > 0 && lda >= cols && cols <= 65536,
               "colsum: rows %lld cols %lld lda %lld", (long long)rows, (long long)cols, (long long)lda);
  const int chunks = colsum_chunks(rows);
  DGEN_CHECK_CELL(L, A, (rows - 1) * lda + cols, "colsum.A");
  DGEN_CHECK_CELL(L, out, cols, "colsum.out");
  DGEN_CHECK_CELL(L, ws, (int64_t)chunks * cols, "colsum.workspace");
  if (L.dry) return 0;
  return colsum_launch(L, cell(L, A), (int)lda, nullptr, 0, (int)rows, (int)cols, cell(L, ws), nullptr, 0,
                       cell(L, out));
}

// dW[i][j] = sum_m X[m][i] dZ[m][j] for a small fan-in (first layer), and
// optionally the bias gradient db[j] = sum_m dZ[m][j] from the same pass.
int launch_dense_small_wgrad(const Launch& L, const dgen_hip_op& op) {
  const int64_t X = op.arg[0], dZ = op.arg[1], dW = op.arg[2], rows = op.arg[3], fan = op.arg[4],
                width = op.arg[5], ws = op.arg[6], db = op.arg[7];
  DGEN_REQUIRE(rows > 0 && rows < (1ll << 31) && fan > 0 && fan <= kMaxW && width > 0 && width <= 65536,
               "dense_small_wgrad: rows %lld fan %lld width %lld", (long long)rows, (long long)fan,
               (long long)width);
  const int chunks = colsum_chunks(rows, (int)fan);
  DGEN_CHECK_CELL(L, X, rows * fan, "dense_small_wgrad.X");
  DGEN_CHECK_CELL(L, dZ, rows * width, "dense_small_wgrad.dZ");
  DGEN_CHECK_CELL(L, dW, fan * width, "dense_small_wgrad.dW");
  if (db >= 0) DGEN_CHECK_CELL(L, db, width, "dense_small_wgrad.db");
  DGEN_CHECK_CELL(L, ws, (int64_t)chunks * (fan + 1) * width, "dense_small_wgrad.workspace");
  if (L.dry) return 0;
  return colsum_launch(L, cell(L, dZ), (int)width, cell(L, X), (int)fan, (int)rows, (int)width, cell(L, ws),
                       cell(L, dW), (int)width, db >= 0 ? cell(L, db) : nullptr);
}

// ---------------------------------------------------------------- heads

// One wave per row; Z and ctrl rows have stride ldz / ldc.  Lane l owns
// elements l, l + 64, ..., l + 64 (HP - 1) of each head group (K, NF <=
// 64 HP: HP = 2 up to 128, 4 up to 256), and every softplus / tanh of a row
// is evaluated once, in registers (the sums add the same terms in the same
// order as a per-group loop).
template <int kHeadPer>
__global__ void k_heads_fwd(const float* __restrict__ Z, int ldz, float* __restrict__ C, int ldc, int rows, int K,
                            int NF) {
  const int m = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (m >= rows) return;
  const float* z = Z + (size_t)m * ldz;
  float* c = C + (size_t)m * ldc;
  float sp[kHeadPer], th[kHeadPer];
  float den = 0.f;
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q) {
    const int k = lane + q * kWave;
    sp[q] = k < K ? softplus(z[k]) : 0.f;
    if (k < K) den += sp[q];
  }
  den = wave_sum(den) + 1e-6f;
  const float rden = rcp_rn(den);
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q) {
    const int k = lane + q * kWave;
    if (k < K) c[k] = sp[q] * rden;
  }
  if (lane == 0) {
    c[K] = softplus(z[K]);
    c[K + 1] = softplus(z[K + 1]);
  }
  float nrm = 0.f;
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q) {
    const int i = lane + q * kWave;
    th[q] = i < NF ? fast_tanh(z[K + 2 + i]) : 0.f;
    if (i < NF) nrm += fabsf(th[q]);
  }
  nrm = wave_sum(nrm) + 1e-4f;
  const float rnrm = rcp_rn(nrm);
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q) {
    const int i = lane + q * kWave;
    if (i < NF) c[K + 2 + i] = th[q] * rnrm;
  }
}

template <int kHeadPer>
__global__ void k_heads_bwd(const float* __restrict__ Z, int ldz, const float* __restrict__ dC, int ldc,
                            float* __restrict__ dZ, int lddz, int rows, int K, int NF) {
  const int m = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (m >= rows) return;
  const float* z = Z + (size_t)m * ldz;
  const float* dc = dC + (size_t)m * ldc;
  float* dz = dZ + (size_t)m * lddz;
  float zk[kHeadPer], sp[kHeadPer], dk[kHeadPer];
  float den = 0.f;
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q) {
    const int k = lane + q * kWave;
    zk[q] = k < K ? z[k] : 0.f;
    dk[q] = k < K ? dc[k] : 0.f;
    sp[q] = softplus(zk[q]);
    if (k < K) den += sp[q];
  }
  den = wave_sum(den) + 1e-6f;
  float dot = 0.f;
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q)
    if (lane + q * kWave < K) dot += dk[q] * (sp[q] / den);
  dot = wave_sum(dot);
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q) {
    const int k = lane + q * kWave;
    if (k < K) dz[k] = (dk[q] - dot) / den * softplus_grad(zk[q]);
  }
  if (lane == 0) {
    dz[K] = dc[K] * softplus_grad(z[K]);
    dz[K + 1] = dc[K + 1] * softplus_grad(z[K + 1]);
  }
  float th[kHeadPer], dt[kHeadPer];
  float nrm = 0.f;
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q) {
    const int i = lane + q * kWave;
    th[q] = i < NF ? tanhf(z[K + 2 + i]) : 0.f;
    dt[q] = i < NF ? dc[K + 2 + i] : 0.f;
    if (i < NF) nrm += fabsf(th[q]);
  }
  nrm = wave_sum(nrm) + 1e-4f;
  float dot2 = 0.f;
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q)
    if (lane + q * kWave < NF) dot2 += dt[q] * (th[q] / nrm);
  dot2 = wave_sum(dot2);
#pragma unroll
  for (int q = 0; q < kHeadPer; ++q) {
    const int i = lane + q * kWave;
    if (i < NF) {
      const float s = th[q];
      const float sg = s > 0.f ? 1.f : (s < 0.f ? -1.f : 0.f);
      dz[K + 2 + i] = (dt[q] - sg * dot2) / nrm * (1.f - s * s);
    }
  }
  // padding columns of the stored dZ row stay exactly zero
  for (int c = K + 2 + NF + lane; c < lddz; c += kWave) dz[c] = 0.f;
}

int launch_heads_fwd(const Launch& L, const dgen_hip_op& op) {
  const int64_t Z = op.arg[0], C = op.arg[1], rows = op.arg[2], K = op.arg[3], NF = op.arg[4];
  const int64_t ld = op.arg[5];
  DGEN_REQUIRE(rows > 0 && K > 0 && NF > 0 && K <= 4 * kWave && NF <= 4 * kWave && ld >= K + 2 + NF,
               "heads_fwd: rows %lld K %lld NF %lld ld %lld",
               (long long)rows, (long long)K, (long long)NF, (long long)ld);
  DGEN_CHECK_CELL(L, Z, rows * ld, "heads_fwd.Z");
  DGEN_CHECK_CELL(L, C, rows * ld, "heads_fwd.ctrl");
  if (L.dry) return 0;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  if (K <= 2 * kWave && NF <= 2 * kWave)
    hipLaunchKernelGGL(k_heads_fwd<2>, grid, block, 0, L.stream, cell(L, Z), (int)ld, cell(L, C), (int)ld,
                       (int)rows, (int)K, (int)NF);
  else
    hipLaunchKernelGGL(k_heads_fwd<4>, grid, block, 0, L.stream, cell(L, Z), (int)ld, cell(L, C), (int)ld,
                       (int)rows, (int)K, (int)NF);
  DGEN_LAUNCH_CHECK("k_heads_fwd");
  return 0;
}

int launch_heads_bwd(const Launch& L, const dgen_hip_op& op) {
  const int64_t Z = op.arg[0], dC = op.arg[1], dZ = op.arg[2], rows = op.arg[3], K = op.arg[4], NF = op.arg[5];
  const int64_t ld = op.arg[6];
  DGEN_REQUIRE(rows > 0 && K > 0 && NF > 0 && K <= 4 * kWave && NF <= 4 * kWave && ld >= K + 2 + NF,
               "heads_bwd: rows %lld K %lld NF %lld ld %lld",
               (long long)rows, (long long)K, (long long)NF, (long long)ld);
  DGEN_CHECK_CELL(L, Z, rows * ld, "heads_bwd.Z");
  DGEN_CHECK_CELL(L, dC, rows * ld, "heads_bwd.dctrl");
  DGEN_CHECK_CELL(L, dZ, rows * ld, "heads_bwd.dZ");
  if (L.dry) return 0;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  if (K <= 2 * kWave && NF <= 2 * kWave)
    hipLaunchKernelGGL(k_heads_bwd<2>, grid, block, 0, L.stream, cell(L, Z), (int)ld, cell(L, dC), (int)ld,
                       cell(L, dZ), (int)ld, (int)rows, (int)K, (int)NF);
  else
    hipLaunchKernelGGL(k_heads_bwd<4>, grid, block, 0, L.stream, cell(L, Z), (int)ld, cell(L, dC), (int)ld,
                       cell(L, dZ), (int)ld, (int)rows, (int)K, (int)NF);
  DGEN_LAUNCH_CHECK("k_heads_bwd");
  return 0;
}

// ---------------------------------------------------------------- Adam
// Adam.step (Optimizers.swift:164-204): t += 1; bias corrections in fp32;
// m = b1 m + (1-b1) g; v = b2 v + (1-b2) g g; p -= lr mhat / (sqrt(vhat)+eps).
// The step counter lives in a device cell; it is read by every thread and
// incremented afterwards by a separate one-thread launch (stream order).
#pragma clang fp contract(off)
__global__ void k_adam(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                       float* __restrict__ v, size_t n, const float* __restrict__ tcell, float lr, float b1, float b2,
                       float eps) {
  const float t = tcell[0] + 1.0f;
  const float bc1 = 1.0f - powf(b1, t);
  const float bc2 = 1.0f - powf(b2, t);
  for (size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (size_t)gridDim.x * blockDim.x) {
    float gj = g[j];
    float mj = b1 * m[j] + (1.0f - b1) * gj;
    float vj = b2 * v[j] + (1.0f - b2) * gj * gj;
    float mh = mj / bc1, vh = vj / bc2;
    p[j] = p[j] - lr * mh / (sqrtf(vh) + eps);
    m[j] = mj;
    v[j] = vj;
  }
}
#pragma clang fp contract(on)

__global__ void k_increment(float* c) {
  if (blockIdx.x == 0 && threadIdx.x == 0) c[0] = c[0] + 1.0f;
}

int launch_adam(const Launch& L, const dgen_hip_op& op) {
  const int64_t P = op.arg[0], G = op.arg[1], M = op.arg[2], V = op.arg[3], n = op.arg[4], tc = op.arg[5];
  DGEN_REQUIRE(n > 0, "adam: n %lld", (long long)n);
  DGEN_CHECK_CELL(L, P, n, "adam.params");
  DGEN_CHECK_CELL(L, G, n, "adam.grads");
  DGEN_CHECK_CELL(L, M, n, "adam.m");
  DGEN_CHECK_CELL(L, V, n, "adam.v");
  DGEN_CHECK_CELL(L, tc, 1, "adam.step");
  if (L.dry) return 0;
  unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, (int64_t)L.cu_count * 8);
  hipLaunchKernelGGL(k_adam, dim3(blocks), dim3(256), 0, L.stream, cell(L, P), cell(L, G), cell(L, M), cell(L, V),
                     (size_t)n, cell(L, tc), op.farg[0], op.farg[1], op.farg[2], op.farg[3]);
  DGEN_LAUNCH_CHECK("k_adam");
  hipLaunchKernelGGL(k_increment, dim3(1), dim3(64), 0, L.stream, cell(L, tc));
  DGEN_LAUNCH_CHECK("k_increment");
  return 0;
}

}  // namespace dgen
