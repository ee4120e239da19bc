// GEMM on the gfx950 matrix cores for the control network: forward layers
// with fused bias+tanh, backward data GEMMs with the fused tanh derivative,
// and weight-gradient GEMMs reduced over the 32k-row batch with a
// deterministic split-K.  Two product modes share the tiling and the fused
// epilogue:
//
// - fp32 products (k_gemm, v_mfma_f32_32x32x2_f32);
// - split-bf16 products (k_gemm_x6, k_gemm_x6d, v_mfma_f32_32x32x16_bf16):
//   each fp32 operand value is split exactly into three bfloat16 parts and
//   the six partial products above 2^-16 of the leading one are accumulated
//   in fp32 (Henry, Tang and Heinecke, "Leveraging the bfloat16 artificial
//   intelligence datatype for higher-precision computations", ARITH 2019),
//   as accurate as the fp32 products against fp64 at 192 matrix-core cycles
//   per 32x32x16 step instead of 512.  A weight operand shared by many row
//   tiles is split once per step into bfloat16 planes (k_split_bf16);
//   k_gemm_x6d copies full tiles of row-major A and those planes global ->
//   LDS with the load-to-LDS instructions and splits A at the fragment read.
//
// The reference lowers these matmuls to 8x8 simdgroup fp32 tiles
// (Sources/DGen/Emit+GEMM.swift:10-80, GEMMPass.swift:60-109); here each
// 256-thread workgroup owns a 128x128 output tile, each wave a 64x64 quadrant
// of four 32x32 MFMA accumulators (64 fp32 registers per lane).
//
// In k_gemm, LDS holds both operand tiles k-major ([BK][BM] and [BK][BN]) so
// every layout (A as [M][K] or [K][M], B as [K][N] or [N][K]) feeds the MFMA
// with conflict-free single-float reads; tiles are double buffered with one
// barrier per k-step.  The k-step depth is a template parameter (16 or 32);
// every launch uses BK = 16: 33 KB of LDS and at most 128 registers per lane,
// so four workgroups share a CU (four waves per SIMD): a 1000-tile grid runs
// in one round on 256 CUs, and each SIMD has other waves' MFMAs to issue
// while one waits at its barrier.  (BK = 32 takes 66 KB, two workgroups per
// CU: 5-10% slower alone.  The phasor carry beside the forward layers holds
// 148 KB of its CU's LDS, so no BK = 16 workgroup lands on its CUs either.)
#include "internal.h"

namespace dgen {

constexpr int BM = 128, BN = 128, LDSROW = BM + 4;
// Row stride of an operand tile that is stored transposed (scalar writes of
// four k values per thread).  The 32 lanes of a store pass cover BK/4
// k-groups x 128/BK rows:
// - BK = 16: 4 k-groups (k = 0, 4, 8, 12) x 8 rows; a stride of 2 mod 32
//   puts them on 32 distinct banks (k-group g at banks 8g .. 8g+7);
// - BK = 32: 8 k-groups x 4 rows; an odd stride does (2 mod 32 would fold
//   the k-groups onto 16 banks, 2-way; measured as bank-conflict cycles).
// The MFMA reads (one k, 32 consecutive rows per pass) are conflict-free
// either way.  A tile stored as float4 rows keeps 132 for 16-byte alignment.
template <int BK>
constexpr int ldsrow_t() { return BK == 16 ? BM + 2 : BM + 1; }
static_assert(ldsrow_t<16>() % 32 == 2 && ldsrow_t<32>() % 32 == 1, "transposed-store bank layout");

typedef float floatx16 __attribute__((ext_vector_type(16)));

enum { EPI_NONE = 0, EPI_BIAS = 1, EPI_BIAS_TANH = 2, EPI_TANH_GRAD = 3 };

template <bool VEC>
__device__ __forceinline__ float4 load4(const float* __restrict__ p, int valid) {
  if (VEC && valid >= 4) return *reinterpret_cast<const float4*>(p);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (valid > 0) v.x = p[0];
  if (valid > 1) v.y = p[1];
  if (valid > 2) v.z = p[2];
  if (valid > 3) v.w = p[3];
  return v;
}

__device__ __forceinline__ float apply_epi(int epi, float acc, int row, int col, const float* __restrict__ bias,
                                           const float* __restrict__ aux, int ldaux) {
  switch (epi) {
    case EPI_BIAS: return acc + bias[col];
    case EPI_BIAS_TANH: return fast_tanh(acc + bias[col]);
    case EPI_TANH_GRAD: {
      float h = aux[(size_t)row * ldaux + col];
      return acc * (1.f - h * h);
    }
    default: return acc;
  }
}

// The epilogue of a 128x128 tile: the MFMA accumulators (four 32x32 blocks
// per wave) to C (bias, tanh, tanh gradient, column partials) or to the
// split-K workspace.  scr0 / scr1: two LDS areas of at least 1280 and 512
// floats that no wave reads any more (the operand tiles after the k-loop's
// last barrier).
// FULLT: the tile lies inside C (no bounds tests on the stores).
template <bool FULLT = false>
__device__ __forceinline__ void gemm_epilogue(floatx16 (&acc)[2][2], float* scr0, float* scr1, int m0, int n0, int by,
                                              int bz, int M, int N, float* __restrict__ C, int ldc, int epi,
                                              const float* __restrict__ bias, const float* __restrict__ aux, int ldaux,
                                              float* __restrict__ ws, float* __restrict__ cs,
                                              const float* __restrict__ cw, int ncw) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, r = lane & 31;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  // Accumulator layout of a 32x32 MFMA block: register v of lane l holds
  // row 8*(v/4) + 4*(l/32) + v%4, column l%32.
  if (!ws && epi == EPI_TANH_GRAD) {
    // per 32x32 block: issue its 16 loads of the tanh outputs, then use them
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int tj = 0; tj < 2; ++tj) {
        const int col = n0 + wn + tj * 32 + r;
        float hv[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + wm + ti * 32 + (v >> 2) * 8 + h * 4 + (v & 3);
          hv[v] = (row < M && col < N) ? aux[(size_t)row * ldaux + col] : 0.f;
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + wm + ti * 32 + (v >> 2) * 8 + h * 4 + (v & 3);
          acc[ti][tj][v] *= 1.f - hv[v] * hv[v];
          if (row < M && col < N) C[(size_t)row * ldc + col] = acc[ti][tj][v];
        }
      }
    if (cs) {
      // column sums of the 128-row tile just stored, weighted by the ncw
      // columns of cw ([M][ncw]) and plain: each lane sums its 32 rows of
      // column wn + tj*32 + r, lanes r and r+32 (the other four rows of
      // every group of eight) are added, then the two waves sharing the
      // columns, top half first; the tile writes rows q < ncw (weighted by
      // cw[.][q]) and ncw (plain) of its partials.  The k-loop's last
      // barrier has retired every read of the operand tiles, so the
      // weights are staged in one of them and the sums meet in the other.
      float* red = scr0;
      if (ncw) {
        // [q][BM] weights of the tile's rows, zero past M (where the
        // accumulators are zero too: those A rows were loaded as zeros)
        float* wt = scr1;
        for (int i = tid; i < ncw * BM; i += 256) {
          const int rr = i / ncw, q = i - rr * ncw;
          wt[q * BM + rr] = m0 + rr < M ? cw[(size_t)m0 * ncw + i] : 0.f;
        }
        __syncthreads();
#pragma unroll 1
        for (int q = 0; q < ncw; ++q) {
          const float* wq = wt + q * BM + wm + h * 4;
          float s0 = 0.f, s1 = 0.f;
#pragma unroll
          for (int ti = 0; ti < 2; ++ti)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              // rows 8g + e (e < 4) of this lane's 32-row block
              const float4 w = *reinterpret_cast<const float4*>(wq + ti * 32 + g * 8);
              s0 = fmaf(w.x, acc[ti][0][g * 4 + 0], s0);
              s1 = fmaf(w.x, acc[ti][1][g * 4 + 0], s1);
              s0 = fmaf(w.y, acc[ti][0][g * 4 + 1], s0);
              s1 = fmaf(w.y, acc[ti][1][g * 4 + 1], s1);
              s0 = fmaf(w.z, acc[ti][0][g * 4 + 2], s0);
              s1 = fmaf(w.z, acc[ti][1][g * 4 + 2], s1);
              s0 = fmaf(w.w, acc[ti][0][g * 4 + 3], s0);
              s1 = fmaf(w.w, acc[ti][1][g * 4 + 3], s1);
            }
          s0 += __shfl_xor(s0, 32, 64);
          s1 += __shfl_xor(s1, 32, 64);
          red[(q * 4 + wave) * 64 + lane] = lane < 32 ? s0 : s1;
        }
      }
      float s[2];
#pragma unroll
      for (int tj = 0; tj < 2; ++tj) {
        s[tj] = 0.f;
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int row = m0 + wm + ti * 32 + (v >> 2) * 8 + h * 4 + (v & 3);
            s[tj] += row < M ? acc[ti][tj][v] : 0.f;
          }
        s[tj] += __shfl_xor(s[tj], 32, 64);
      }
      red[(ncw * 4 + wave) * 64 + lane] = lane < 32 ? s[0] : s[1];
      __syncthreads();
      if (wave < 2) {
        const int col = n0 + wn + lane;
        if (col < N)
          for (int q = 0; q <= ncw; ++q)
            cs[((size_t)by * (ncw + 1) + q) * N + col] = red[(q * 4 + wave) * 64 + lane] + red[(q * 4 + wave + 2) * 64 + lane];
      }
    }
    return;
  }
  // one uniform branch per epilogue kind, then a straight store loop
  auto store_all = [&](auto f) {
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int tj = 0; tj < 2; ++tj) {
        const int col = n0 + wn + tj * 32 + r;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + wm + ti * 32 + (v >> 2) * 8 + h * 4 + (v & 3);
          if (FULLT || (row < M && col < N)) f(row, col, acc[ti][tj][v]);
        }
      }
  };
  if (ws) {
    store_all([&](int row, int col, float a) { ws[((size_t)bz * M + row) * N + col] = a; });
  } else if (epi == EPI_BIAS_TANH) {
    store_all([&](int row, int col, float a) { C[(size_t)row * ldc + col] = fast_tanh(a + bias[col]); });
  } else if (epi == EPI_BIAS) {
    store_all([&](int row, int col, float a) { C[(size_t)row * ldc + col] = a + bias[col]; });
  } else {
    store_all([&](int row, int col, float a) { C[(size_t)row * ldc + col] = a; });
  }
}

// A_KMAJ: A stored [K][M] (else [M][K]); B_NK: B stored [N][K] (else [K][N]).
// VA / VB: the operand's rows are 16-byte aligned, so its tiles load as
// float4 (the heads' 127-column weights are not, their activations are).
// FULL: every tile and k-step lies inside the matrices and both operands
// are aligned, with byte extents below 2^31: tiles load by raw buffer
// loads, the thread's offset fixed in a VGPR and the k-step's in an SGPR,
// with no bounds tests (the generic path spends ~80 VALU and SALU
// instructions per k-step on them).
template <int BK, bool A_KMAJ, bool B_NK, bool VA, bool VB, bool FULL = false>
__global__ __launch_bounds__(256, BK == 16 ? 4 : 2) void k_gemm(const float* __restrict__ A, const float* __restrict__ B,
                                              float* __restrict__ C, int M, int N, int K, int lda, int ldb, int ldc,
                                              int epi, const float* __restrict__ bias, const float* __restrict__ aux,
                                              int ldaux, int kchunk, float* __restrict__ ws,
                                              float* __restrict__ cs, const float* __restrict__ cw, int ncw) {
  static_assert(BK == 16 || BK == 32, "k-step depth");
  // float4 loads per thread per operand tile
  constexpr int LPT = BM * BK / 4 / 256;
  constexpr int LDSROW_T = ldsrow_t<BK>();
  __shared__ __align__(16) float As_[2][BK * LDSROW];
  __shared__ float Bs_[2][BK * LDSROW];
  constexpr int RA = A_KMAJ ? LDSROW : LDSROW_T;  // A is transposed when stored [M][K]
  constexpr int RB = B_NK ? LDSROW_T : LDSROW;    // B is transposed when stored [N][K]
  auto As = [&](int b, int k, int m) -> float& { return As_[b][k * RA + m]; };
  auto Bs = [&](int b, int k, int n) -> float& { return Bs_[b][k * RB + n]; };

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, r = lane & 31;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  // Workgroups are dealt to the 8 XCDs round-robin by launch order; renumber
  // them (over the whole grid, split index outermost) so that each XCD runs a
  // contiguous run of tiles: the N tiles of one row block share their A rows,
  // and the tiles of one k-split share both operand chunks, in that XCD's L2.
  int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  {
    const int tiles = gridDim.x * gridDim.y, total = tiles * gridDim.z;
    if (total % 8 == 0) {
      const int hw = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
      const int lg = (hw % 8) * (total / 8) + hw / 8;
      bz = lg / tiles;
      bx = (lg % tiles) % gridDim.x;
      by = (lg % tiles) / gridDim.x;
    }
  }
  const int m0 = by * BM, n0 = bx * BN;
  const int kbeg = bz * kchunk;
  const int kend = min(K, kbeg + kchunk);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  float4 ra[LPT], rb[LPT];

  // FULL: per-thread byte offsets of its LPT float4 loads at k-step 0
  unsigned va_off[LPT], vb_off[LPT];
  if constexpr (FULL) {
#pragma unroll
    for (int p = 0; p < LPT; ++p) {
      const int q = tid + p * 256;
      if (!A_KMAJ) {
        const int i = q / (BK / 4), kq = (q % (BK / 4)) * 4;
        va_off[p] = 4u * (unsigned)((m0 + i) * lda + kq);
      } else {
        const int kk = q / (BM / 4), iq = (q % (BM / 4)) * 4;
        va_off[p] = 4u * (unsigned)(kk * lda + m0 + iq);
      }
      if (!B_NK) {
        const int kk = q / (BN / 4), jq = (q % (BN / 4)) * 4;
        vb_off[p] = 4u * (unsigned)(kk * ldb + n0 + jq);
      } else {
        const int j = q / (BK / 4), kq = (q % (BK / 4)) * 4;
        vb_off[p] = 4u * (unsigned)((n0 + j) * ldb + kq);
      }
    }
  }

  auto load_tile = [&](int k0) {
    if constexpr (FULL) {
      const auto rsa = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A), 0,
                                                         (int)(4u * (unsigned)(A_KMAJ ? K * lda : M * lda)), 0x00020000);
      const auto rsb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), 0,
                                                         (int)(4u * (unsigned)(B_NK ? N * ldb : K * ldb)), 0x00020000);
      // k-step offset: along k within a row, or k rows down
      const unsigned sa = 4u * (unsigned)(A_KMAJ ? k0 * lda : k0);
      const unsigned sb = 4u * (unsigned)(B_NK ? k0 : k0 * ldb);
#pragma unroll
      for (int p = 0; p < LPT; ++p) {
        ra[p] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsa, va_off[p], sa, 0));
        rb[p] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsb, vb_off[p], sb, 0));
      }
      return;
    }
#pragma unroll
    for (int p = 0; p < LPT; ++p) {
      const int q = tid + p * 256;
      if (!A_KMAJ) {  // [M][K]: float4 along k, BK/4 per row
        const int i = q / (BK / 4), kq = (q % (BK / 4)) * 4;
        const int row = m0 + i, k = k0 + kq;
        int valid = (row < M) ? min(4, kend - k) : 0;
        ra[p] = load4<VA>(A + (size_t)row * lda + k, valid);
      } else {  // [K][M]: float4 along m
        const int kk = q / (BM / 4), iq = (q % (BM / 4)) * 4;
        const int k = k0 + kk, col = m0 + iq;
        int valid = (k < kend) ? min(4, M - col) : 0;
        ra[p] = load4<VA>(A + (size_t)k * lda + col, valid);
      }
      if (!B_NK) {  // [K][N]: float4 along n
        const int kk = q / (BN / 4), jq = (q % (BN / 4)) * 4;
        const int k = k0 + kk, col = n0 + jq;
        int valid = (k < kend) ? min(4, N - col) : 0;
        rb[p] = load4<VB>(B + (size_t)k * ldb + col, valid);
      } else {  // [N][K]: float4 along k
        const int j = q / (BK / 4), kq = (q % (BK / 4)) * 4;
        const int col = n0 + j, k = k0 + kq;
        int valid = (col < N) ? min(4, kend - k) : 0;
        rb[p] = load4<VB>(B + (size_t)col * ldb + k, valid);
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int p = 0; p < LPT; ++p) {
      const int q = tid + p * 256;
      if (!A_KMAJ) {
        const int i = q / (BK / 4), kq = (q % (BK / 4)) * 4;
        As(buf, kq + 0, i) = ra[p].x;
        As(buf, kq + 1, i) = ra[p].y;
        As(buf, kq + 2, i) = ra[p].z;
        As(buf, kq + 3, i) = ra[p].w;
      } else {
        const int kk = q / (BM / 4), iq = (q % (BM / 4)) * 4;
        *reinterpret_cast<float4*>(&As(buf, kk, iq)) = ra[p];
      }
      if (!B_NK) {
        const int kk = q / (BN / 4), jq = (q % (BN / 4)) * 4;
        *reinterpret_cast<float4*>(&Bs(buf, kk, jq)) = rb[p];
      } else {
        const int j = q / (BK / 4), kq = (q % (BK / 4)) * 4;
        Bs(buf, kq + 0, j) = rb[p].x;
        Bs(buf, kq + 1, j) = rb[p].y;
        Bs(buf, kq + 2, j) = rb[p].z;
        Bs(buf, kq + 3, j) = rb[p].w;
      }
    }
  };

  int buf = 0;
  if (kbeg < kend) {
    load_tile(kbeg);
    store_tile(0);
  }
  __syncthreads();
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) load_tile(k0 + BK);
    // operand fragments double-buffered in registers: step s+1's LDS reads
    // are issued before step s's four MFMAs
    float fa0[2], fa1[2], fb0[2], fb1[2];
    auto frag = [&](int st, int slot) {
      const int k = 2 * st + h;
      fa0[slot] = As(buf, k, wm + r);
      fa1[slot] = As(buf, k, wm + 32 + r);
      fb0[slot] = Bs(buf, k, wn + r);
      fb1[slot] = Bs(buf, k, wn + 32 + r);
    };
    frag(0, 0);
#pragma unroll
    for (int st = 0; st < BK / 2; ++st) {
      const int cur = st & 1;
      if (st + 1 < BK / 2) frag(st + 1, cur ^ 1);
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[cur], fb0[cur], acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[cur], fb1[cur], acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[cur], fb0[cur], acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[cur], fb1[cur], acc[1][1], 0, 0, 0);
      // keep the reads for the next step ahead of this step's MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // MFMA
    }
    if (more) store_tile(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  gemm_epilogue(acc, As_[0], As_[1], m0, n0, by, bz, M, N, C, ldc, epi, bias, aux, ldaux, ws, cs, cw, ncw);
}

// ---------------------------------------------------------------------------
// Split-bf16 GEMM (the same tiles, epilogues and operand layouts as k_gemm).
//
// Each fp32 operand value x is split exactly into three bfloat16 parts,
// x = h + m + l (h = bf16(x), m = bf16(x - h), l = bf16(x - h - m); each
// part carries the next 8 significant bits, so the three hold all 24), and
// a product is the sum of the six partial products whose significance
// reaches 2^-16 of h*h: l*h + h*l + m*m + m*h + h*m + h*h (smallest first),
// each exact in the fp32 accumulator of v_mfma_f32_32x32x16_bf16 (Henry,
// Tang and Heinecke, "Leveraging the bfloat16 Artificial Intelligence
// Datatype For Higher-Precision Computations", ARITH 2019: the "bf16x6"
// scheme).  The dropped terms (m*l, l*m, l*l) are below 2^-23 of |h*h|, so
// the result is as accurate as an fp32 product accumulated in fp32: against
// fp64, measured on this hardware, relative L2 errors 3.6e-8 / 3.4e-7 /
// 3.2e-6 at K = 16 / 512 / 32000 where the fp32 MFMA (32x32x2) gives
// 7.3e-8 / 3.9e-7 / 3.2e-6.  Six bf16 MFMAs of 32x32x16 take 192 cycles
// where the eight fp32 32x32x2 MFMAs of the same 32x32x16 product take 512.
// (Values beyond the largest bfloat16, |x| > 3.39e38, would split to
// infinities; inputs are never near.)
//
// LDS holds per k-step (BK = 16) and operand the three planes as
// [plane][k-half][128 rows][8 k-values] (16 bytes per row and half): a
// thread stages 8 k-values of one row (one 16-byte write per plane) and a
// wave's MFMA operand read (32 rows x 2 halves of 16 bytes) is contiguous.
// Double buffered: 48 KB per workgroup, three workgroups per CU.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two values rounded to bfloat16 as one packed word (v_cvt_pk_bf16_f32),
// and the rounded values back as fp32: the low half shifted up, the high
// half masked (one operation each, where converting each rounded value
// back on its own costs a second conversion and a shift).
__device__ __forceinline__ unsigned bf16_pair(float a, float b, float& ra, float& rb) {
  const bf16x2 p = {(__bf16)a, (__bf16)b};
  unsigned u = __builtin_bit_cast(unsigned, p);
  // (opaque: else the compiler converts a again on its own for the low half)
  asm("" : "+v"(u));
  ra = __builtin_bit_cast(float, u << 16);
  rb = __builtin_bit_cast(float, u & 0xffff0000u);
  return u;
}

__device__ __forceinline__ void split8(const float (&x)[8], uint4& ph, uint4& pm, uint4& pl) {
  unsigned h[4], m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a0, a1, b0, b1;
    h[i] = bf16_pair(x[2 * i], x[2 * i + 1], a0, a1);
    const float r0 = x[2 * i] - a0, r1 = x[2 * i + 1] - a1;
    m[i] = bf16_pair(r0, r1, b0, b1);
    const bf16x2 q = {(__bf16)(r0 - b0), (__bf16)(r1 - b1)};
    l[i] = __builtin_bit_cast(unsigned, q);
  }
  ph = make_uint4(h[0], h[1], h[2], h[3]);
  pm = make_uint4(m[0], m[1], m[2], m[3]);
  pl = make_uint4(l[0], l[1], l[2], l[3]);
}

// BPL: B arrives already split (DGEN_HIP_K_SPLIT_BF16 planes in bpl, K8
// groups of 8 k-values per column): its tile loads are one 16-byte load per
// plane and nothing is split in the tile (B_NK and VB are then unused).
template <bool A_KMAJ, bool B_NK, bool VA, bool VB, bool FULL, bool BPL>
__global__ __launch_bounds__(256, 3) void k_gemm_x6(const float* __restrict__ A, const float* __restrict__ B,
                                                    float* __restrict__ C, int M, int N, int K, int lda, int ldb,
                                                    int ldc, int epi, const float* __restrict__ bias,
                                                    const float* __restrict__ aux, int ldaux, int kchunk,
                                                    float* __restrict__ ws, float* __restrict__ cs,
                                                    const float* __restrict__ cw, int ncw,
                                                    const uint4* __restrict__ bpl, int K8) {
  constexpr int BK = 16;
  // [buffer][operand][plane][k-half][row]: 8 bf16 per entry
  __shared__ uint4 Xs[2][2][3][2][BM];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, r = lane & 31;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  {
    // XCD-contiguous tile order, as in k_gemm
    const int tiles = gridDim.x * gridDim.y, total = tiles * gridDim.z;
    if (total % 8 == 0) {
      const int hw = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
      const int lg = (hw % 8) * (total / 8) + hw / 8;
      bz = lg / tiles;
      bx = (lg % tiles) % gridDim.x;
      by = (lg % tiles) / gridDim.x;
    }
  }
  const int m0 = by * BM, n0 = bx * BN;
  const int kbeg = bz * kchunk;
  const int kend = min(K, kbeg + kchunk);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // staging: thread (si, sh) holds k-values 8*sh .. 8*sh+7 of row si of
  // each operand tile (A row m0+si, B column n0+si)
  const int si = tid & (BM - 1), sh = tid >> 7;
  float xa[8], xb[BPL ? 1 : 8];
  uint4 pb[BPL ? 3 : 1];
  auto load_tile = [&](int k0) {
    const int kk = k0 + 8 * sh;
    if (!A_KMAJ) {  // [M][K]: 8 consecutive values of one row
      const int row = m0 + si;
      const float* p = A + (size_t)row * lda + kk;
      if (FULL || (VA && row < M && kk + 8 <= kend)) {
        const float4 u = *reinterpret_cast<const float4*>(p), w = *reinterpret_cast<const float4*>(p + 4);
        xa[0] = u.x; xa[1] = u.y; xa[2] = u.z; xa[3] = u.w;
        xa[4] = w.x; xa[5] = w.y; xa[6] = w.z; xa[7] = w.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xa[j] = (row < M && kk + j < kend) ? p[j] : 0.f;
      }
    } else {  // [K][M]: one value in each of 8 rows (coalesced across the wave)
      const int col = m0 + si;
      if constexpr (FULL) {
        // raw buffer loads: the lane's column in a VGPR, each row's offset in
        // an SGPR (sh is uniform in a wave), no address arithmetic per load
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A), 0, (int)(4u * (unsigned)(K * lda)),
                                                          0x00020000);
        const int ku = k0 + 8 * __builtin_amdgcn_readfirstlane(sh);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          xa[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, 4u * (unsigned)col,
                                                                                  (int)(4u * (unsigned)((ku + j) * lda)), 0));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          xa[j] = (col < M && kk + j < kend) ? A[(size_t)(kk + j) * lda + col] : 0.f;
      }
    }
    if constexpr (BPL) {  // planes: 16 bytes per plane (zero past K8 and N)
      const int kg = (k0 >> 3) + sh, col = n0 + si;
      const bool ok = FULL || (col < N && kg < K8);
      const size_t plane = (size_t)K8 * N, at = (size_t)kg * N + col;
#pragma unroll
      for (int q = 0; q < 3; ++q) pb[q] = ok ? bpl[q * plane + at] : make_uint4(0u, 0u, 0u, 0u);
    } else if (!B_NK) {  // [K][N]
      const int col = n0 + si;
      if constexpr (FULL) {
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), 0, (int)(4u * (unsigned)(K * ldb)),
                                                          0x00020000);
        const int ku = k0 + 8 * __builtin_amdgcn_readfirstlane(sh);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          xb[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, 4u * (unsigned)col,
                                                                                  (int)(4u * (unsigned)((ku + j) * ldb)), 0));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          xb[j] = (col < N && kk + j < kend) ? B[(size_t)(kk + j) * ldb + col] : 0.f;
      }
    } else {  // [N][K]
      const int row = n0 + si;
      const float* p = B + (size_t)row * ldb + kk;
      if (FULL || (VB && row < N && kk + 8 <= kend)) {
        const float4 u = *reinterpret_cast<const float4*>(p), w = *reinterpret_cast<const float4*>(p + 4);
        xb[0] = u.x; xb[1] = u.y; xb[2] = u.z; xb[3] = u.w;
        xb[4] = w.x; xb[5] = w.y; xb[6] = w.z; xb[7] = w.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xb[j] = (row < N && kk + j < kend) ? p[j] : 0.f;
      }
    }
  };
  auto store_tile = [&](int buf) {
    uint4 p0, p1, p2;
    split8(xa, p0, p1, p2);
    Xs[buf][0][0][sh][si] = p0;
    Xs[buf][0][1][sh][si] = p1;
    Xs[buf][0][2][sh][si] = p2;
    if constexpr (BPL) {
      p0 = pb[0];
      p1 = pb[1];
      p2 = pb[2];
    } else {
      split8(xb, p0, p1, p2);
    }
    Xs[buf][1][0][sh][si] = p0;
    Xs[buf][1][1][sh][si] = p1;
    Xs[buf][1][2][sh][si] = p2;
  };

  int buf = 0;
  if (kbeg < kend) {
    load_tile(kbeg);
    store_tile(0);
  }
  __syncthreads();
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) load_tile(k0 + BK);
    // this wave's operand parts: rows wm + 32 ti + r of A, columns
    // wn + 32 tj + r of B, k-half h (8 values each)
    bf16x8 fa[2][3], fb[2][3];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        fa[t][q] = __builtin_bit_cast(bf16x8, Xs[buf][0][q][h][wm + 32 * t + r]);
        fb[t][q] = __builtin_bit_cast(bf16x8, Xs[buf][1][q][h][wn + 32 * t + r]);
      }
    // the six partial products, smallest first, each over the four blocks
    // (four independent accumulators between dependent MFMAs)
    constexpr int pa[6] = {2, 0, 1, 1, 0, 0}, pb[6] = {0, 2, 1, 0, 1, 0};
#pragma unroll
    for (int q = 0; q < 6; ++q)
#pragma unroll
      for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
          acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ti][pa[q]], fb[tj][pb[q]], acc[ti][tj], 0, 0, 0);
    if (more) store_tile(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  gemm_epilogue(acc, reinterpret_cast<float*>(&Xs[0][0][0][0][0]), reinterpret_cast<float*>(&Xs[1][0][0][0][0]), m0,
                n0, by, bz, M, N, C, ldc, epi, bias, aux, ldaux, ws, cs, cw, ncw);
}

// Split-bf16 GEMM for full tiles of a row-major A and a pre-split B (the
// MLP's forward and data-gradient layers): both operand tiles of a k-step
// are copied global -> LDS by the load-to-LDS instructions (no staging
// registers), in two stages: each k-step waits for its own copies (at the
// barrier), starts the next k-step's copies into the other stage, then reads
// its fragments, splits A and runs the MFMAs while those copies land.  A
// stage holds the fp32 A tile (128 rows x 4 16-byte quarters, quarter q of
// row R in slot 4R + (q ^ f(R)), f(R) = ((R >> 1) ^ (R >> 3)) & 3, so the
// fragment reads are free of bank conflicts) and B's three planes
// ([plane][k-half][128 columns], 16 bytes each): 20 KB.  Three workgroups
// per CU (157 registers; at four the allocator spills, and the spill
// reloads wait behind the copies in flight).
__device__ __forceinline__ int aswz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void k_gemm_x6d(
    const float* __restrict__ A, float* __restrict__ C, int M, int N, int K, int lda, int ldc, int epi,
    const float* __restrict__ bias, const float* __restrict__ aux, int ldaux, float* __restrict__ cs,
    const float* __restrict__ cw, int ncw, const uint4* __restrict__ bpl, int K8) {
  constexpr int BK = 16, ASLOTS = BM * 4, SLOTS = ASLOTS + 3 * 2 * BN;
  // the two stages are separate LDS objects: a read of one is then not held
  // back by the copies in flight to the other
  __shared__ uint4 L0[SLOTS];
  __shared__ uint4 L1[SLOTS];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, r = lane & 31;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  int bx = blockIdx.x, by = blockIdx.y;
  {
    const int total = gridDim.x * gridDim.y;
    if (total % 8 == 0) {
      const int hw = blockIdx.y * gridDim.x + blockIdx.x;
      const int lg = (hw % 8) * (total / 8) + hw / 8;
      bx = lg % gridDim.x;
      by = lg / gridDim.x;
    }
  }
  const int m0 = by * BM, n0 = bx * BN;
  // this lane's copies (element offsets): A slots (2w + i)*64 + lane, B
  // slots (3w + j)*64 + lane
  unsigned aoff[2], boff[3];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int s = (wave * 2 + i) * 64 + lane, row = s >> 2, q = (s & 3) ^ aswz(row);
    aoff[i] = (unsigned)((m0 + row) * lda + 4 * q);
  }
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int u = (wave * 3 + j) * 64 + lane, p = u / (2 * BN), hh = (u / BN) & 1, col = u % BN;
    boff[j] = (unsigned)((p * K8 + hh) * N + n0 + col);
  }
  auto issue = [&](uint4* Ld, int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(A + aoff[i] + k0),
                                       (__attribute__((address_space(3))) void*)&Ld[(wave * 2 + i) * 64], 16, 0, 0);
#pragma unroll
    for (int j = 0; j < 3; ++j)
      __builtin_amdgcn_global_load_lds((const void*)(bpl + boff[j] + (unsigned)((k0 >> 3) * N)),
                                       (__attribute__((address_space(3))) void*)&Ld[ASLOTS + (wave * 3 + j) * 64], 16,
                                       0, 0);
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // one k-step on the stage in Lc, the next one's copies into Ln
  auto step = [&](const uint4* Lc, uint4* Ln, int knext) {
    // this stage's copies landed (the barrier waits for them) and every
    // wave is done reading Ln
    __syncthreads();
    if (knext < K) issue(Ln, knext);
    bf16x8 fb[2][3];
#pragma unroll
    for (int tj = 0; tj < 2; ++tj)
#pragma unroll
      for (int q = 0; q < 3; ++q) fb[tj][q] = __builtin_bit_cast(bf16x8, Lc[ASLOTS + (q * 2 + h) * BN + wn + 32 * tj + r]);
    constexpr int pa[6] = {2, 0, 1, 1, 0, 0}, pb[6] = {0, 2, 1, 0, 1, 0};
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
      const int R = wm + 32 * ti + r, f = aswz(R);
      const float4 x0 = __builtin_bit_cast(float4, Lc[4 * R + ((2 * h) ^ f)]);
      const float4 x1 = __builtin_bit_cast(float4, Lc[4 * R + ((2 * h + 1) ^ f)]);
      const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      uint4 u0, u1, u2;
      split8(x, u0, u1, u2);
      const bf16x8 fa[3] = {__builtin_bit_cast(bf16x8, u0), __builtin_bit_cast(bf16x8, u1),
                            __builtin_bit_cast(bf16x8, u2)};
#pragma unroll
      for (int q = 0; q < 6; ++q)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj)
          acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[pa[q]], fb[tj][pb[q]], acc[ti][tj], 0, 0, 0);
    }
  };

  issue(L0, 0);
  // K is a multiple of 2 * BK here: the stages alternate L0, L1
  for (int k0 = 0; k0 < K; k0 += 2 * BK) {
    step(L0, L1, k0 + BK);
    step(L1, L0, k0 + 2 * BK);
  }
  // every wave's reads of the last stage done before the epilogue's LDS use
  __syncthreads();
  gemm_epilogue<true>(acc, reinterpret_cast<float*>(&L0[0]), reinterpret_cast<float*>(&L1[0]), m0, n0, by, 0, M, N,
                      C, ldc, epi, bias, aux, ldaux, nullptr, cs, cw, ncw);
}

// Three bfloat16 planes of an fp32 matrix, for an operand that many tiles
// of the split-bf16 GEMM share (the weights): value (k, n) at
// src[k*ldk + n*ldn] (0 <= k < K, 0 <= n < N) goes to plane p at
// dst[(p*K8 + k/8)*N + n] element k%8 (uint4 = 8 bf16; K8 = ceil(K/8); zero
// for k >= K): the 8 k-values of column n that a GEMM thread stages are one
// 16-byte load per plane.
__global__ void k_split_bf16(const float* __restrict__ src, uint4* __restrict__ dst, int K, int N, int ldk, int ldn,
                             int K8) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= K8 * N) return;
  const int kg = i / N, n = i - kg * N;
  float x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = kg * 8 + j;
    x[j] = k < K ? src[(size_t)k * ldk + (size_t)n * ldn] : 0.f;
  }
  uint4 h, m, l;
  split8(x, h, m, l);
  const size_t plane = (size_t)K8 * N;
  dst[i] = h;
  dst[plane + i] = m;
  dst[2 * plane + i] = l;
}

int launch_split_bf16(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=src [1]=planes [2]=K [3]=N [4]=ld_k [5]=ld_n [6]=groups of 8 k-values (0: ceil(K/8))
  const int64_t src = op.arg[0], dst = op.arg[1], K = op.arg[2], N = op.arg[3], ldk = op.arg[4], ldn = op.arg[5];
  DGEN_REQUIRE(K > 0 && N > 0 && K < (1 << 24) && N < (1 << 24) && ldk >= 0 && ldn >= 0,
               "split_bf16: K %lld N %lld ld %lld %lld", (long long)K, (long long)N, (long long)ldk, (long long)ldn);
  const int64_t K8 = op.arg[6] > 0 ? op.arg[6] : (K + 7) / 8;
  DGEN_REQUIRE(K8 >= (K + 7) / 8 && K8 < (1 << 21), "split_bf16: %lld groups for K %lld", (long long)K8, (long long)K);
  DGEN_REQUIRE(K8 * N < (1ll << 31), "split_bf16: %lld x %lld too large", (long long)K, (long long)N);
  DGEN_REQUIRE(dst % 4 == 0, "split_bf16: planes cell %lld not 16-byte aligned", (long long)dst);
  DGEN_CHECK_CELL(L, src, (K - 1) * ldk + (N - 1) * ldn + 1, "split_bf16.src");
  DGEN_CHECK_CELL(L, dst, 3 * K8 * N * 4, "split_bf16.planes");
  if (L.dry) return 0;
  const int64_t n = K8 * N;
  hipLaunchKernelGGL(k_split_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, L.stream, cell(L, src),
                     reinterpret_cast<uint4*>(cell(L, dst)), (int)K, (int)N, (int)ldk, (int)ldn, (int)K8);
  DGEN_LAUNCH_CHECK("k_split_bf16");
  return 0;
}

// C = sum over the k-splits of the partial products, in split order, then
// the epilogue.  V4: each thread owns four consecutive columns (N, ldc and the
// workspace rows allow float4) and keeps 16 splits' loads in flight.
template <bool V4>
__global__ void k_splitk_reduce(const float* __restrict__ ws, float* __restrict__ C, int M, int N, int ldc, int splits,
                                int epi, const float* __restrict__ bias, const float* __restrict__ aux, int ldaux) {
  constexpr int CW = V4 ? 4 : 1;
  const size_t idx = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * CW;
  if (idx >= (size_t)M * N) return;
  const int row = (int)(idx / N), col = (int)(idx % N);
  const size_t plane = (size_t)M * N;
  float s[CW];
#pragma unroll
  for (int e = 0; e < CW; ++e) s[e] = 0.f;
  int z = 0;
  for (; z + 16 <= splits; z += 16) {
    float v[16][CW];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if constexpr (V4) {
        const float4 t = *reinterpret_cast<const float4*>(ws + (size_t)(z + q) * plane + idx);
        v[q][0] = t.x;
        v[q][1] = t.y;
        v[q][2] = t.z;
        v[q][3] = t.w;
      } else {
        v[q][0] = ws[(size_t)(z + q) * plane + idx];
      }
    }
#pragma unroll
    for (int q = 0; q < 16; ++q)
#pragma unroll
      for (int e = 0; e < CW; ++e) s[e] += v[q][e];
  }
  for (; z < splits; ++z)
#pragma unroll
    for (int e = 0; e < CW; ++e) s[e] += ws[(size_t)z * plane + idx + e];
#pragma unroll
  for (int e = 0; e < CW; ++e) C[(size_t)row * ldc + col + e] = apply_epi(epi, s[e], row, col + e, bias, aux, ldaux);
}

template <int BK, bool AK, bool BT, bool VA>
static void launch_vb(bool vb, dim3 g, hipStream_t s, const float* A, const float* B, float* C, int M, int N, int K,
                      int lda, int ldb, int ldc, int epi, const float* bias, const float* aux, int ldaux, int kchunk,
                      float* ws, float* cs, const float* cw, int ncw, bool full) {
  if constexpr (VA) {
    if (vb && full) {
      hipLaunchKernelGGL((k_gemm<BK, AK, BT, true, true, true>), g, dim3(256), 0, s, A, B, C, M, N, K, lda, ldb, ldc,
                         epi, bias, aux, ldaux, kchunk, ws, cs, cw, ncw);
      return;
    }
  }
  if (vb)
    hipLaunchKernelGGL((k_gemm<BK, AK, BT, VA, true>), g, dim3(256), 0, s, A, B, C, M, N, K, lda, ldb, ldc, epi, bias,
                       aux, ldaux, kchunk, ws, cs, cw, ncw);
  else
    hipLaunchKernelGGL((k_gemm<BK, AK, BT, VA, false>), g, dim3(256), 0, s, A, B, C, M, N, K, lda, ldb, ldc, epi, bias,
                       aux, ldaux, kchunk, ws, cs, cw, ncw);
}

template <int BK, bool AK, bool BT>
static void launch_variant(bool va, bool vb, dim3 g, hipStream_t s, const float* A, const float* B, float* C, int M,
                           int N, int K, int lda, int ldb, int ldc, int epi, const float* bias, const float* aux,
                           int ldaux, int kchunk, float* ws, float* cs, const float* cw, int ncw, bool full) {
  if (va)
    launch_vb<BK, AK, BT, true>(vb, g, s, A, B, C, M, N, K, lda, ldb, ldc, epi, bias, aux, ldaux, kchunk, ws, cs, cw, ncw, full);
  else
    launch_vb<BK, AK, BT, false>(vb, g, s, A, B, C, M, N, K, lda, ldb, ldc, epi, bias, aux, ldaux, kchunk, ws, cs, cw, ncw, full);
}

template <bool AK, bool BT>
static void launch_x6(bool va, bool vb, bool full, dim3 g, hipStream_t s, const float* A, const float* B, float* C,
                      int M, int N, int K, int lda, int ldb, int ldc, int epi, const float* bias, const float* aux,
                      int ldaux, int kchunk, float* ws, float* cs, const float* cw, int ncw, const uint4* bpl,
                      int K8) {
#define DGEN_X6(VA_, VB_, F_, P_)                                                                                   \
  hipLaunchKernelGGL((k_gemm_x6<AK, P_ ? false : BT, VA_, P_ || VB_, F_, P_>), g, dim3(256), 0, s, A, B, C, M, N, \
                     K, lda, ldb, ldc, epi, bias, aux, ldaux, kchunk, ws, cs, cw, ncw, bpl, K8)
  if (bpl) {
    if (full) DGEN_X6(true, true, true, true);
    else if (va) DGEN_X6(true, true, false, true);
    else DGEN_X6(false, true, false, true);
  } else if (full) DGEN_X6(true, true, true, false);
  else if (va && vb) DGEN_X6(true, true, false, false);
  else if (va) DGEN_X6(true, false, false, false);
  else if (vb) DGEN_X6(false, true, false, false);
  else DGEN_X6(false, false, false, false);
#undef DGEN_X6
}

template <int BK>
static void launch_layout(int64_t alay, int64_t blay, bool va, bool vb, dim3 g, hipStream_t s, const float* A,
                          const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc, int epi,
                          const float* bias, const float* aux, int ldaux, int kchunk, float* ws, float* cs,
                          const float* cw, int ncw, bool full) {
  if (alay == 0 && blay == 0)
    launch_variant<BK, false, false>(va, vb, g, s, A, B, C, M, N, K, lda, ldb, ldc, epi, bias, aux, ldaux, kchunk, ws,
                                     cs, cw, ncw, full);
  else if (alay == 0 && blay == 1)
    launch_variant<BK, false, true>(va, vb, g, s, A, B, C, M, N, K, lda, ldb, ldc, epi, bias, aux, ldaux, kchunk, ws,
                                    cs, cw, ncw, full);
  else if (alay == 1 && blay == 0)
    launch_variant<BK, true, false>(va, vb, g, s, A, B, C, M, N, K, lda, ldb, ldc, epi, bias, aux, ldaux, kchunk, ws,
                                    cs, cw, ncw, full);
  else
    launch_variant<BK, true, true>(va, vb, g, s, A, B, C, M, N, K, lda, ldb, ldc, epi, bias, aux, ldaux, kchunk, ws,
                                   cs, cw, ncw, full);
}

int launch_gemm(const Launch& L, const dgen_hip_op& op) {
  const int64_t A = op.arg[0], Bc = op.arg[1], Cc = op.arg[2], M = op.arg[3], N = op.arg[4], K = op.arg[5];
  const int64_t lda = op.arg[6], ldb = op.arg[7], ldc = op.arg[8], alay = op.arg[9], blay = op.arg[10];
  const int64_t epi = op.arg[11], bias = op.arg[12], aux = op.arg[13], ldaux = op.arg[14];
  const int64_t split = op.arg[15], ws = op.arg[16], colsum = op.arg[17], cwc = op.arg[18], ncw64 = op.arg[19];
  const int64_t mode = op.arg[20];
  // arg[21] is read with the split-bf16 products only (ops written before it
  // existed leave it 0)
  const int64_t planes = mode == 1 ? op.arg[21] : -1;
  DGEN_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31),
               "gemm: M %lld N %lld K %lld", (long long)M, (long long)N, (long long)K);
  DGEN_REQUIRE(alay == 0 || alay == 1, "gemm: a_layout %lld", (long long)alay);
  DGEN_REQUIRE(blay == 0 || blay == 1, "gemm: b_layout %lld", (long long)blay);
  DGEN_REQUIRE(epi >= 0 && epi <= 3, "gemm: epilogue %lld", (long long)epi);
  DGEN_REQUIRE(split >= 1 && split <= 1024, "gemm: split_k %lld", (long long)split);
  DGEN_REQUIRE(mode == 0 || mode == 1, "gemm: product mode %lld (0 fp32, 1 split bf16)", (long long)mode);
  // B's split-bf16 planes (DGEN_HIP_K_SPLIT_BF16 of op(B) as [K][N]), or -1
  const int64_t K8 = (K + 7) / 8;
  if (planes >= 0) {
    DGEN_REQUIRE(planes % 4 == 0, "gemm: B planes cell %lld not 16-byte aligned", (long long)planes);
    DGEN_CHECK_CELL(L, planes, 3 * K8 * N * 4, "gemm.B_planes");
  }
  DGEN_REQUIRE(ldc >= N, "gemm: ldc %lld < N %lld", (long long)ldc, (long long)N);
  DGEN_REQUIRE(alay == 0 ? lda >= K : lda >= M, "gemm: lda %lld too small", (long long)lda);
  DGEN_CHECK_CELL(L, A, alay == 0 ? (M - 1) * lda + K : (K - 1) * lda + M, "gemm.A");
  if (planes < 0) {  // with planes the kernels read B only through them
    DGEN_REQUIRE(blay == 0 ? ldb >= N : ldb >= K, "gemm: ldb %lld too small", (long long)ldb);
    DGEN_CHECK_CELL(L, Bc, blay == 0 ? (K - 1) * ldb + N : (N - 1) * ldb + K, "gemm.B");
  }
  DGEN_CHECK_CELL(L, Cc, (M - 1) * ldc + N, "gemm.C");
  if (epi == EPI_BIAS || epi == EPI_BIAS_TANH) DGEN_CHECK_CELL(L, bias, N, "gemm.bias");
  if (epi == EPI_TANH_GRAD) {
    DGEN_REQUIRE(ldaux >= N, "gemm: ld aux %lld", (long long)ldaux);
    DGEN_CHECK_CELL(L, aux, (M - 1) * ldaux + N, "gemm.aux");
  }
  constexpr int BK = 16;
  // k-chunk per split, a multiple of BK
  int64_t kchunk = (K + split - 1) / split;
  kchunk = (kchunk + BK - 1) / BK * BK;
  const int64_t splits = (K + kchunk - 1) / kchunk;
  if (split > 1) DGEN_CHECK_CELL(L, ws, splits * M * N, "gemm.workspace");
  const int ncw = colsum >= 0 && ncw64 > 0 ? (int)ncw64 : 0;
  if (colsum >= 0) {
    DGEN_REQUIRE(epi == EPI_TANH_GRAD && splits == 1, "gemm: column partials need the tanh-gradient epilogue, no split");
    DGEN_REQUIRE(ncw64 >= 0 && ncw64 <= 4, "gemm: %lld column-sum weights (0..4)", (long long)ncw64);
    DGEN_CHECK_CELL(L, colsum, (M + BM - 1) / BM * (ncw + 1) * N, "gemm.column_partials");
    if (ncw) DGEN_CHECK_CELL(L, cwc, M * ncw, "gemm.column_weights");
  }
  DGEN_REQUIRE((M + BM - 1) / BM <= 65535 && splits <= 65535, "gemm: grid too large");
  if (L.dry) return 0;
  const bool va = (lda % 4 == 0) && (A % 4 == 0), vb = (ldb % 4 == 0) && (Bc % 4 == 0);
  // full tiles and k-steps, and byte extents that fit the buffer loads' 32-bit offsets
  const int64_t ext_a = 4 * (alay ? K * lda : M * lda), ext_b = 4 * (blay ? N * ldb : K * ldb);
  const bool full = va && vb && M % BM == 0 && N % BN == 0 && K % BK == 0 && ext_a < (1ll << 31) &&
                    ext_b < (1ll << 31);
  dim3 g((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM), (unsigned)splits);
  const float* pa = cell(L, A);
  const float* pb = cell(L, Bc);
  float* pc = cell(L, Cc);
  const float* pbias = (epi == EPI_BIAS || epi == EPI_BIAS_TANH) ? cell(L, bias) : nullptr;
  const float* paux = epi == EPI_TANH_GRAD ? cell(L, aux) : nullptr;
  float* pws = split > 1 ? cell(L, ws) : nullptr;
  float* pcs = colsum >= 0 ? cell(L, colsum) : nullptr;
  const float* pcw = ncw ? cell(L, cwc) : nullptr;
  const int e = split > 1 ? EPI_NONE : (int)epi;
  if (mode == 1) {
    const uint4* pbpl = planes >= 0 ? reinterpret_cast<const uint4*>(cell(L, planes)) : nullptr;
    // (full tiles: raw buffer loads over the operands, so their byte extents stay below 2^31)
    const bool full6 = va && (vb || pbpl) && M % BM == 0 && N % BN == 0 && K % BK == 0 && ext_a < (1ll << 31) &&
                       ext_b < (1ll << 31);
#define DGEN_X6L(AK_, BT_)                                                                                          \
  launch_x6<AK_, BT_>(va, vb, full6, g, L.stream, pa, pb, pc, M, N, K, lda, ldb, ldc, e, pbias, paux, ldaux, kchunk, \
                      pws, pcs, pcw, ncw, pbpl, (int)K8)
    if (pbpl && full6 && alay == 0 && splits == 1 && K % 32 == 0 && (int64_t)M * lda < (1ll << 32) &&
        3 * K8 * N < (1ll << 32)) {
      hipLaunchKernelGGL(k_gemm_x6d, g, dim3(256), 0, L.stream, pa, pc, (int)M, (int)N, (int)K, (int)lda, (int)ldc, e,
                         pbias, paux, (int)ldaux, pcs, pcw, ncw, pbpl, (int)K8);
    } else if (alay == 0 && blay == 0) DGEN_X6L(false, false);
    else if (alay == 0) DGEN_X6L(false, true);
    else if (blay == 0) DGEN_X6L(true, false);
    else DGEN_X6L(true, true);
#undef DGEN_X6L
    DGEN_LAUNCH_CHECK("k_gemm_x6");
  } else {
    launch_layout<BK>(alay, blay, va, vb, g, L.stream, pa, pb, pc, M, N, K, lda, ldb, ldc, e, pbias, paux, ldaux,
                      kchunk, pws, pcs, pcw, ncw, full);
    DGEN_LAUNCH_CHECK("k_gemm");
  }
  if (split > 1) {
    const size_t total = (size_t)M * N;
    if (N % 4 == 0 && ws % 4 == 0)
      hipLaunchKernelGGL(k_splitk_reduce<true>, dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0, L.stream, pws,
                         pc, (int)M, (int)N, (int)ldc, (int)splits, (int)epi, pbias, paux, (int)ldaux);
    else
      hipLaunchKernelGGL(k_splitk_reduce<false>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, L.stream, pws,
                         pc, (int)M, (int)N, (int)ldc, (int)splits, (int)epi, pbias, paux, (int)ldaux);
    DGEN_LAUNCH_CHECK("k_splitk_reduce");
  }
  return 0;
}

}  // namespace dgen
