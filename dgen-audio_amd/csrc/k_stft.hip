// Hop-gated STFT round trip with learnable per-bin gains, and the gain
// gradient.
//
// Reference graph (the DGenLazy idiom of Tests/DGenLazyTests/
// STFTIdentityTests.swift:152-187): frame = x.buffer(size: N, hop: H)
// .reshape([N]) * hann(N) (bufferView, Sources/DGen/HigherOps.swift:738-792);
// (re, im) = signalTensorFFT(frame) (tensorFFT, HigherOps+FFT.swift:16-34);
// the spectrum times the gains; signalTensorIFFT (:36-59: real part, 1/N);
// overlapAdd(hop: H) (Emit+FFT.swift:6-62), so that
//   y[t] = sum over hop frames h (multiples of H) of z_h[t - h], 0 <= t-h < N,
// where window h holds x[h-N+1 .. h] (zero before frame 0).  The gains
// g[0..N/2] scale the one-sided spectrum as its Hermitian reconstruction:
// bins k and N-k both by g_k.
//
// k_stft_fwd: a workgroup owns an output tile [a0, a0 + kTile) of one signal
// and every window whose outputs reach it (hop frames in (a0-N, a0+kTile)),
// recomputing the few that straddle the tile's left edge instead of
// exchanging partial sums.  A real N-point transform is an N/2-point complex
// FFT (fft_lds.h) plus the even/odd split; after the gains, the Hermitian
// pre-processing and an N/2-point inverse FFT give two real output samples
// per complex value.  W windows (one per M/8-thread slot) are transformed at
// once, then their outputs are gathered into the tile accumulator position
// by position in window order (atomic-free, deterministic).  The tile then
// yields y, dL/dy = 2 (y - x)/T and its share of the loss sum (y - x)^2 / T.
//
// k_stft_bwd: dL/dg_k = sum over windows (c_k/N) Re(X_k conj(E_k)), with X
// the window's spectrum, E the spectrum of dL/dy over the window's outputs
// (zero past T) and c_k = 1 at k = 0, N/2, else 2.  Each workgroup sums a run
// of windows of one signal into a partial row; the column sum reduces them.
#include "fft_lds.h"

namespace dgen {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 8192;   // output samples owned by a forward workgroup
constexpr int kRounds = 8;    // window rounds per backward workgroup

struct StftArgs {
  const float* x;      // [S][T]
  const float* win;    // [N]
  const float* gains;  // [N/2 + 1]
  const float* dyin;   // [S][T] (backward)
  float* y;            // [S][T] or null
  float* dy;           // [S][T] or null
  float* lossp;        // [S][ntiles] or null
  float* gpart;        // [S][nblk][N/2 + 1] (backward)
  int S, T, H, ntiles, nblk;
  float invT;
};

// Real N-point spectrum bins k and M-k (k = 0: bins 0 and M) from the
// N/2-point complex transform Z of the even/odd-packed signal.
__device__ __forceinline__ void split_bins(const SwzBuf& Z, int k, int M, float invN, c2& Xk, c2& Xm) {
  const int km = (M - k) & (M - 1);
  const c2 zk = Z[k], zm = Z[km];
  const c2 e = {0.5f * (zk.x + zm.x), 0.5f * (zk.y - zm.y)};
  const c2 o = {0.5f * (zk.y + zm.y), 0.5f * (zm.x - zk.x)};
  const c2 wk = cis(-(float)k * invN);
  const c2 wo = cmul(wk, o);
  Xk = cadd(e, wo);
  Xm = k == 0 ? c2{e.x - o.x, 0.0f} : cconj(csub(e, wo));
}

// split_bins on values already read: zk = Z[k], zm = Z[(M-k) mod M].
__device__ __forceinline__ void split_pair(c2 zk, c2 zm, int k, float invN, c2& Xk, c2& Xm) {
  const c2 e = {0.5f * (zk.x + zm.x), 0.5f * (zk.y - zm.y)};
  const c2 o = {0.5f * (zk.y + zm.y), 0.5f * (zm.x - zk.x)};
  const c2 wk = cis(-(float)k * invN);
  const c2 wo = cmul(wk, o);
  Xk = cadd(e, wo);
  Xm = k == 0 ? c2{e.x - o.x, 0.0f} : cconj(csub(e, wo));
}

// dst[0..n) = src[0..n): every load of the thread in flight before its LDS
// writes (a loop that stored each load as it arrived waited out one memory
// latency per iteration).
template <int n>
__device__ __forceinline__ void stage(float* dst, const float* __restrict__ src, int tid) {
  constexpr int Q = (n + kThreads - 1) / kThreads;
  float v[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) v[q] = src[min(tid + q * kThreads, n - 1)];
#pragma unroll
  for (int q = 0; q < Q; ++q)
    if (tid + q * kThreads < n) dst[tid + q * kThreads] = v[q];
}

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
  if (threadIdx.x == 0)
    for (int w = 0; w < kThreads / 64; ++w) t += red[w];
  return t;
}

struct FwdLds {
  float acc[kTile];
  c2 buf[2048];
  float gain[1025];
  float red[kThreads / 64];
};

template <int LOGN>
__global__ __launch_bounds__(kThreads) void k_stft_fwd(StftArgs a) {
  constexpr int N = 1 << LOGN, M = N / 2, LOGM = LOGN - 1, P = M / 8, W = kThreads / P;
  constexpr int U = M / 2 / P + 1;  // bin pairs per thread
  // a window's P threads lie in one wave when P <= 64: its transforms and
  // bins need only wave-level ordering; the gather reads every slot
  constexpr bool WL = P <= 64;
  static_assert(W * M == 2048, "window slots must fill the FFT buffer");
  __shared__ FwdLds L;
  const int tid = threadIdx.x, slot = tid / P, j = tid % P;
  const int s = blockIdx.y, tile = blockIdx.x, H = a.H;
  const int a0 = tile * kTile, a1 = min(a.T, a0 + kTile);
  const float* xs = a.x + (size_t)s * a.T;
  stage<M + 1>(L.gain, a.gains, tid);
  for (int i = tid; i < kTile; i += kThreads) L.acc[i] = 0.0f;
  // windows h = w*H with outputs [h, h+N) meeting [a0, a1)
  const int w_lo = a0 - N < 0 ? 0 : (a0 - N) / H + 1;
  const int w_hi = (a1 - 1) / H;
  const int nw = w_hi - w_lo + 1;
  const SwzBuf buf(L.buf, slot * M);
  const int sj = buf.part(j);
  // after the inverse transform a slot's region holds its N real outputs in
  // order: slot q's at zs + q * 2 * M
  const float* zs = reinterpret_cast<const float*>(L.buf);
  constexpr int kZStride = 2 * M;
  constexpr float invN = 1.0f / (float)N;
  // the window values this thread multiplies (samples 2n, 2n+1 of its first
  // pass inputs n), in registers for every round
  float2 hw[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int n = in_pos<M, pass_radix(LOGM, 0)>(j, e);
    hw[e] = float2{a.win[2 * n], a.win[2 * n + 1]};
  }
  // this thread's window samples of round r (element e of the first pass
  // needs samples 2n and 2n+1 of the window, n = in_pos(j, e)); the next
  // round's are loaded while this one is transformed and gathered
  float px[16];
  auto fetch = [&](int r0) {
    const int w = w_lo + r0 + slot;
    const bool live = w <= w_hi;
    const int h = w * H;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int n = in_pos<M, pass_radix(LOGM, 0)>(j, e);
      const int t0 = h - N + 1 + 2 * n;
      px[2 * e] = live && t0 >= 0 ? xs[t0] : 0.0f;
      px[2 * e + 1] = live && t0 + 1 >= 0 ? xs[t0 + 1] : 0.0f;
    }
  };
  __syncthreads();
  fetch(0);
  for (int r0 = 0; r0 < nw; r0 += W) {
    c2 v[8];
    int op[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = c2{px[2 * e] * hw[e].x, px[2 * e + 1] * hw[e].y};
    fft<LOGM, false, WL>(buf, j, v, op);
    if (r0 + W < nw) fetch(r0 + W);
    fft_store<LOGM>(buf, j, v);
    lds_sync<WL>();
    // gains on the one-sided spectrum, then the Hermitian inverse
    // pre-processing: z'_k = (G_k + conj G_{M-k}) + i (G_k - conj G_{M-k}) W_N^{-k}
    // (each thread owns the pairs k, M-k with k = j + u*P, so the update is
    // in place; all of a thread's spectrum reads are issued first)
    c2 zk[U], zm[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // k = j + u*P < M for every u (pairs past M/2 are read and skipped)
      zk[u] = buf.at(sj, u * P);
      zm[u] = buf[(M - j - u * P) & (M - 1)];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = j + u * P;
      if (k > M / 2) continue;
      c2 Xk, Xm;
      split_pair(zk[u], zm[u], k, invN, Xk, Xm);
      const float gk = L.gain[k], gm = L.gain[M - k];
      Xk = c2{Xk.x * gk, Xk.y * gk};
      Xm = c2{Xm.x * gm, Xm.y * gm};
      if (k == 0) {
        buf[0] = c2{Xk.x + Xm.x, Xk.x - Xm.x};
      } else {
        const c2 wk = cis(-(float)k * invN);
        const c2 o1 = cmul(c2{Xk.x - Xm.x, Xk.y + Xm.y}, cconj(wk));
        buf[k] = c2{(Xk.x + Xm.x) - o1.y, (Xk.y - Xm.y) + o1.x};
        if (k != M - k) {
          const c2 o2 = cmul(c2{Xm.x - Xk.x, Xm.y + Xk.y}, c2{-wk.x, -wk.y});
          buf[M - k] = c2{(Xm.x + Xk.x) - o2.y, (Xm.y - Xk.y) + o2.x};
        }
      }
    }
    lds_sync<WL>();
    fft_load<LOGM>(buf, j, v);
    lds_sync<WL>();
    fft<LOGM, true, WL>(buf, j, v, op);
    // complex output q holds samples 2q, 2q+1 (unnormalised): scale by 1/N
    float* zb = buf.raw();
#pragma unroll
    for (int e = 0; e < 8; ++e) *reinterpret_cast<float2*>(zb + 2 * op[e]) = float2{v[e].x * invN, v[e].y * invN};
    lds_barrier();
    // gather this round's windows into the tile, position by position
    const int wb = w_lo + r0, hb = wb * H;
    const int nq = min(W, w_hi - wb + 1);
    const int span = (nq - 1) * H + N;
    if constexpr (W <= 4) {
      // span <= W*N = 4096 (H <= N): 16 positions per thread, gathered 4
      // at a time with every slot read and accumulator read of a batch
      // issued before its first sum (a position loop waited out LDS latency
      // at every position); a slot that does not cover a position adds +0
      // (exact)
      constexpr int kPos = W * N / kThreads, kBatch = 4;
#pragma unroll
      for (int i0 = 0; i0 < kPos; i0 += kBatch) {
        float z[kBatch][W], ac[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          const int p = tid + (i0 + b) * kThreads;
#pragma unroll
          for (int q = 0; q < W; ++q) {
            const int ii = p - q * H;
            const bool ok = q < nq && ii >= 0 && ii < N;
            z[b][q] = zs[q * kZStride + (ok ? ii : 0)];
            z[b][q] = ok ? z[b][q] : 0.0f;
          }
          ac[b] = L.acc[min(max(hb + p - a0, 0), kTile - 1)];
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          const int p = tid + (i0 + b) * kThreads, t = hb + p;
          float sum = 0.0f;
#pragma unroll
          for (int q = 0; q < W; ++q) sum += z[b][q];
          if (p < span && t >= a0 && t < a1) L.acc[t - a0] = ac[b] + sum;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      for (int p = tid; p < span; p += kThreads) {
        const int t = hb + p;
        if (t < a0 || t >= a1) continue;
        float sum = 0.0f;
        for (int q = 0; q < nq; ++q) {
          const int i = p - q * H;
          if (i >= 0 && i < N) sum += zs[q * kZStride + i];
        }
        L.acc[t - a0] += sum;
      }
    }
    lds_barrier();
  }
  float ls = 0.0f;
  // the tile's input samples are loaded 8 at a time, all in flight before use
  for (int t8 = a0 + tid; t8 < a1; t8 += 8 * kThreads) {
    float xv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) xv[q] = xs[min(t8 + q * kThreads, a1 - 1)];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int t = t8 + q * kThreads;
      if (t >= a1) break;
      const float yv = L.acc[t - a0];
      const float d = yv - xv[q];
      const size_t i = (size_t)s * a.T + t;
      if (a.y) a.y[i] = yv;
      if (a.dy) a.dy[i] = 2.0f * d * a.invT;
      ls += d * d;
    }
  }
  if (a.lossp) {
    const float tot = block_sum(ls, L.red);
    if (tid == 0) a.lossp[(size_t)s * a.ntiles + tile] = tot * a.invT;
  }
}

struct BwdLds {
  c2 buf[2048];
  c2 aux[2048];
};

template <int LOGN>
__global__ __launch_bounds__(kThreads) void k_stft_bwd(StftArgs a) {
  constexpr int N = 1 << LOGN, M = N / 2, LOGM = LOGN - 1, P = M / 8, W = kThreads / P;
  constexpr int U = M / 2 / P + 1;  // bin pairs per thread
  constexpr bool WL = P <= 64;       // a window's threads lie in one wave
  static_assert(W * M == 2048, "window slots must fill the FFT buffer");
  __shared__ BwdLds L;
  const int tid = threadIdx.x, slot = tid / P, j = tid % P;
  const int s = blockIdx.y, blk = blockIdx.x, H = a.H;
  const int nwin = (a.T + H - 1) / H;
  const int wb = blk * kRounds * W, we = min(nwin, wb + kRounds * W);
  const float* xs = a.x + (size_t)s * a.T;
  const float* gs = a.dyin + (size_t)s * a.T;
  const SwzBuf buf(L.buf, slot * M);
  const SwzBuf spec(L.aux, slot * M);
  // the window values this thread multiplies, in registers for every round
  float2 hw[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int n = in_pos<M, pass_radix(LOGM, 0)>(j, e);
    hw[e] = float2{a.win[2 * n], a.win[2 * n + 1]};
  }
  constexpr float invN = 1.0f / (float)N;
  float acc_k[U], acc_m[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc_k[u] = acc_m[u] = 0.0f;
  __syncthreads();
  for (int r0 = 0; r0 < we - wb; r0 += W) {
    const int w = wb + r0 + slot;
    const bool live = w < we;
    const int h = w * H;
    {
      // the analysis window x[h-N+1 .. h] * hann (-> spec) and dL/dy over
      // the window's outputs [h, h+N) (-> buf), transformed together
      c2 vx[8], vg[8];
      int op[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int n = in_pos<M, pass_radix(LOGM, 0)>(j, e);
        const int t0 = h - N + 1 + 2 * n;
        const float x0 = live && t0 >= 0 ? xs[t0] : 0.0f;
        const float x1 = live && t0 + 1 >= 0 ? xs[t0 + 1] : 0.0f;
        vx[e] = c2{x0 * hw[e].x, x1 * hw[e].y};
        const int g0 = h + 2 * n;
        vg[e] = c2{live && g0 < a.T ? gs[g0] : 0.0f, live && g0 + 1 < a.T ? gs[g0 + 1] : 0.0f};
      }
      fft2<LOGM, false, WL>(spec, buf, j, vx, vg, op);
      fft_store<LOGM>(spec, j, vx);
      fft_store<LOGM>(buf, j, vg);
      lds_sync<WL>();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = j + u * P;
      if (k > M / 2) break;
      c2 Xk, Xm, Ek, Em;
      split_bins(spec, k, M, invN, Xk, Xm);
      split_bins(buf, k, M, invN, Ek, Em);
      acc_k[u] += Xk.x * Ek.x + Xk.y * Ek.y;
      acc_m[u] += Xm.x * Em.x + Xm.y * Em.y;
    }
    // the next round overwrites this slot's buffers
    lds_sync<WL>();
  }
  // every slot's reads are done before the partial rows reuse the buffers
  lds_barrier();
  // slots' partial sums -> one row: bins k (acc_k) and M-k (acc_m; bin M for k = 0)
  float* part = reinterpret_cast<float*>(L.buf);  // [W][M + 1]
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int k = j + u * P;
    if (k > M / 2) break;
    part[slot * (M + 1) + k] = acc_k[u];
    if (M - k != k) part[slot * (M + 1) + M - k] = acc_m[u];
  }
  lds_barrier();
  float* row = a.gpart + ((size_t)s * a.nblk + blk) * (M + 1);
  for (int b = tid; b <= M; b += kThreads) {
    float t = 0.0f;
    for (int q = 0; q < W; ++q) t += part[q * (M + 1) + b];
    const float ck = (b == 0 || b == M) ? 1.0f : 2.0f;
    row[b] = t * ck * invN;
  }
}

using StftKernel = void (*)(StftArgs);

StftKernel fwd_kernel(int logn) {
  switch (logn) {
    case 6: return k_stft_fwd<6>;
    case 7: return k_stft_fwd<7>;
    case 8: return k_stft_fwd<8>;
    case 9: return k_stft_fwd<9>;
    case 10: return k_stft_fwd<10>;
    case 11: return k_stft_fwd<11>;
    default: return nullptr;
  }
}

StftKernel bwd_kernel(int logn) {
  switch (logn) {
    case 6: return k_stft_bwd<6>;
    case 7: return k_stft_bwd<7>;
    case 8: return k_stft_bwd<8>;
    case 9: return k_stft_bwd<9>;
    case 10: return k_stft_bwd<10>;
    case 11: return k_stft_bwd<11>;
    default: return nullptr;
  }
}

int stft_shape(int64_t S, int64_t T, int64_t N, int64_t H, int& logn, const char* who) {
  logn = 0;
  while ((1ll << logn) < N) ++logn;
  DGEN_REQUIRE((1ll << logn) == N && logn >= 6 && logn <= 11, "%s: N %lld must be a power of two in [64, 2048]",
               who, (long long)N);
  DGEN_REQUIRE(S > 0 && S <= 65535 && T > 0 && T < (1ll << 30) && H >= 1 && H <= N,
               "%s: S %lld T %lld H %lld", who, (long long)S, (long long)T, (long long)H);
  return 0;
}

}  // namespace

int stft_windows_per_block(int64_t N) { return kRounds * (kThreads * 16 / (int)N); }
int stft_tile() { return kTile; }

int launch_stft_fwd(const Launch& L, const dgen_hip_op& op) {
  const int64_t x = op.arg[0], win = op.arg[1], gains = op.arg[2], y = op.arg[3], dy = op.arg[4], lossp = op.arg[5];
  const int64_t S = op.arg[6], T = op.arg[7], N = op.arg[8], H = op.arg[9];
  int logn;
  if (int rc = stft_shape(S, T, N, H, logn, "stft_fwd")) return rc;
  const int64_t ntiles = (T + kTile - 1) / kTile;
  DGEN_CHECK_CELL(L, x, S * T, "stft_fwd.x");
  DGEN_CHECK_CELL(L, win, N, "stft_fwd.window");
  DGEN_CHECK_CELL(L, gains, N / 2 + 1, "stft_fwd.gains");
  if (y >= 0) DGEN_CHECK_CELL(L, y, S * T, "stft_fwd.y");
  if (dy >= 0) DGEN_CHECK_CELL(L, dy, S * T, "stft_fwd.dy");
  if (lossp >= 0) DGEN_CHECK_CELL(L, lossp, S * ntiles, "stft_fwd.loss_partials");
  DGEN_REQUIRE(ntiles <= (1ll << 31) - 1, "stft_fwd: too many tiles");
  if (L.dry) return 0;
  StftArgs a{};
  a.x = cell(L, x);
  a.win = cell(L, win);
  a.gains = cell(L, gains);
  a.y = y >= 0 ? cell(L, y) : nullptr;
  a.dy = dy >= 0 ? cell(L, dy) : nullptr;
  a.lossp = lossp >= 0 ? cell(L, lossp) : nullptr;
  a.S = (int)S;
  a.T = (int)T;
  a.H = (int)H;
  a.ntiles = (int)ntiles;
  a.invT = 1.0f / (float)T;
  hipLaunchKernelGGL(fwd_kernel(logn), dim3((unsigned)ntiles, (unsigned)S), dim3(kThreads), 0, L.stream, a);
  DGEN_LAUNCH_CHECK("k_stft_fwd");
  return 0;
}

int launch_stft_bwd(const Launch& L, const dgen_hip_op& op) {
  const int64_t x = op.arg[0], win = op.arg[1], dy = op.arg[2], gpart = op.arg[3];
  const int64_t S = op.arg[4], T = op.arg[5], N = op.arg[6], H = op.arg[7];
  int logn;
  if (int rc = stft_shape(S, T, N, H, logn, "stft_bwd")) return rc;
  const int64_t nwin = (T + H - 1) / H;
  const int64_t wpb = stft_windows_per_block(N);
  const int64_t nblk = (nwin + wpb - 1) / wpb;
  DGEN_CHECK_CELL(L, x, S * T, "stft_bwd.x");
  DGEN_CHECK_CELL(L, win, N, "stft_bwd.window");
  DGEN_CHECK_CELL(L, dy, S * T, "stft_bwd.dy");
  DGEN_CHECK_CELL(L, gpart, S * nblk * (N / 2 + 1), "stft_bwd.grad_partials");
  if (L.dry) return 0;
  StftArgs a{};
  a.x = cell(L, x);
  a.win = cell(L, win);
  a.dyin = cell(L, dy);
  a.gpart = cell(L, gpart);
  a.S = (int)S;
  a.T = (int)T;
  a.H = (int)H;
  a.nblk = (int)nblk;
  hipLaunchKernelGGL(bwd_kernel(logn), dim3((unsigned)nblk, (unsigned)S), dim3(kThreads), 0, L.stream, a);
  DGEN_LAUNCH_CHECK("k_stft_bwd");
  return 0;
}

}  // namespace dgen
