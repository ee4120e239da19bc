// Hop-gated batched multi-scale spectral loss and its gradient, all FFT
// sizes fused (spectralLossFFTBatched + BatchedReduce and the GradSpec /
// GradIFFT / GradRead chain, Sources/DGen/Emit+SpectralLoss.swift:719-1235;
// HarmonicE2E's fullBatchedLoss, Examples/HarmonicE2E/Trainer.swift:538-583).
//
// Per FFT size N (hop H = N/4) and hop frame f = w*H the reference windows
// x[f-N+1 .. f] (zero outside [0,T)) with the symmetric Hann
// 0.5*(1 - cos(2 pi i/(N-1))), transforms prediction and target, and over the
// bins k = 0..N/2 accumulates |m1 - m2| and |log(m1+eps) - log(m2+eps)|.
// Its gradient spectrum G_k = dmag_k * X_k / max(m1, eps) (bins above N/2
// zero) goes through an unnormalised inverse transform whose real part,
// times the window, is added to dx over the window's samples.
//
// Work decomposition (one workgroup = 256 threads):
// - the workgroup owns an output tile [a, a+4096) of one batch lane and all
//   windows whose hop frame lies in it, for every size;
// - a real N-point transform is an N/2-point complex Stockham FFT of
//   z[n] = s[2n] + i s[2n+1] plus the even/odd split; the real-output
//   inverse is the mirror image (Hermitian pre-processing, N/2-point inverse
//   FFT giving g[2n] + i g[2n+1]);
// - windows processed together are 4 hops (= N samples) apart, so their
//   overlap-add into the tile's LDS accumulator never collides; groups run
//   in a fixed order, so the sums are deterministic and atomic-free;
// - the accumulator spans [a-2047, a+4096); the part left of a belongs to the
//   previous tile and is added by k_mss_combine, which also forms the
//   per-frame loss signal.
// The FFT passes are the shared LDS Stockham transform of fft_lds.h.  For
// N <= 1024 a window's N/16 threads lie in one wave, so its transforms and
// bins are ordered by wave-level syncs and the waves run independently; one
// workgroup barrier per group guards the shared accumulator.
#include "fft_lds.h"

namespace dgen {

constexpr int kTile = kMssTile;    // output samples owned by a workgroup
constexpr int kHalo = kMssHalo;    // largest N - 1
constexpr int kAcc = kMssAcc;
constexpr int kThreads = 256;
constexpr int kMaxSizes = 8;
constexpr float kLogEps = 1e-8f;   // DGenSpectralConfig.logMagnitudeEpsilon (GradientConfig.swift:38)
constexpr float kMagEps = 1e-8f;   // safeMag = max(mag, 1e-8) (Emit+SpectralLoss.swift:1005-1006)
// loss-mode bits (DGEN_HIP_MSS_*): each term's lossMode .l2 (else .l1) and
// useSmoothLogMagnitude for the log term (HigherOps.swift:49-65)
constexpr int kL2Lin = 1, kL2Log = 2, kSmoothLog = 4;

struct MssArgs {
  const float* x;
  const float* tgt;
  float* part;                     // [B][ntiles][kAcc]
  float* wloss[kMaxSizes];         // per size: [nwin][B][2] (lin, log)
  const float* hann[kMaxSizes];    // per size: DGEN_HIP_K_FFT_TABLES output (Hann [N], cos [N-1], sin [N-1])
  int logn[kMaxSizes];
  int nsizes, B, T, ntiles;
  float gl, gg;                    // upstream gradient of each window's lin / log sum
  int mode;                        // kL2Lin | kL2Log | kSmoothLog (the generic kernel only)
};

__device__ __forceinline__ float sgn(float v) { return v > 0.f ? 1.f : (v < 0.f ? -1.f : 0.f); }
// Hardware square root, natural log (via log2) and reciprocal, each within
// ~1 ulp; the loss and its gradient are checked against the fp64 oracle.
__device__ __forceinline__ float hw_sqrt(float v) { return __builtin_amdgcn_sqrtf(v); }
__device__ __forceinline__ float hw_log(float v) { return __builtin_amdgcn_logf(v) * 0.69314718055994531f; }
__device__ __forceinline__ float hw_rcp(float v) { return __builtin_amdgcn_rcpf(v); }

// LDS of the launch (every size runs in it, one after the other).
// The tile accumulator holds dx of samples [a - kHalo, a + kTile) (whole
// 64-sample blocks), stored swizzled: sample i lives at
// i ^ (((i >> 6) & 7) << 3), its 8-float group within its 64-sample block
// flipped by the block index.  A group's windows start N samples apart, and
// in the overlap-add each lane of a window adds a pair of samples, a window's
// lanes covering one aligned run of 2*min(N/16, 32) floats; unswizzled, the
// windows that share a 16- or 32-lane LDS cycle (N <= 256) would all hit the
// same banks, swizzled each falls on its own (32 or 64 banks).  Pairs (even
// sample index) stay together and 8-byte aligned, and the layout needs no
// padding.
__device__ __forceinline__ int accp(int i) { return i ^ (((i >> 6) & 7) << 3); }

struct MssLds {
  static constexpr int kAccN = kAcc + 1;  // 64-sample blocks
  float acc[kAccN];
  c2 buf[2048];                    // FFT slots: (4096/N windows) x (N/2), swizzled
  c2 aux[2048];                    // second signal's spectrum / gradient spectrum
  float red[kThreads / 64][2];
  c2 tw[1024];                     // this size's exp(-2 pi i k / N), k < N/2, correctly rounded
};
static_assert(MssLds::kAccN % 64 == 0, "the accumulator swizzle works on whole 64-sample blocks");

// One FFT size: 4 groups of 4096/N windows, windows in a group 4 hops apart.
// tid: the thread's index, opaque to the optimiser in each call (else every
// size's values that depend only on it would be hoisted out of the size loop
// and held in registers together)
// GEN: the generic bin arithmetic (a.mode's L1/L2 terms and smooth log
// magnitude); otherwise the trainer's L1 magnitude and log(mag + eps) terms
template <int LOGN, bool GEN>
__device__ __forceinline__ void mss_size(const MssArgs& a, MssLds& L, int si, int b, int tile, int tid) {
  constexpr int N = 1 << LOGN, M = N / 2, LOGM = LOGN - 1, H = N / 4, P = M / 8, W = kThreads / P;
  static_assert(W * M == 2048, "window slots must fill the FFT buffer");
  // accumulator index of sample t: t - (a0 - kHalo); for an output pair of a
  // window with hop frame f: f - a0 + kOff + 2 op[e]
  constexpr int kOff = kHalo - (N - 1);
  // a window's P threads (and its FFT slots) lie in one wave when P <= 64:
  // its transforms and bins then need only wave-level ordering; the
  // workgroup barrier is kept for the shared accumulator (windows of
  // consecutive groups overlap) and for the cross-wave loss sums (P > 64)
  constexpr bool WL = P <= 64;
  const int slot = tid / P, j = tid % P;
  const SwzBuf buf(L.buf, slot * M);
  const SwzBuf spec(L.aux, slot * M);
  const int sj = buf.part(j);  // spec.part(j) too
  const int a0 = tile * kTile;
  const int nwin = (a.T + H - 1) / H;
  const float* xs = a.x + (size_t)b * a.T;
  const float* ts = a.tgt + (size_t)b * a.T;
  // The size's table cell holds hann[N] | cos[N-1] | sin[N-1] in the
  // reference's radix-2 layout (stage with half-size h at h-1): the last
  // stage's row is cos, sin(2 pi k / N), k < N/2.  The window values this
  // thread multiplies (samples 2n, 2n+1 of the first pass's inputs n and of
  // the last pass's outputs n) are kept in registers for every group.
  const float* tab = a.hann[si];
  float2 hin[8], hout[8];
  {
    int opl[8];
    pass_positions<M, pass_radix(LOGM, pass_count(LOGM) - 1), pass_span(LOGM, pass_count(LOGM) - 1)>(j, opl);
    // all of the thread's loads in flight before any LDS write (a loop that
    // stored each load as it arrived waited out one memory latency per
    // iteration)
    constexpr int TP = (M + kThreads - 1) / kThreads;
    float cv[TP], sv[TP];
#pragma unroll
    for (int q = 0; q < TP; ++q) {
      const int k = min(tid + q * kThreads, M - 1);
      cv[q] = tab[N + (M - 1) + k];
      sv[q] = tab[2 * N - 1 + (M - 1) + k];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int n = in_pos<M, pass_radix(LOGM, 0)>(j, e);
      hin[e] = float2{tab[2 * n], tab[2 * n + 1]};
      hout[e] = float2{tab[2 * opl[e]], tab[2 * opl[e] + 1]};
    }
#pragma unroll
    for (int q = 0; q < TP; ++q)
      if (tid + q * kThreads < M) L.tw[tid + q * kThreads] = c2{cv[q], -sv[q]};
  }
  lds_barrier();
  const RegTwiddle<LOGM> tw(TableTwiddle{L.tw, M}, j);
  // window samples of group g for this thread: element e of the first pass
  // needs samples s0 + 2n and s0 + 2n + 1, n = in_pos(j, e)
  float pt[16], px[16];
  // (a window inside [0, T) needs no per-sample checks: its loads are one
  // base address plus constant offsets)
  auto fetch = [&](int g) {
    const int w = a0 / H + g + 4 * slot;
    const bool live = w < nwin && w * H < a0 + kTile;
    const int s0 = w * H - N + 1;
    if (live && s0 >= 0 && s0 + N <= a.T) {
      const float* tb = ts + s0 + 2 * j;
      const float* xb = xs + s0 + 2 * j;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        constexpr int R0 = pass_radix(LOGM, 0);
        const int o = 2 * in_off<M, R0>(e);
        pt[2 * e] = tb[o];
        pt[2 * e + 1] = tb[o + 1];
        px[2 * e] = xb[o];
        px[2 * e + 1] = xb[o + 1];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int n = in_pos<M, pass_radix(LOGM, 0)>(j, e);
        const int t0 = s0 + 2 * n, t1 = t0 + 1;
        const bool i0 = live && t0 >= 0 && t0 < a.T, i1 = live && t1 >= 0 && t1 < a.T;
        pt[2 * e] = i0 ? ts[t0] : 0.0f;
        pt[2 * e + 1] = i1 ? ts[t1] : 0.0f;
        px[2 * e] = i0 ? xs[t0] : 0.0f;
        px[2 * e + 1] = i1 ? xs[t1] : 0.0f;
      }
    }
  };
  fetch(0);
#pragma unroll 1
  for (int g = 0; g < 4; ++g) {
    const int w = a0 / H + g + 4 * slot;
    const bool live = w < nwin && w * H < a0 + kTile;
    const int f = w * H;
    const int s0 = f - N + 1;  // first sample of the window
    c2 v[8];
    int op[8];
    // ---- forward transforms of the target (in spec) and the prediction (in
    //      buf), run together
    {
      c2 vt[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float2 h = hin[e];
        vt[e] = c2{pt[2 * e] * h.x, pt[2 * e + 1] * h.y};
        v[e] = c2{px[2 * e] * h.x, px[2 * e + 1] * h.y};
      }
      fft2<LOGM, false, WL>(spec, buf, j, vt, v, op, tw);
      fft_store<LOGM>(spec, j, vt);
      fft_store<LOGM>(buf, j, v);
      lds_sync<WL>();
    }
    if (g + 1 < 4) fetch(g + 1);  // overlaps the bins and the inverse transform
    // ---- bins: pair (k, M-k) for k = 0..M/2 gives every bin 0..N/2; each
    //      thread owns the pairs k = j + i*P (i < NB)
    float lin = 0.f, lg = 0.f;
    auto bin_pair = [&](int k, c2 zx, c2 zxm, c2 zt, c2 ztm) {
        // even/odd split: E = (Z_k + conj Z_{M-k})/2, O = (Z_k - conj Z_{M-k})/(2i)
        const c2 ex = {0.5f * (zx.x + zxm.x), 0.5f * (zx.y - zxm.y)};
        const c2 ox = {0.5f * (zx.y + zxm.y), 0.5f * (zxm.x - zx.x)};
        const c2 et = {0.5f * (zt.x + ztm.x), 0.5f * (zt.y - ztm.y)};
        const c2 ot = {0.5f * (zt.y + ztm.y), 0.5f * (ztm.x - zt.x)};
        const c2 wk = L.tw[k];  // W_N^k (k <= N/4)
        const c2 wox = cmul(wk, ox), wot = cmul(wk, ot);
        // X_k = E + W^k O ; X_{M-k} = conj(E - W^k O)   (k = 0: X_0 and X_M)
        c2 X[2] = {cadd(ex, wox), cconj(csub(ex, wox))};
        c2 Tt[2] = {cadd(et, wot), cconj(csub(et, wot))};
        if (k == 0) {  // X_M = E_0 - O_0 (real parts; imaginary parts vanish)
          X[1] = {ex.x - ox.x, 0.f};
          Tt[1] = {et.x - ot.x, 0.f};
        }
        const int nb = (k == M / 2) ? 1 : 2;  // k = M/2 is its own mirror
        c2 G[2] = {{0.f, 0.f}, {0.f, 0.f}};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          if (q >= nb) break;
          if constexpr (!GEN) {
            const float m1 = hw_sqrt(X[q].x * X[q].x + X[q].y * X[q].y);
            const float m2 = hw_sqrt(Tt[q].x * Tt[q].x + Tt[q].y * Tt[q].y);
            const float dlog = hw_log(m1 + kLogEps) - hw_log(m2 + kLogEps);
            lin += fabsf(m1 - m2);
            lg += fabsf(dlog);
            const float dmag = a.gl * sgn(m1 - m2) + a.gg * sgn(dlog) * hw_rcp(m1 + kLogEps);
            const float sc = dmag * hw_rcp(fmaxf(m1, kMagEps));
            G[q] = {sc * X[q].x, sc * X[q].y};
          } else {
            // Emit+SpectralLoss.swift:150-188 (forward) and :232-291 (GradSpec):
            // the log term's magnitude is sqrt(p + eps^2) when smooth (its
            // difference log m1 - log m2, its gradient over that magnitude
            // twice), else m + eps in the log and max(m, 1e-8) below X
            const bool l2lin = (a.mode & kL2Lin) != 0, l2log = (a.mode & kL2Log) != 0;
            const bool smooth = (a.mode & kSmoothLog) != 0;
            const float p1 = X[q].x * X[q].x + X[q].y * X[q].y;
            const float p2 = Tt[q].x * Tt[q].x + Tt[q].y * Tt[q].y;
            const float m1 = hw_sqrt(p1), m2 = hw_sqrt(p2);
            const float s1 = smooth ? hw_sqrt(p1 + kLogEps * kLogEps) : m1 + kLogEps;
            const float s2 = smooth ? hw_sqrt(p2 + kLogEps * kLogEps) : m2 + kLogEps;
            const float dl = m1 - m2, dg = hw_log(s1) - hw_log(s2);
            lin += l2lin ? dl * dl : fabsf(dl);
            lg += l2log ? dg * dg : fabsf(dg);
            const float sl = l2lin ? 2.f * dl : sgn(dl), sg = l2log ? 2.f * dg : sgn(dg);
            const float rm = hw_rcp(fmaxf(m1, kMagEps)), rs = hw_rcp(s1);
            const float sc = smooth ? a.gl * sl * rm + a.gg * sg * rs * rs : (a.gl * sl + a.gg * sg * rs) * rm;
            G[q] = {sc * X[q].x, sc * X[q].y};
          }
        }
        // inverse pre-processing (Hermitian extension of the one-sided G):
        //   E'_k = (G_k + conj G_{M-k})/2, O'_k = (G_k - conj G_{M-k})/2 * W_N^{-k},
        //   z'_k = E'_k + i O'_k ; bin 0: E' = Re G_0 + Re G_M, O' = Re G_0 - Re G_M
        if (k == 0) {
          const float e0 = G[0].x + G[1].x, o0 = G[0].x - G[1].x;
          spec[0] = {e0, o0};
        } else {
          const c2 gk = G[0], gm = nb == 2 ? G[1] : G[0];
          const c2 winv = cconj(wk);
          const c2 e1 = {0.5f * (gk.x + gm.x), 0.5f * (gk.y - gm.y)};
          const c2 o1 = cmul(c2{0.5f * (gk.x - gm.x), 0.5f * (gk.y + gm.y)}, winv);
          spec[k] = {e1.x - o1.y, e1.y + o1.x};
          if (nb == 2) {
            // index M-k: G_{M-k} = gm, mirror gk, twiddle W_N^{-(M-k)} = -W_N^{k}
            const c2 e2 = {0.5f * (gm.x + gk.x), 0.5f * (gm.y - gk.y)};
            const c2 o2 = cmul(c2{0.5f * (gm.x - gk.x), 0.5f * (gm.y + gk.y)}, c2{-wk.x, -wk.y});
            spec[M - k] = {e2.x - o2.y, e2.y + o2.x};
          }
        }
    };
    constexpr int NB = (M / 2) / P + 1;
    if constexpr (WL) {
      // every spectrum read issued before the first pair is processed (a
      // one-pair loop waited out an LDS round trip per pair)
      c2 zxa[NB], zxb[NB], zta[NB], ztb[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        // k = j + i*P < M for every i (pairs past M/2 are read and skipped)
        const int km = (M - j - i * P) & (M - 1);
        zxa[i] = buf.at(sj, i * P);
        zxb[i] = buf[km];
        zta[i] = spec.at(sj, i * P);
        ztb[i] = spec[km];
      }
#pragma unroll
      for (int i = 0; i < NB; ++i)
        if (j + i * P <= M / 2) bin_pair(j + i * P, zxa[i], zxb[i], zta[i], ztb[i]);
    } else {
      // N = 2048: the hoisted reads would push the kernel past 256 registers
#pragma unroll 1
      for (int k = j; k <= M / 2; k += P) {
        const int km = (M - k) & (M - 1);
        bin_pair(k, buf[k], buf[km], spec[k], spec[km]);
      }
    }
    // ---- per-window loss sums over the window's P threads
#pragma unroll
    for (int off = 1; off < (P < 64 ? P : 64); off <<= 1) {
      lin += __shfl_xor(lin, off, 64);
      lg += __shfl_xor(lg, off, 64);
    }
    if (P > 64) {
      const int wv = tid >> 6;
      if ((tid & 63) == 0) {
        L.red[wv][0] = lin;
        L.red[wv][1] = lg;
      }
    }
    lds_sync<WL>();
    if (j == 0 && live) {
      float sl = lin, sg = lg;
      if (P > 64) {
        const int w0 = (slot * P) >> 6;
        sl = 0.f;
        sg = 0.f;
        for (int q = 0; q < P / 64; ++q) {
          sl += L.red[w0 + q][0];
          sg += L.red[w0 + q][1];
        }
      }
      float* wl = a.wloss[si] + ((size_t)w * a.B + b) * 2;
      wl[0] = sl;
      wl[1] = sg;
    }
    // ---- real-output inverse transform and windowed overlap-add
    fft_load<LOGM>(spec, j, v);
    fft<LOGM, true, WL>(buf, j, v, op, tw);
    // each accumulator element of a group belongs to one thread (the group's
    // windows are disjoint), so all of the thread's reads are issued before
    // its adds and writes.  Output pair e holds samples t, t+1 with
    // t = s0 + 2 op[e]; t - (a0 - (N-1)) = f - a0 + 2 op[e] is even, so the
    // pair is one 8-byte LDS access.  Pairs outside the tile's range read a
    // clamped element and are not written; a pair with one sample outside
    // [0, T) writes only the other.
    if (live && s0 >= 0 && s0 + N <= a.T) {
      // the whole window inside [0, T): every pair is written
      float2 ac[8];
      int ai[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ai[e] = accp(f - a0 + kOff + 2 * op[e]);
        ac[e] = *reinterpret_cast<const float2*>(&L.acc[ai[e]]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float2 h = hout[e];
        *reinterpret_cast<float2*>(&L.acc[ai[e]]) = float2{ac[e].x + v[e].x * h.x, ac[e].y + v[e].y * h.y};
      }
    } else {
      constexpr int kAccN = MssLds::kAccN;
      float2 ac[8];
      int ai[8];
      bool a0w[8], a1w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = s0 + 2 * op[e];
        a0w[e] = live && t >= 0 && t < a.T;
        a1w[e] = live && t + 1 >= 0 && t + 1 < a.T;
        ai[e] = accp(min(max(t - (a0 - kHalo), 0), kAccN - 2));
        ac[e] = *reinterpret_cast<const float2*>(&L.acc[ai[e]]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float2 h = hout[e];
        const float2 r = {ac[e].x + v[e].x * h.x, ac[e].y + v[e].y * h.y};
        if (a0w[e] && a1w[e]) *reinterpret_cast<float2*>(&L.acc[ai[e]]) = r;
        else if (a0w[e]) L.acc[ai[e]] = r.x;
        else if (a1w[e]) L.acc[ai[e] + 1] = r.y;
      }
    }
    // every wave's overlap-add of group g lands before any of group g + 1
    lds_barrier();
  }
}

// All sizes in one launch, in the op's size order: the tile accumulator
// stays in LDS from the first size to the last and is written to the tile
// partials once.
template <bool GEN>
__global__ __launch_bounds__(kThreads) void k_mss(MssArgs a) {
  extern __shared__ float4 smem4[];
  MssLds& L = *reinterpret_cast<MssLds*>(smem4);
  const int tile = blockIdx.x, b = blockIdx.y;
  for (int i = threadIdx.x; i < MssLds::kAccN; i += kThreads) L.acc[i] = 0.f;
  lds_barrier();
  for (int s = 0; s < a.nsizes; ++s) {
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    switch (a.logn[s]) {
      case 6: mss_size<6, GEN>(a, L, s, b, tile, tid); break;
      case 7: mss_size<7, GEN>(a, L, s, b, tile, tid); break;
      case 8: mss_size<8, GEN>(a, L, s, b, tile, tid); break;
      case 9: mss_size<9, GEN>(a, L, s, b, tile, tid); break;
      case 10: mss_size<10, GEN>(a, L, s, b, tile, tid); break;
      default: mss_size<11, GEN>(a, L, s, b, tile, tid); break;
    }
  }
  float* part = a.part + ((size_t)b * a.ntiles + tile) * kAcc;
  for (int i = threadIdx.x; i < kAcc; i += kThreads) part[i] = L.acc[accp(i)];
}

int launch_spectral_loss(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=x ([B][T]) [1]=target ([B][T]) [2]=tile partials ([B][ntiles][6143]) [3]=B [4]=T [5]=n_sizes
  //      [6..13]=N_s [14..21]=per-window loss cells ([nwin_s][B][2]) [22..29]=FFT tables ([3 N_s - 2])
  //      [30]=loss mode (kL2Lin | kL2Log | kSmoothLog; 0: L1 terms, log(mag + eps))
  // farg: [0]=lin upstream grad per window [1]=log upstream grad per window
  const int64_t x = op.arg[0], tgt = op.arg[1], part = op.arg[2], B = op.arg[3], T = op.arg[4], ns = op.arg[5];
  const int64_t mode = op.arg[30];
  DGEN_REQUIRE(mode >= 0 && mode <= (kL2Lin | kL2Log | kSmoothLog), "spectral_loss: loss mode %lld", (long long)mode);
  DGEN_REQUIRE(B > 0 && B <= 65535 && T > 0 && T <= (1 << 26) && ns >= 1 && ns <= kMaxSizes,
               "spectral_loss: B %lld T %lld sizes %lld", (long long)B, (long long)T, (long long)ns);
  const int64_t ntiles = (T + kTile - 1) / kTile;
  DGEN_CHECK_CELL(L, x, B * T, "spectral_loss.x");
  DGEN_CHECK_CELL(L, tgt, B * T, "spectral_loss.target");
  DGEN_CHECK_CELL(L, part, B * ntiles * kAcc, "spectral_loss.tile_partials");
  MssArgs a{};
  for (int s = 0; s < ns; ++s) {
    const int64_t n = op.arg[6 + s];
    int lg = 0;
    while ((1ll << lg) < n) ++lg;
    DGEN_REQUIRE((1ll << lg) == n && lg >= 6 && lg <= 11, "spectral_loss: size %lld not a power of two in [64, 2048]",
                 (long long)n);
    const int64_t nwin = (T + n / 4 - 1) / (n / 4);
    DGEN_CHECK_CELL(L, op.arg[14 + s], nwin * B * 2, "spectral_loss.window_loss");
    DGEN_CHECK_CELL(L, op.arg[22 + s], 3 * n - 2, "spectral_loss.fft_tables");
    a.logn[s] = lg;
    if (!L.dry) {
      a.wloss[s] = cell(L, op.arg[14 + s]);
      a.hann[s] = cell(L, op.arg[22 + s]);
    }
  }
  if (L.dry) return 0;
  a.x = cell(L, x);
  a.tgt = cell(L, tgt);
  a.part = cell(L, part);
  a.nsizes = (int)ns;
  a.B = (int)B;
  a.T = (int)T;
  a.ntiles = (int)ntiles;
  a.gl = op.farg[0];
  a.gg = op.farg[1];
  a.mode = (int)mode;
  const dim3 grid((unsigned)ntiles, (unsigned)B);
  if (mode)
    hipLaunchKernelGGL(k_mss<true>, grid, dim3(kThreads), sizeof(MssLds), L.stream, a);
  else
    hipLaunchKernelGGL(k_mss<false>, grid, dim3(kThreads), sizeof(MssLds), L.stream, a);
  DGEN_LAUNCH_CHECK("k_mss");
  return 0;
}

// dx[b][t] = the owning tile's accumulator + the next tile's halo part, and
// the per-frame loss signal (Emit+SpectralLoss.swift:914-938 batch mean,
// Functions.swift:945-955 normalize by maxFrameCount).
struct CombineArgs {
  int nsizes;
  int hop[kMaxSizes];
  const float* wloss[kMaxSizes];
};

// With w_mse != 0 the trainer's time-domain term joins in
// (Trainer.swift:547-551): w * sum_b (x - tgt)^2 / B per frame, first in the
// frame's loss, and its gradient 2 w (x - tgt) / B added to dx.
__global__ void k_mss_combine(CombineArgs g, const float* __restrict__ part, float* __restrict__ dx,
                              float* __restrict__ lossf, int B, int T, int ntiles, float wl, float wg,
                              float max_frames, const float* __restrict__ xs, const float* __restrict__ ts,
                              float w_mse) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (t >= T) return;
  const float inv_b = 1.0f / (float)B;
  if (dx) {
    const int tile = t / kTile, a0 = tile * kTile;
    const float* p = part + ((size_t)b * ntiles + tile) * kAcc;
    float v = p[t - a0 + kHalo];
    const int a1 = a0 + kTile;
    if (tile + 1 < ntiles && t >= a1 - kHalo) v += p[kAcc + (t - a1 + kHalo)];
    if (w_mse != 0.f) {
      const size_t i = (size_t)b * T + t;
      v += w_mse * (2.f * (xs[i] - ts[i])) * inv_b;
    }
    dx[(size_t)b * T + t] = v;
  }
  if (b == 0 && lossf) {
    float lf = 0.f;
    if (w_mse != 0.f) {
      float s = 0.f;
      for (int bb = 0; bb < B; ++bb) {
        const float d = xs[(size_t)bb * T + t] - ts[(size_t)bb * T + t];
        s = s + d * d;
      }
      lf = s * inv_b * w_mse;
    }
    for (int s = 0; s < g.nsizes; ++s) {
      const int hop = g.hop[s];
      if (t % hop) continue;
      const int w = t / hop;
      float lin = 0.f, lg = 0.f;
      // loads of 8 lanes in flight at a time; the adds keep lane order
#pragma unroll 8
      for (int bb = 0; bb < B; ++bb) {
        lin = lin + g.wloss[s][((size_t)w * B + bb) * 2 + 0];
        lg = lg + g.wloss[s][((size_t)w * B + bb) * 2 + 1];
      }
      lin = lin / (float)B / max_frames;
      lg = lg / (float)B / max_frames;
      lf = lf + lin * wl + lg * wg;
    }
    lossf[t] = lf;
  }
}

int launch_spectral_gather(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=dx ([B][T]) or -1 [1]=loss frames ([T]) or -1 [2]=B [3]=T [4]=n_sizes [5..12]=N_s
  //      [13]=tile partials [21..28]=per-window loss cells
  //      with farg[3] != 0: [29]=x ([B][T]) [30]=target ([B][T])
  // farg: [0]=lin weight per size [1]=log weight per size [2]=maxFrameCount
  //       [3]=weight of the time-domain MSE term (0: none)
  const int64_t dx = op.arg[0], lossf = op.arg[1], B = op.arg[2], T = op.arg[3], ns = op.arg[4];
  DGEN_REQUIRE(dx >= 0 || lossf >= 0, "spectral_gather: neither dx nor loss frames requested");
  const float w_mse = op.farg[3];
  if (w_mse != 0.f) {
    DGEN_CHECK_CELL(L, op.arg[29], B * T, "spectral_gather.x");
    DGEN_CHECK_CELL(L, op.arg[30], B * T, "spectral_gather.target");
  }
  const int64_t part = op.arg[13];
  DGEN_REQUIRE(B > 0 && B <= 65535 && T > 0 && T <= (1 << 26) && ns >= 1 && ns <= kMaxSizes,
               "spectral_gather: B %lld T %lld sizes %lld", (long long)B, (long long)T, (long long)ns);
  const int64_t ntiles = (T + kTile - 1) / kTile;
  if (dx >= 0) DGEN_CHECK_CELL(L, dx, B * T, "spectral_gather.dx");
  if (lossf >= 0) DGEN_CHECK_CELL(L, lossf, T, "spectral_gather.loss_frames");
  DGEN_CHECK_CELL(L, part, B * ntiles * kAcc, "spectral_gather.tile_partials");
  CombineArgs g{};
  g.nsizes = (int)ns;
  for (int s = 0; s < ns; ++s) {
    const int64_t n = op.arg[5 + s];
    DGEN_REQUIRE(n >= 64 && n <= 2048 && (n & (n - 1)) == 0, "spectral_gather: size %lld", (long long)n);
    const int64_t hop = n / 4;
    const int64_t nwin = (T + hop - 1) / hop;
    DGEN_CHECK_CELL(L, op.arg[21 + s], nwin * B * 2, "spectral_gather.window_loss");
    if (!L.dry) {
      g.hop[s] = (int)hop;
      g.wloss[s] = cell(L, op.arg[21 + s]);
    }
  }
  if (L.dry) return 0;
  // without dx only the lane-0 row of blocks (the loss signal) is launched
  hipLaunchKernelGGL(k_mss_combine, dim3((unsigned)((T + 255) / 256), (unsigned)(dx >= 0 ? B : 1)), dim3(256), 0,
                     L.stream, g, cell(L, part), dx >= 0 ? cell(L, dx) : nullptr, lossf >= 0 ? cell(L, lossf) : nullptr,
                     (int)B, (int)T, (int)ntiles, op.farg[0], op.farg[1], op.farg[2],
                     w_mse != 0.f ? cell(L, op.arg[29]) : nullptr, w_mse != 0.f ? cell(L, op.arg[30]) : nullptr, w_mse);
  DGEN_LAUNCH_CHECK("k_mss_combine");
  return 0;
}

}  // namespace dgen
