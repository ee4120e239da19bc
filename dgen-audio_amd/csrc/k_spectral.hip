// Hop-gated batched spectral loss (spectralLossFFTBatched + BatchedReduce and
// the GradSpec / GradIFFT / GradRead backward chain,
// Sources/DGen/Emit+SpectralLoss.swift:719-1235) for one FFT size per launch.
//
// The reference runs one thread per (frame, batch) with a serial N-point FFT
// in threadgroup scratch and idles on non-hop frames.  Here one workgroup
// owns one (hop window, batch) pair: the window is read once, multiplied by
// the symmetric Hann table and scattered in bit-reversed order into LDS; the
// prediction and target spectra are transformed together (radix-2 stages,
// all butterflies of a stage in parallel); magnitudes, the L1 and log-L1
// terms and the gradient spectrum are formed in place; the unnormalised
// inverse transform and the window multiply produce the window's time
// gradient.  A gather kernel then sums, for every sample, the <= N/H+1
// windows that contain it (atomic-free, fixed order) and forms the
// per-frame loss signal.
#include "internal.h"

namespace dgen {

constexpr float kLogEps = 1e-8f;  // DGenSpectralConfig.logMagnitudeEpsilon (GradientConfig.swift:38)
constexpr float kMagEps = 1e-8f;  // safeMag = max(mag, 1e-8) (Emit+SpectralLoss.swift:1005-1006)
constexpr int kMaxSizes = 8;

__device__ __forceinline__ float sgn(float v) { return v > 0.f ? 1.f : (v < 0.f ? -1.f : 0.f); }

__device__ __forceinline__ void fft_stages(float* re0, float* im0, float* re1, float* im1, const float* twre,
                                           const float* twim, int n, int logn, float dir, bool two) {
  for (int s = 0; s < logn; ++s) {
    const int half = 1 << s;
    for (int idx = threadIdx.x; idx < n / 2; idx += blockDim.x) {
      const int g = idx >> s, k = idx & (half - 1);
      const int i = (g << (s + 1)) + k, j = i + half;
      const float wr = twre[half - 1 + k];
      const float wi = dir * twim[half - 1 + k];
      {
        const float br = re0[j], bi = im0[j];
        const float tr = wr * br - wi * bi, ti = wr * bi + wi * br;
        const float ar = re0[i], ai = im0[i];
        re0[i] = ar + tr;
        im0[i] = ai + ti;
        re0[j] = ar - tr;
        im0[j] = ai - ti;
      }
      if (two) {
        const float br = re1[j], bi = im1[j];
        const float tr = wr * br - wi * bi, ti = wr * bi + wi * br;
        const float ar = re1[i], ai = im1[i];
        re1[i] = ar + tr;
        im1[i] = ai + ti;
        re1[j] = ar - tr;
        im1[j] = ai - ti;
      }
    }
    __syncthreads();
  }
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nw; ++i) s += red[i];
  __syncthreads();
  return s;
}

// tables = hann[N] | twre[N-1] | twim[N-1]
__global__ void k_spectral_loss(const float* __restrict__ x, const float* __restrict__ tgt,
                                const float* __restrict__ tables, float* __restrict__ wloss, float* __restrict__ wgrad,
                                int B, int T, int n, int logn, int hop, float gl, float gg) {
  extern __shared__ float sm[];
  float* re1 = sm;
  float* im1 = re1 + n;
  float* re2 = im1 + n;
  float* im2 = re2 + n;
  float* scale = im2 + n;          // n/2 + 1
  float* red = scale + n / 2 + 1;  // 16
  const float* hann = tables;
  const float* twre = tables + n;
  const float* twim = tables + 2 * n - 1;
  const int w = blockIdx.x, b = blockIdx.y;
  const int f = w * hop;  // the hop frame whose window ends here
  const float* xs = x + (size_t)b * T;
  const float* ts = tgt + (size_t)b * T;

  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int tt = f - (n - 1) + i;
    const bool in = tt >= 0 && tt < T;
    const float hw = hann[i];
    const int p = (int)(__brev((unsigned)i) >> (32 - logn));
    re1[p] = (in ? xs[tt] : 0.f) * hw;
    im1[p] = 0.f;
    re2[p] = (in ? ts[tt] : 0.f) * hw;
    im2[p] = 0.f;
  }
  __syncthreads();
  fft_stages(re1, im1, re2, im2, twre, twim, n, logn, -1.f, true);

  float lin = 0.f, lg = 0.f;
  for (int k = threadIdx.x; k <= n / 2; k += blockDim.x) {
    const float m1 = sqrtf(re1[k] * re1[k] + im1[k] * im1[k]);
    const float m2 = sqrtf(re2[k] * re2[k] + im2[k] * im2[k]);
    const float dlog = logf(m1 + kLogEps) - logf(m2 + kLogEps);
    lin += fabsf(m1 - m2);
    lg += fabsf(dlog);
    const float dmag = gl * sgn(m1 - m2) + gg * sgn(dlog) / (m1 + kLogEps);
    scale[k] = dmag / fmaxf(m1, kMagEps);
  }
  lin = block_sum(lin, red);
  lg = block_sum(lg, red);
  if (threadIdx.x == 0) {
    wloss[((size_t)w * B + b) * 2 + 0] = lin;
    wloss[((size_t)w * B + b) * 2 + 1] = lg;
  }
  // gradient spectrum, bins above N/2 zeroed, scattered bit-reversed
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int p = (int)(__brev((unsigned)i) >> (32 - logn));
    const bool keep = i <= n / 2;
    re2[p] = keep ? scale[i] * re1[i] : 0.f;
    im2[p] = keep ? scale[i] * im1[i] : 0.f;
  }
  __syncthreads();
  fft_stages(re2, im2, nullptr, nullptr, twre, twim, n, logn, 1.f, false);
  float* out = wgrad + ((size_t)w * B + b) * n;
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = re2[i] * hann[i];
}

int launch_spectral_loss(const Launch& L, const dgen_hip_op& op) {
  const int64_t x = op.arg[0], tgt = op.arg[1], wl = op.arg[2], wg = op.arg[3], B = op.arg[4], T = op.arg[5],
                n = op.arg[6], hop = op.arg[7], tab = op.arg[8];
  DGEN_REQUIRE(B > 0 && B <= 65535 && T > 0 && n >= 2 && n <= 8192 && (n & (n - 1)) == 0 && hop >= 1,
               "spectral_loss: B %lld T %lld N %lld hop %lld", (long long)B, (long long)T, (long long)n,
               (long long)hop);
  const int64_t nwin = (T + hop - 1) / hop;
  DGEN_CHECK_CELL(L, x, B * T, "spectral_loss.x");
  DGEN_CHECK_CELL(L, tgt, B * T, "spectral_loss.target");
  DGEN_CHECK_CELL(L, wl, nwin * B * 2, "spectral_loss.window_loss");
  DGEN_CHECK_CELL(L, wg, nwin * B * n, "spectral_loss.window_grad");
  DGEN_CHECK_CELL(L, tab, 3 * n - 2, "spectral_loss.tables");
  if (L.dry) return 0;
  int logn = 0;
  while ((1ll << logn) < n) ++logn;
  const int threads = (int)std::min<int64_t>(256, std::max<int64_t>(64, n / 2));
  const size_t lds = (size_t)(4 * n + n / 2 + 1 + 16) * sizeof(float);
  hipLaunchKernelGGL(k_spectral_loss, dim3((unsigned)nwin, (unsigned)B), dim3(threads), lds, L.stream, cell(L, x),
                     cell(L, tgt), cell(L, tab), cell(L, wl), cell(L, wg), (int)B, (int)T, (int)n, logn, (int)hop,
                     op.farg[0], op.farg[1]);
  DGEN_LAUNCH_CHECK("k_spectral_loss");
  return 0;
}

struct GatherArgs {
  int nsizes;
  int n[kMaxSizes];
  int hop[kMaxSizes];
  const float* wgrad[kMaxSizes];
  const float* wloss[kMaxSizes];
};

__global__ void k_spectral_gather(GatherArgs g, float* __restrict__ dx, float* __restrict__ lossf, int B, int T,
                                  float wl, float wg, float max_frames) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (t >= T) return;
  float acc = 0.f;
  for (int s = 0; s < g.nsizes; ++s) {
    const int n = g.n[s], hop = g.hop[s];
    const int nwin = (T + hop - 1) / hop;
    const int wlo = (t + hop - 1) / hop;
    const int whi = min(nwin - 1, (t + n - 1) / hop);
    for (int w = wlo; w <= whi; ++w) {
      const int off = t - (w * hop - n + 1);
      acc += g.wgrad[s][((size_t)w * B + b) * n + off];
    }
  }
  dx[(size_t)b * T + t] = acc;
  if (b == 0 && lossf) {
    float lf = 0.f;
    for (int s = 0; s < g.nsizes; ++s) {
      const int hop = g.hop[s];
      if (t % hop) continue;
      const int w = t / hop;
      float lin = 0.f, lg = 0.f;
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
  const int64_t dx = op.arg[0], lossf = op.arg[1], B = op.arg[2], T = op.arg[3], ns = op.arg[4];
  const int64_t hop_div = op.arg[29];
  DGEN_REQUIRE(B > 0 && B <= 65535 && T > 0 && ns >= 1 && ns <= kMaxSizes && hop_div >= 1,
               "spectral_gather: B %lld T %lld sizes %lld hop_div %lld", (long long)B, (long long)T, (long long)ns,
               (long long)hop_div);
  DGEN_CHECK_CELL(L, dx, B * T, "spectral_gather.dx");
  if (lossf >= 0) DGEN_CHECK_CELL(L, lossf, T, "spectral_gather.loss_frames");
  GatherArgs g{};
  g.nsizes = (int)ns;
  for (int s = 0; s < ns; ++s) {
    const int64_t n = op.arg[5 + s];
    DGEN_REQUIRE(n >= 2 && (n & (n - 1)) == 0 && n <= 8192, "spectral_gather: size %lld", (long long)n);
    const int64_t hop = std::max<int64_t>(1, n / hop_div);
    const int64_t nwin = (T + hop - 1) / hop;
    DGEN_CHECK_CELL(L, op.arg[13 + s], nwin * B * n, "spectral_gather.window_grad");
    DGEN_CHECK_CELL(L, op.arg[21 + s], nwin * B * 2, "spectral_gather.window_loss");
    if (!L.dry) {
      g.n[s] = (int)n;
      g.hop[s] = (int)hop;
      g.wgrad[s] = cell(L, op.arg[13 + s]);
      g.wloss[s] = cell(L, op.arg[21 + s]);
    }
  }
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_spectral_gather, dim3((unsigned)((T + 255) / 256), (unsigned)B), dim3(256), 0, L.stream, g,
                     cell(L, dx), lossf >= 0 ? cell(L, lossf) : nullptr, (int)B, (int)T, op.farg[0], op.farg[1],
                     op.farg[2]);
  DGEN_LAUNCH_CHECK("k_spectral_gather");
  return 0;
}

}  // namespace dgen
