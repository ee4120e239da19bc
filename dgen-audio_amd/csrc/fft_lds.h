// LDS Stockham FFT shared by the spectral-loss and STFT kernels.
//
// A complex M-point transform (M = 2^LOGM, 8 <= M <= 1024) is done by M/8
// threads, each holding 8 values in registers between passes; the passes
// follow the Stockham autosort formulation of Govindaraju et al., "High
// Performance Discrete Fourier Transforms on Graphics Processors" (SC 2008):
// pass with radix R and span Ns reads v_r = in[j + r*M/R], twiddles by
// exp(-+2 pi i r (j mod Ns)/(Ns R)), does an R-point DFT and writes
// out[(j/Ns)*Ns*R + j mod Ns + r*Ns].  Radix 8 passes first, then one 4 or 2.
// Every thread of the workgroup must call fft() together (it contains
// workgroup barriers); each group of M/8 threads works on its own buffer.
// With WAVE, the M/8 threads of every buffer lie in one wave and the passes
// are ordered by wave_sync() instead of workgroup barriers (each wave then
// runs its transforms without waiting for the others).
//
// Buffers are padded: complex value i lives at i + i/8.  A Stockham pass
// writes R consecutive values per thread, a stride of 8R bytes across the
// wave, which on the 32-bank LDS would put most lanes of a store on the same
// bank pair; the pad spreads them over 16 pairs and keeps the passes' reads
// (consecutive indices) contiguous.
#pragma once

#include "internal.h"

namespace dgen {

struct c2 {
  float x, y;
};

// Storage (in complex values) for n padded values, n a multiple of 8.
__host__ __device__ constexpr int lds_pad(int n) { return n + n / 8; }

// View of one padded FFT buffer.
struct PadBuf {
  c2* p;
  __device__ __forceinline__ c2& operator[](int i) const { return p[i + (i >> 3)]; }
};
__device__ __forceinline__ c2 cadd(c2 a, c2 b) { return {a.x + b.x, a.y + b.y}; }
__device__ __forceinline__ c2 csub(c2 a, c2 b) { return {a.x - b.x, a.y - b.y}; }
__device__ __forceinline__ c2 cmul(c2 a, c2 b) { return {fmaf(a.x, b.x, -a.y * b.y), fmaf(a.x, b.y, a.y * b.x)}; }
__device__ __forceinline__ c2 cconj(c2 a) { return {a.x, -a.y}; }
// multiply by -i (forward) or +i (inverse)
template <bool INV>
__device__ __forceinline__ c2 mul_mi(c2 a) { return INV ? c2{-a.y, a.x} : c2{a.y, -a.x}; }
// exp(sgn * 2 pi i * rev), rev in revolutions (v_cos/v_sin take revolutions)
__device__ __forceinline__ c2 cis(float rev) { return {__builtin_amdgcn_cosf(rev), __builtin_amdgcn_sinf(rev)}; }

// Twiddle sources of the passes.  A pass of radix R and span NS multiplies
// input r of butterfly k by W^(r k) with W = exp(-+2 pi i / (NS R)).
// - HwTwiddle: W^1 from the hardware sin/cos (about 2 ulp), higher powers by
//   complex products (up to six for radix 8);
// - TableTwiddle: every power read from a table of correctly rounded values
//   t[i] = exp(-2 pi i i / N), i < N/2 = M (the last radix-2 stage's row of
//   the reference's Float twiddle table, HigherOps.swift:84-91), as
//   W_M^e = W_N^(2e) = +-t[2e mod M].  The products' rounding compounds in
//   windows whose spectrum spans many decades (the spectral loss's
//   log-magnitude gradient amplifies it), so the spectral loss uses tables.
struct HwTwiddle {
  static constexpr bool kTable = false;
  __device__ __forceinline__ c2 get(int) const { return {1.f, 0.f}; }
};
struct TableTwiddle {
  static constexpr bool kTable = true;
  const c2* t;  // M values, in LDS
  int m;
  // W_M^e for 0 <= e < M (forward sign)
  __device__ __forceinline__ c2 get(int e) const {
    const int i = 2 * e;
    const bool hi = i >= m;
    const c2 w = t[hi ? i - m : i];
    return hi ? c2{-w.x, -w.y} : w;
  }
};

template <bool INV>
__device__ __forceinline__ void dft2(c2* v) {
  const c2 a = v[0], b = v[1];
  v[0] = cadd(a, b);
  v[1] = csub(a, b);
}

template <bool INV>
__device__ __forceinline__ void dft4(c2* v) {
  const c2 s02 = cadd(v[0], v[2]), d02 = csub(v[0], v[2]);
  const c2 s13 = cadd(v[1], v[3]), d13 = mul_mi<INV>(csub(v[1], v[3]));
  v[0] = cadd(s02, s13);
  v[2] = csub(s02, s13);
  v[1] = cadd(d02, d13);
  v[3] = csub(d02, d13);
}

template <bool INV>
__device__ __forceinline__ void dft8(c2* v) {
  c2 e[4] = {v[0], v[2], v[4], v[6]};
  c2 o[4] = {v[1], v[3], v[5], v[7]};
  dft4<INV>(e);
  dft4<INV>(o);
  constexpr float h = 0.70710678118654752f;
  // o_k *= w8^k, w8 = exp(-+2 pi i / 8)
  o[1] = INV ? c2{h * (o[1].x - o[1].y), h * (o[1].x + o[1].y)} : c2{h * (o[1].x + o[1].y), h * (o[1].y - o[1].x)};
  o[2] = mul_mi<INV>(o[2]);
  o[3] = INV ? c2{-h * (o[3].x + o[3].y), h * (o[3].x - o[3].y)} : c2{h * (o[3].y - o[3].x), -h * (o[3].x + o[3].y)};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = cadd(e[k], o[k]);
    v[k + 4] = csub(e[k], o[k]);
  }
}

template <int R, bool INV>
__device__ __forceinline__ void dftR(c2* v) {
  if (R == 8) dft8<INV>(v);
  else if (R == 4) dft4<INV>(v);
  else dft2<INV>(v);
}

// Radix of pass p for an M-point transform: 8s first, then one 4 or 2.
__host__ __device__ constexpr int pass_radix(int logm, int p) {
  return (logm - 3 * p) >= 3 ? 8 : (logm - 3 * p == 2 ? 4 : 2);
}
__host__ __device__ constexpr int pass_count(int logm) { return (logm + 2) / 3; }
__host__ __device__ constexpr int pass_span(int logm, int p) {
  return p == 0 ? 1 : pass_span(logm, p - 1) * pass_radix(logm, p - 1);
}

// One Stockham pass over this thread's 8 values v (already read): twiddle,
// R-point DFTs, and the output positions.  j = thread index within the
// window; butterfly u of the thread is bj = j + u*M/8.
// The twiddles of input r (1 <= r < R) of butterfly k: w[r] *= W^(r k).
template <int M, int R, int NS, bool INV, class TW>
__device__ __forceinline__ void twiddle(c2* w, int k, const TW& tw) {
  if constexpr (TW::kTable) {
    constexpr int S = M / (NS * R);  // W = W_M^S; r k S < M
#pragma unroll
    for (int r = 1; r < R; ++r) {
      const c2 t = tw.get(r * k * S);
      w[r] = cmul(w[r], INV ? cconj(t) : t);
    }
  } else {
    const float rev = (INV ? 1.0f : -1.0f) * (float)k / (float)(NS * R);
    const c2 t1 = cis(rev);
    c2 t = t1;
#pragma unroll
    for (int r = 1; r < R; ++r) {
      w[r] = cmul(w[r], t);
      if (r + 1 < R) t = cmul(t, t1);
    }
  }
}

template <int M, int R, int NS, bool INV, class TW = HwTwiddle>
__device__ __forceinline__ void pass_compute(c2* v, int j, int* outpos, const TW& tw = TW{}) {
  constexpr int BPT = 8 / R;
#pragma unroll
  for (int u = 0; u < BPT; ++u) {
    const int bj = j + u * (M / 8);
    const int k = bj % NS;
    c2* w = v + u * R;
    if (NS > 1) twiddle<M, R, NS, INV>(w, k, tw);
    dftR<R, INV>(w);
    const int base = (bj / NS) * NS * R + k;
#pragma unroll
    for (int r = 0; r < R; ++r) outpos[u * R + r] = base + r * NS;
  }
}

// Input positions of pass with radix R: element u*R + r <- bj + r*M/R.
template <int M, int R>
__device__ __forceinline__ int in_pos(int j, int e) {
  const int u = e / R, r = e % R;
  return j + u * (M / 8) + r * (M / R);
}

// Middle passes 1 .. npass-2 in LDS (in place; a barrier separates each
// pass's reads from its writes).
template <int LOGM, int P, bool INV, bool WAVE = false, class TW = HwTwiddle>
__device__ __forceinline__ void mid_passes(PadBuf buf, int j, c2* v, const TW& tw = TW{}) {
  constexpr int M = 1 << LOGM;
  if constexpr (P < pass_count(LOGM) - 1) {
    constexpr int R = pass_radix(LOGM, P), NS = pass_span(LOGM, P);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = buf[in_pos<M, R>(j, e)];
    lds_sync<WAVE>();
    int op[8];
    pass_compute<M, R, NS, INV>(v, j, op, tw);
#pragma unroll
    for (int e = 0; e < 8; ++e) buf[op[e]] = v[e];
    lds_sync<WAVE>();
    mid_passes<LOGM, P + 1, INV, WAVE>(buf, j, v, tw);
  }
}

// Full M-point FFT: v holds the first pass's inputs (v[e] = input at
// in_pos of pass 0); on return v holds the last pass's outputs at positions
// op[e].  Uses buf (M complex, this window's slot) between passes.
template <int LOGM, bool INV, bool WAVE = false, class TW = HwTwiddle>
__device__ __forceinline__ void fft(PadBuf buf, int j, c2* v, int* op, const TW& tw = TW{}) {
  constexpr int M = 1 << LOGM;
  constexpr int NP = pass_count(LOGM);
  {
    constexpr int R = pass_radix(LOGM, 0);
    pass_compute<M, R, 1, INV>(v, j, op, tw);
  }
  if constexpr (NP > 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e) buf[op[e]] = v[e];
    lds_sync<WAVE>();
    mid_passes<LOGM, 1, INV, WAVE>(buf, j, v, tw);
    constexpr int RL = pass_radix(LOGM, NP - 1), NSL = pass_span(LOGM, NP - 1);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = buf[in_pos<M, RL>(j, e)];
    lds_sync<WAVE>();
    pass_compute<M, RL, NSL, INV>(v, j, op, tw);
  }
}

// Two M-point transforms of the same direction in one pass sequence (a and
// b in buffers bufa and bufb): each pass's twiddles, positions and LDS round
// trip serve both, and the two butterflies give the scheduler independent
// work.  Each signal's arithmetic is exactly that of fft().
template <int M, int R, int NS, bool INV, class TW = HwTwiddle>
__device__ __forceinline__ void pass_compute2(c2* va, c2* vb, int j, int* outpos, const TW& tw = TW{}) {
  constexpr int BPT = 8 / R;
#pragma unroll
  for (int u = 0; u < BPT; ++u) {
    const int bj = j + u * (M / 8);
    const int k = bj % NS;
    c2* wa = va + u * R;
    c2* wb = vb + u * R;
    if (NS > 1) {
      if constexpr (TW::kTable) {
        constexpr int S = M / (NS * R);
#pragma unroll
        for (int r = 1; r < R; ++r) {
          const c2 t0 = tw.get(r * k * S);
          const c2 t = INV ? cconj(t0) : t0;
          wa[r] = cmul(wa[r], t);
          wb[r] = cmul(wb[r], t);
        }
      } else {
        const float rev = (INV ? 1.0f : -1.0f) * (float)k / (float)(NS * R);
        const c2 t1 = cis(rev);
        c2 t = t1;
#pragma unroll
        for (int r = 1; r < R; ++r) {
          wa[r] = cmul(wa[r], t);
          wb[r] = cmul(wb[r], t);
          if (r + 1 < R) t = cmul(t, t1);
        }
      }
    }
    dftR<R, INV>(wa);
    dftR<R, INV>(wb);
    const int base = (bj / NS) * NS * R + k;
#pragma unroll
    for (int r = 0; r < R; ++r) outpos[u * R + r] = base + r * NS;
  }
}

template <int LOGM, int P, bool INV, bool WAVE, class TW = HwTwiddle>
__device__ __forceinline__ void mid_passes2(PadBuf bufa, PadBuf bufb, int j, c2* va, c2* vb, const TW& tw = TW{}) {
  constexpr int M = 1 << LOGM;
  if constexpr (P < pass_count(LOGM) - 1) {
    constexpr int R = pass_radix(LOGM, P), NS = pass_span(LOGM, P);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      va[e] = bufa[in_pos<M, R>(j, e)];
      vb[e] = bufb[in_pos<M, R>(j, e)];
    }
    lds_sync<WAVE>();
    int op[8];
    pass_compute2<M, R, NS, INV>(va, vb, j, op, tw);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bufa[op[e]] = va[e];
      bufb[op[e]] = vb[e];
    }
    lds_sync<WAVE>();
    mid_passes2<LOGM, P + 1, INV, WAVE>(bufa, bufb, j, va, vb, tw);
  }
}

// fft() of two signals at once: on return va / vb hold their last pass's
// outputs at positions op[e].
template <int LOGM, bool INV, bool WAVE = false, class TW = HwTwiddle>
__device__ __forceinline__ void fft2(PadBuf bufa, PadBuf bufb, int j, c2* va, c2* vb, int* op, const TW& tw = TW{}) {
  constexpr int M = 1 << LOGM;
  constexpr int NP = pass_count(LOGM);
  {
    constexpr int R = pass_radix(LOGM, 0);
    pass_compute2<M, R, 1, INV>(va, vb, j, op, tw);
  }
  if constexpr (NP > 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bufa[op[e]] = va[e];
      bufb[op[e]] = vb[e];
    }
    lds_sync<WAVE>();
    mid_passes2<LOGM, 1, INV, WAVE>(bufa, bufb, j, va, vb, tw);
    constexpr int RL = pass_radix(LOGM, NP - 1), NSL = pass_span(LOGM, NP - 1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      va[e] = bufa[in_pos<M, RL>(j, e)];
      vb[e] = bufb[in_pos<M, RL>(j, e)];
    }
    lds_sync<WAVE>();
    pass_compute2<M, RL, NSL, INV>(va, vb, j, op, tw);
  }
}

}  // namespace dgen
