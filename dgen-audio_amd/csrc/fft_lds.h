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
// Buffer layout: the W slots of M values share one buffer of W*M = 2048
// complex values, and value i of slot q lives at swz(q*M + i), where
// swz(I) = I ^ h(I >> 4) and h is linear over GF(2) (bit 4 of I flips bit 0,
// bit 5 flips bit 2, bit 6 flips bits 1 and 3, bit 7 flips bit 4).  Across
// the lanes of a wave a pass reads consecutive indices and writes runs of NS
// consecutive indices NS*R apart (stride R when NS = 1); through swz every
// one of these accesses puts each group of 16 lanes on 16 distinct 8-byte
// bank pairs (a 32-bank LDS) and each group of 32 lanes on 32 (64 banks),
// for every slot count.  swz is a bijection on every aligned block of 256
// values and is linear, so for an index a + c whose parts have no common
// bits, swz(a + c) = swz(a) ^ swz(c): a thread computes swz of its own part
// once and each access adds one XOR with a compile-time constant.
#pragma once

#include "internal.h"

namespace dgen {

// 8-byte aligned so that every access is one ds_read_b64 / ds_write_b64 (at
// 4-byte alignment each splits into two 4-byte halves, each half strided 8
// bytes across the lanes: two LDS passes, each 2-way bank conflicted)
struct alignas(8) c2 {
  float x, y;
};

// The buffer swizzle (see the header comment).
__host__ __device__ constexpr int swz(int i) {
  return i ^ ((i >> 4) & 1) ^ ((i >> 3) & 4) ^ ((i >> 5) & 2) ^ ((i >> 3) & 8) ^ ((i >> 3) & 16);
}

// View of one slot of the swizzled buffer.
// A slot's values occupy the positions [slot*M, slot*M + M) in some order
// (M >= 32: swz changes bits 0-4 only).
struct SwzBuf {
  c2* p;      // the workgroup's buffer (all slots)
  int start;  // slot * M
  int base;   // swz(slot * M)
  __device__ __forceinline__ SwzBuf(c2* buffer, int slot_start)
      : p(buffer), start(slot_start), base(swz(slot_start)) {}
  // value i (0 <= i < M) of the slot
  __device__ __forceinline__ c2& operator[](int i) const { return p[base ^ swz(i)]; }
  // the swizzled position of this thread's part t of an index ...
  // (opaque to the optimiser: each access then costs one XOR where it is
  // made, instead of every address of every pass being hoisted out of the
  // callers' loops into a register of its own)
  __device__ __forceinline__ int part(int t) const {
    int v = base ^ swz(t);
    asm volatile("" : "+v"(v));
    return v;
  }
  // ... and the value at index t + c, c a constant with no bits in common with t
  __device__ __forceinline__ c2& at(int st, int c) const { return p[st ^ swz(c)]; }
  // the slot's region as raw floats (2*M of them)
  __device__ __forceinline__ float* raw() const { return reinterpret_cast<float*>(p + start); }
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
//   log-magnitude gradient amplifies it), so the spectral loss uses tables;
// - RegTwiddle (below): the same table values for one thread's butterflies,
//   read once into registers.
struct HwTwiddle {
  static constexpr bool kTable = false;
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
  // forward-sign twiddle of input r of butterfly u (index k within its span)
  template <int M, int R, int NS>
  __device__ __forceinline__ c2 pass_tw(int, int r, int k) const {
    return get(r * k * (M / (NS * R)));
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
__host__ __device__ constexpr int ilog2c(int n) { return n <= 1 ? 0 : 1 + ilog2c(n / 2); }

// The table twiddles of one thread's butterflies, in registers.  They depend
// only on the thread's index j within its slot, so every transform of a
// kernel uses the same ones; the values are TableTwiddle's.  Butterflies u of
// a pass share their index k (and twiddles) when NS divides M/8.
template <int LOGM>
struct RegTwiddle {
  static constexpr bool kTable = true;
  static constexpr int M = 1 << LOGM, NP = pass_count(LOGM);
  template <int R, int NS>
  static constexpr int nu() { return (M / 8) % NS == 0 ? 1 : 8 / R; }
  c2 w[NP][4][7];  // [pass][u][r - 1]; pass 0 has no twiddles
  template <int P>
  __device__ __forceinline__ void fill(const TableTwiddle& t, int j) {
    if constexpr (P < NP) {
      constexpr int R = pass_radix(LOGM, P), NS = pass_span(LOGM, P);
#pragma unroll
      for (int u = 0; u < nu<R, NS>(); ++u) {
        const int k = (j + u * (M / 8)) % NS;
#pragma unroll
        for (int r = 1; r < R; ++r) w[P][u][r - 1] = t.pass_tw<M, R, NS>(u, r, k);
      }
      fill<P + 1>(t, j);
    }
  }
  __device__ __forceinline__ RegTwiddle(const TableTwiddle& t, int j) { fill<1>(t, j); }
  template <int MM, int R, int NS>
  __device__ __forceinline__ c2 pass_tw(int u, int r, int) const {
    static_assert(MM == M, "twiddles of another transform size");
    return w[ilog2c(NS) / 3][nu<R, NS>() == 1 ? 0 : u][r - 1];
  }
};

// Pass positions.  Input element u*R + r of a thread is index bj + r*M/R
// (bj = j + u*M/8): the thread part j plus a constant; output element
// u*R + r goes to (bj/NS)*NS*R + bj%NS + r*NS: a per-butterfly part plus the
// constant r*NS.  In both the two parts have no common bits.
template <int M, int R>
__host__ __device__ constexpr int in_off(int e) {
  return (e / R) * (M / 8) + (e % R) * (M / R);
}
template <int M, int R>
__device__ __forceinline__ int in_pos(int j, int e) {
  return j + in_off<M, R>(e);
}
template <int M, int R, int NS>
__device__ __forceinline__ int out_base(int j, int u) {
  const int bj = j + u * (M / 8);
  return (bj / NS) * NS * R + bj % NS;
}
template <int M, int R, int NS>
__device__ __forceinline__ void pass_positions(int j, int* op) {
#pragma unroll
  for (int u = 0; u < 8 / R; ++u) {
    const int b = out_base<M, R, NS>(j, u);
#pragma unroll
    for (int r = 0; r < R; ++r) op[u * R + r] = b + r * NS;
  }
}
// A pass's inputs from buf (sj = buf.part(j)) and its outputs into buf.
template <int M, int R>
__device__ __forceinline__ void pass_load(const SwzBuf& buf, int sj, c2* v) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = buf.at(sj, in_off<M, R>(e));
}
template <int M, int R, int NS>
__device__ __forceinline__ void pass_store(const SwzBuf& buf, int j, const c2* v) {
#pragma unroll
  for (int u = 0; u < 8 / R; ++u) {
    const int sb = buf.part(out_base<M, R, NS>(j, u));
#pragma unroll
    for (int r = 0; r < R; ++r) buf.at(sb, r * NS) = v[u * R + r];
  }
}

// One Stockham pass over this thread's 8 values v (already read): twiddle
// and R-point DFTs.  j = thread index within the window; butterfly u of the
// thread is bj = j + u*M/8.  The twiddles of input r (1 <= r < R) of
// butterfly k: w[r] *= W^(r k).
template <int M, int R, int NS, bool INV, class TW>
__device__ __forceinline__ void twiddle(c2* w, int u, int k, const TW& tw) {
  if constexpr (TW::kTable) {
#pragma unroll
    for (int r = 1; r < R; ++r) {
      const c2 t = tw.template pass_tw<M, R, NS>(u, r, k);
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
    const int k = (j + u * (M / 8)) % NS;
    c2* w = v + u * R;
    if (NS > 1) twiddle<M, R, NS, INV>(w, u, k, tw);
    dftR<R, INV>(w);
  }
  pass_positions<M, R, NS>(j, outpos);
}

// Middle passes 1 .. npass-2 in LDS (in place; a sync separates each pass's
// reads from its writes).
template <int LOGM, int P, bool INV, bool WAVE = false, class TW = HwTwiddle>
__device__ __forceinline__ void mid_passes(const SwzBuf& buf, int j, int sj, c2* v, const TW& tw = TW{}) {
  constexpr int M = 1 << LOGM;
  if constexpr (P < pass_count(LOGM) - 1) {
    constexpr int R = pass_radix(LOGM, P), NS = pass_span(LOGM, P);
    pass_load<M, R>(buf, sj, v);
    lds_sync<WAVE>();
    int op[8];
    pass_compute<M, R, NS, INV>(v, j, op, tw);
    pass_store<M, R, NS>(buf, j, v);
    lds_sync<WAVE>();
    mid_passes<LOGM, P + 1, INV, WAVE>(buf, j, sj, v, tw);
  }
}

// The first pass's inputs of an M-point transform from buf, and the last
// pass's outputs into buf (at op[e] of fft()).
template <int LOGM>
__device__ __forceinline__ void fft_load(const SwzBuf& buf, int j, c2* v) {
  pass_load<1 << LOGM, pass_radix(LOGM, 0)>(buf, buf.part(j), v);
}
template <int LOGM>
__device__ __forceinline__ void fft_store(const SwzBuf& buf, int j, const c2* v) {
  constexpr int NP = pass_count(LOGM);
  pass_store<1 << LOGM, pass_radix(LOGM, NP - 1), pass_span(LOGM, NP - 1)>(buf, j, v);
}

// Full M-point FFT: v holds the first pass's inputs (v[e] = input at
// in_pos of pass 0); on return v holds the last pass's outputs at positions
// op[e].  Uses buf (M complex, this window's slot) between passes.
template <int LOGM, bool INV, bool WAVE = false, class TW = HwTwiddle>
__device__ __forceinline__ void fft(const SwzBuf& buf, int j, c2* v, int* op, const TW& tw = TW{}) {
  constexpr int M = 1 << LOGM;
  constexpr int NP = pass_count(LOGM);
  constexpr int R0 = pass_radix(LOGM, 0);
  pass_compute<M, R0, 1, INV>(v, j, op, tw);
  if constexpr (NP > 1) {
    pass_store<M, R0, 1>(buf, j, v);
    lds_sync<WAVE>();
    const int sj = buf.part(j);
    mid_passes<LOGM, 1, INV, WAVE>(buf, j, sj, v, tw);
    constexpr int RL = pass_radix(LOGM, NP - 1), NSL = pass_span(LOGM, NP - 1);
    pass_load<M, RL>(buf, sj, v);
    lds_sync<WAVE>();
    pass_compute<M, RL, NSL, INV>(v, j, op, tw);
  }
}

// Two M-point transforms of the same direction in one pass sequence (a and
// b in buffers bufa and bufb of the same slot): each pass's twiddles,
// positions and LDS round trip serve both, and the two butterflies give the
// scheduler independent work.  Each signal's arithmetic is exactly that of
// fft().
template <int M, int R, int NS, bool INV, class TW = HwTwiddle>
__device__ __forceinline__ void pass_compute2(c2* va, c2* vb, int j, int* outpos, const TW& tw = TW{}) {
  constexpr int BPT = 8 / R;
#pragma unroll
  for (int u = 0; u < BPT; ++u) {
    const int k = (j + u * (M / 8)) % NS;
    c2* wa = va + u * R;
    c2* wb = vb + u * R;
    if (NS > 1) {
      if constexpr (TW::kTable) {
#pragma unroll
        for (int r = 1; r < R; ++r) {
          const c2 t0 = tw.template pass_tw<M, R, NS>(u, r, k);
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
  }
  pass_positions<M, R, NS>(j, outpos);
}

template <int LOGM, int P, bool INV, bool WAVE, class TW = HwTwiddle>
__device__ __forceinline__ void mid_passes2(const SwzBuf& bufa, const SwzBuf& bufb, int j, int sj, c2* va, c2* vb,
                                            const TW& tw = TW{}) {
  constexpr int M = 1 << LOGM;
  if constexpr (P < pass_count(LOGM) - 1) {
    constexpr int R = pass_radix(LOGM, P), NS = pass_span(LOGM, P);
    pass_load<M, R>(bufa, sj, va);
    pass_load<M, R>(bufb, sj, vb);
    lds_sync<WAVE>();
    int op[8];
    pass_compute2<M, R, NS, INV>(va, vb, j, op, tw);
    pass_store<M, R, NS>(bufa, j, va);
    pass_store<M, R, NS>(bufb, j, vb);
    lds_sync<WAVE>();
    mid_passes2<LOGM, P + 1, INV, WAVE>(bufa, bufb, j, sj, va, vb, tw);
  }
}

// fft() of two signals at once (bufa and bufb: the same slot of two
// buffers): on return va / vb hold their last pass's outputs at positions
// op[e].
template <int LOGM, bool INV, bool WAVE = false, class TW = HwTwiddle>
__device__ __forceinline__ void fft2(const SwzBuf& bufa, const SwzBuf& bufb, int j, c2* va, c2* vb, int* op,
                                     const TW& tw = TW{}) {
  constexpr int M = 1 << LOGM;
  constexpr int NP = pass_count(LOGM);
  constexpr int R0 = pass_radix(LOGM, 0);
  pass_compute2<M, R0, 1, INV>(va, vb, j, op, tw);
  if constexpr (NP > 1) {
    pass_store<M, R0, 1>(bufa, j, va);
    pass_store<M, R0, 1>(bufb, j, vb);
    lds_sync<WAVE>();
    const int sj = bufa.part(j);  // bufb.part(j) too: the slots start alike
    mid_passes2<LOGM, 1, INV, WAVE>(bufa, bufb, j, sj, va, vb, tw);
    constexpr int RL = pass_radix(LOGM, NP - 1), NSL = pass_span(LOGM, NP - 1);
    pass_load<M, RL>(bufa, sj, va);
    pass_load<M, RL>(bufb, sj, vb);
    lds_sync<WAVE>();
    pass_compute2<M, RL, NSL, INV>(va, vb, j, op, tw);
  }
}

}  // namespace dgen
