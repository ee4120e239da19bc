// Static-temporality tables: blocks of the schedule whose values depend only
// on constants, evaluated once at configure time (the reference evaluates them
// every run, but with identical results because every run starts from zeroed
// state: LazyGraph.run -> zeroAllBuffers, Sources/DGenLazy/Realize.swift:285-290).
//
// All arithmetic here is the reference's fp32 recurrences evaluated
// sequentially; contraction is disabled so the tables are bit-identical to a
// strict IEEE evaluation of the same expressions.
#pragma clang fp contract(off)

#include "internal.h"

namespace dgen {

// u_accum (Sources/DGen/Definitions.swift:215-246) with constant increment,
// reset 0; output = clip(pre-increment value, lo, hi).  The chain is
// sequential in fp32.  Where next lies in [mn, mn + span * 0.99) the wrap
// quotient (next - mn) / span rounds below 1, so k = 0 and w = next exactly:
// those frames skip the division; the others take the full expression.  One
// wave runs the (uniform) chain in every lane; lane t % 64 keeps frame t, and
// each 64 frames leave in one coalesced store (a lone lane storing every
// frame is bound by its outstanding-store limit).
__global__ __launch_bounds__(64) void k_accum_table(float* out, int frames, float step, float mn, float mx, float lo,
                                                    float hi) {
  const int lane = threadIdx.x;
  float acc = 0.f;
  const float span = mx - mn;
  const float safe = span * 0.99f;
  // a block of 64 adds moves acc by at most 64 step plus 64 roundings of
  // half an ulp of |acc| <= |mn| + |mx| (+ a margin)
  const float drift = 65.f * step + 65.f * (fabsf(mx) + fabsf(mn) + fabsf(step)) * 1.2e-7f;
  for (int t0 = 0; t0 < frames; t0 += 64) {
    float mine = 0.f;
    const int n = min(64, frames - t0);
    if (n == 64 && step >= 0.f && acc - mn >= 0.f && (acc - mn) + drift < safe * 0.999f) {
      // every frame of the block takes the k = 0 path: branch-free
#pragma unroll
      for (int j = 0; j < 64; ++j) {
        mine = lane == j ? acc : mine;
        acc = acc + step;
      }
      const float p = mine < lo ? lo : mine;
      out[t0 + lane] = p > hi ? hi : p;
      continue;
    }
    for (int j = 0; j < n; ++j) {
      const float prev = acc;
      const float next = acc + step;
      const float d = next - mn;
      float w;
      if (d >= 0.f && d < safe) {
        w = next;
      } else {
        const float k = floorf(d / span);
        w = next - k * span;
        if (w >= mx) w = w - span;
      }
      acc = w;
      const float p = prev < lo ? lo : prev;
      if (lane == j) mine = p > hi ? hi : p;
    }
    if (lane < n) out[t0 + lane] = mine;
  }
}

int launch_accum_table(const Launch& L, const dgen_hip_op& op) {
  const int64_t out = op.arg[0], frames = op.arg[1];
  DGEN_REQUIRE(frames > 0 && frames <= (1 << 26), "accum_table: frames %lld", (long long)frames);
  DGEN_REQUIRE(op.farg[2] > op.farg[1], "accum_table: max must exceed min");
  DGEN_CHECK_CELL(L, out, frames, "accum_table.out");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_accum_table, dim3(1), dim3(64), 0, L.stream, cell(L, out), (int)frames, op.farg[0],
                     op.farg[1], op.farg[2], op.farg[3], op.farg[4]);
  DGEN_LAUNCH_CHECK("k_accum_table");
  return 0;
}

// Signal.noise(): xorshift32 on a zeroed float cell (state 0 -> 1), output
// s / 2^32 (Sources/DGen/Renderer/CRenderer.swift:685-693).  Every run starts
// from the zeroed cell, so the per-run stream is this fixed sequence:
// s_1 = xs(1), s_{n+1} = xs(s_n), out[n] = s_{n+1} / 2^32.
//
// xs is linear over GF(2) (shifts and xors), so s_n = M^(n-1) s_1 with M the
// 32x32 bit matrix whose column b is xs(1 << b).  Each of kNoiseThreads
// threads jumps to the start of its run of frames with M^chunk raised to its
// index (binary powering of bit matrices) and steps the run sequentially.
constexpr int kNoiseThreads = 256;

__device__ __forceinline__ uint32_t xs32(uint32_t s) {
  s ^= s << 13;
  s ^= s >> 17;
  s ^= s << 5;
  return s;
}
struct BitMat {
  uint32_t c[32];  // column b = image of bit b
};
__device__ __forceinline__ uint32_t bm_apply(const BitMat& m, uint32_t x) {
  uint32_t y = 0u;
#pragma unroll
  for (int b = 0; b < 32; ++b) y ^= ((x >> b) & 1u) ? m.c[b] : 0u;
  return y;
}
__device__ __forceinline__ BitMat bm_mul(const BitMat& a, const BitMat& b) {  // a after b
  BitMat r;
#pragma unroll
  for (int k = 0; k < 32; ++k) r.c[k] = bm_apply(a, b.c[k]);
  return r;
}
__device__ __forceinline__ BitMat bm_pow(BitMat base, uint32_t e) {
  BitMat r;
#pragma unroll
  for (int k = 0; k < 32; ++k) r.c[k] = 1u << k;
  while (e) {
    if (e & 1u) r = bm_mul(base, r);
    base = bm_mul(base, base);
    e >>= 1;
  }
  return r;
}

__global__ __launch_bounds__(kNoiseThreads) void k_noise_table(float* out, int frames) {
  const int i = threadIdx.x;
  const int chunk = (frames + kNoiseThreads - 1) / kNoiseThreads;
  const int t0 = i * chunk, t1 = min(frames, t0 + chunk);
  if (t0 >= t1) return;
  BitMat m;
#pragma unroll
  for (int b = 0; b < 32; ++b) m.c[b] = xs32(1u << b);
  uint32_t s = bm_apply(bm_pow(bm_pow(m, (uint32_t)chunk), (uint32_t)i), xs32(1u));  // s_{t0 + 1}
  for (int t = t0; t < t1; ++t) {
    out[t] = (float)s / 4294967296.0f;
    s = xs32(s);
  }
}

int launch_noise_table(const Launch& L, const dgen_hip_op& op) {
  const int64_t out = op.arg[0], frames = op.arg[1];
  DGEN_REQUIRE(frames > 0 && frames <= (1 << 26), "noise_table: frames %lld", (long long)frames);
  DGEN_CHECK_CELL(L, out, frames, "noise_table.out");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_noise_table, dim3(1), dim3(kNoiseThreads), 0, L.stream, cell(L, out), (int)frames);
  DGEN_LAUNCH_CHECK("k_noise_table");
  return 0;
}

// Row schedule of a sampleRow read driven by a playhead table
// (Sources/DGen/Emit+RowSelection.swift:164-197: fmod wrap, floor/ceil with
// wrap to 0, frac, 1-frac).  Produces
//   lerp[t][8]   = lo, hi, frac, 1-frac, slot(lo), slot(hi), 0, 0
//   seg_rows[s][4] = distinct rows touched by frame segment s, in the order
//                  its frames first touch them (-1 unused)
//   row_list[f][kRowEntries] = (segment*4 + slot) entries that touch row f,
//                  in segment order (-1 unused)
//   flag[0]      = 0 ok; else the largest of 1 (a segment touches > 4 rows),
//                  2 (a row has > kRowEntries entries), 3 (a non-finite playhead)
// The gradient of a row read is then reduced per row in a fixed order.
// Two passes: a thread per segment (its frames in order), then a thread per
// row (every segment's rows, in segment order).
constexpr int kSlots = 4;
constexpr int kSchedThreads = 256;

__global__ __launch_bounds__(kSchedThreads) void k_row_segments(const float* play, float* lerp, float* seg_rows,
                                                                 float* seg_status, int rows, int frames, int seg) {
  const int s = blockIdx.x * kSchedThreads + threadIdx.x;
  const int nseg = (frames + seg - 1) / seg;
  if (s >= nseg) return;
  const float nr = (float)rows;
  int srow[kSlots] = {-1, -1, -1, -1};
  int nslot = 0;
  float status = 0.f;
  for (int t = s * seg; t < frames && t < (s + 1) * seg; ++t) {
    float w = fmodf(play[t], nr);
    if (w < 0.f) w = w + nr;
    float fl = floorf(w);
    if (!(fl >= 0.f && fl < nr)) {  // non-finite playhead: keep every index in range
      fl = 0.f;
      w = 0.f;
      status = fmaxf(status, 3.f);
    }
    float ce = fl + 1.0f;
    if (ce >= nr) ce = 0.f;
    const float frac = w - fl;
    const int ids[2] = {(int)fl, (int)ce};
    int slots[2] = {0, 0};
    for (int q = 0; q < 2; ++q) {
      int found = -1;
      for (int j = 0; j < nslot; ++j)
        if (srow[j] == ids[q]) found = j;
      if (found < 0) {
        if (nslot < kSlots) {
          srow[nslot] = ids[q];
          found = nslot++;
        } else {
          status = fmaxf(status, 1.f);
          found = 0;
        }
      }
      slots[q] = found;
    }
    float* e = lerp + (size_t)t * 8;
    e[0] = fl;
    e[1] = ce;
    e[2] = frac;
    e[3] = 1.0f - frac;
    e[4] = (float)slots[0];
    e[5] = (float)slots[1];
    e[6] = 0.f;
    e[7] = 0.f;
  }
  for (int j = 0; j < kSlots; ++j) seg_rows[s * kSlots + j] = (float)srow[j];
  seg_status[s] = status;
}

// The segments' rows pass through LDS in tiles of kSegTile segments, read
// once per workgroup instead of once per row.
constexpr int kSegTile = 4096;

__global__ __launch_bounds__(kSchedThreads) void k_row_lists(const float* seg_rows, const float* seg_status,
                                                              float* row_list, float* row_status, int rows,
                                                              int nseg) {
  __shared__ float4 tile[kSegTile];
  const int f = blockIdx.x * kSchedThreads + threadIdx.x;
  int q = 0;
  float status = 0.f;
  float ent[kRowEntries];
#pragma unroll
  for (int k = 0; k < kRowEntries; ++k) ent[k] = -1.f;
  for (int s0 = 0; s0 < nseg; s0 += kSegTile) {
    const int n = min(kSegTile, nseg - s0);
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kSchedThreads)
      tile[i] = *reinterpret_cast<const float4*>(seg_rows + (size_t)(s0 + i) * kSlots);
    __syncthreads();
    if (f >= rows) continue;
    for (int i = 0; i < n; ++i) {
      const float4 r = tile[i];
      const float rv[kSlots] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int j = 0; j < kSlots; ++j) {
        if ((int)rv[j] != f || rv[j] < 0.f) continue;
        if (q < kRowEntries) {
#pragma unroll
          for (int k = 0; k < kRowEntries; ++k)
            if (k == q) ent[k] = (float)((s0 + i) * kSlots + j);
          ++q;
        } else {
          status = 2.f;
        }
      }
    }
  }
  if (f >= rows) return;
  float* lst = row_list + (size_t)f * kRowEntries;
#pragma unroll
  for (int k = 0; k < kRowEntries; ++k) lst[k] = ent[k];
  // the row's status, and (row 0) the segments' largest
  if (f == 0)
    for (int s = 0; s < nseg; ++s) status = fmaxf(status, seg_status[s]);
  row_status[f] = status;
}

// flag = the largest status (one workgroup, fixed order).
__global__ __launch_bounds__(kSchedThreads) void k_row_flag(const float* row_status, float* flag, int rows) {
  __shared__ float red[kSchedThreads];
  float m = 0.f;
  for (int f = threadIdx.x; f < rows; f += kSchedThreads) m = fmaxf(m, row_status[f]);
  red[threadIdx.x] = m;
  __syncthreads();
  for (int w = kSchedThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + w]);
    __syncthreads();
  }
  if (threadIdx.x == 0) flag[0] = red[0];
}

int launch_row_schedule(const Launch& L, const dgen_hip_op& op) {
  const int64_t play = op.arg[0], lerp = op.arg[1], segr = op.arg[2], rowl = op.arg[3], flag = op.arg[4];
  const int64_t rows = op.arg[5], frames = op.arg[6], seg = op.arg[7];
  DGEN_REQUIRE(rows > 0 && frames > 0 && seg > 0 && frames <= (1 << 26) && rows <= (1 << 22),
               "row_schedule: rows %lld frames %lld seg %lld", (long long)rows, (long long)frames, (long long)seg);
  const int64_t nseg = (frames + seg - 1) / seg;
  DGEN_CHECK_CELL(L, play, frames, "row_schedule.playhead");
  DGEN_CHECK_CELL(L, lerp, frames * 8, "row_schedule.lerp");
  DGEN_CHECK_CELL(L, segr, nseg * kSlots, "row_schedule.seg_rows");
  DGEN_CHECK_CELL(L, rowl, rows * kRowEntries, "row_schedule.row_list");
  DGEN_CHECK_CELL(L, flag, 1, "row_schedule.flag");
  const int64_t ws = op.arg[8];
  DGEN_CHECK_CELL(L, ws, nseg + rows, "row_schedule.workspace");
  DGEN_REQUIRE(segr % 4 == 0, "row_schedule: segment rows cell must be 16-byte aligned");
  if (L.dry) return 0;
  float* seg_status = cell(L, ws);
  float* row_status = seg_status + nseg;
  hipLaunchKernelGGL(k_row_segments, dim3((unsigned)((nseg + kSchedThreads - 1) / kSchedThreads)),
                     dim3(kSchedThreads), 0, L.stream, cell(L, play), cell(L, lerp), cell(L, segr), seg_status,
                     (int)rows, (int)frames, (int)seg);
  DGEN_LAUNCH_CHECK("k_row_segments");
  hipLaunchKernelGGL(k_row_lists, dim3((unsigned)((rows + kSchedThreads - 1) / kSchedThreads)), dim3(kSchedThreads),
                     0, L.stream, cell(L, segr), seg_status, cell(L, rowl), row_status, (int)rows, (int)nseg);
  DGEN_LAUNCH_CHECK("k_row_lists");
  hipLaunchKernelGGL(k_row_flag, dim3(1), dim3(kSchedThreads), 0, L.stream, row_status, cell(L, flag), (int)rows);
  DGEN_LAUNCH_CHECK("k_row_flag");
  return 0;
}

// Spectral-loss tables for one FFT size (Sources/DGen/HigherOps.swift:71-99):
// symmetric Hann 0.5*(1-cos(2*pi*i/(N-1))) and twiddles cos/sin(2*pi*k/(2h))
// at offset h-1, all evaluated in double and rounded to float.
// out = hann[N] | twre[N-1] | twim[N-1].
// rect: useHannWindow false, the all-1.0 window (HigherOps.swift:69-76).
__global__ void k_fft_tables(float* out, int n, int rect) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const double two_pi = 6.283185307179586476925286766559;
  if (i < n) out[i] = rect ? 1.0f : (float)(0.5 * (1.0 - cos(two_pi * (double)i / (double)(n - 1))));
  if (i < n - 1) {
    int h = 1;
    while (2 * h - 1 <= i) h <<= 1;  // i in [h-1, 2h-1)
    const int k = i - (h - 1);
    const double ang = two_pi * (double)k / (double)(2 * h);
    out[n + i] = (float)cos(ang);
    out[2 * n - 1 + i] = (float)sin(ang);
  }
}

int launch_fft_tables(const Launch& L, const dgen_hip_op& op) {
  const int64_t out = op.arg[0], n = op.arg[1], rect = op.arg[2];
  DGEN_REQUIRE(n >= 2 && n <= 65536 && (n & (n - 1)) == 0, "fft_tables: N=%lld must be a power of two", (long long)n);
  DGEN_REQUIRE(rect == 0 || rect == 1, "fft_tables: window kind %lld", (long long)rect);
  DGEN_CHECK_CELL(L, out, 3 * n - 2, "fft_tables.out");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_fft_tables, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, L.stream, cell(L, out), (int)n,
                     (int)rect);
  DGEN_LAUNCH_CHECK("k_fft_tables");
  return 0;
}

}  // namespace dgen
