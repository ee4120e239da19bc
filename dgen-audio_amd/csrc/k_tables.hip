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
// reset 0; output = clip(pre-increment value, lo, hi).
__global__ void k_accum_table(float* out, int frames, float step, float mn, float mx, float lo, float hi) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  float acc = 0.f;
  const float span = mx - mn;
  for (int t = 0; t < frames; ++t) {
    float prev = acc;
    float next = acc + step;
    float k = floorf((next - mn) / span);
    float w = next - k * span;
    if (w >= mx) w = w - span;
    acc = w;
    float p = prev < lo ? lo : prev;
    out[t] = p > hi ? hi : p;
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
// from the zeroed cell, so the per-run stream is this fixed sequence.
__global__ void k_noise_table(float* out, int frames) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  uint32_t s = 0u;
  for (int t = 0; t < frames; ++t) {
    if (s == 0u) s = 1u;
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    out[t] = (float)s / 4294967296.0f;
  }
}

int launch_noise_table(const Launch& L, const dgen_hip_op& op) {
  const int64_t out = op.arg[0], frames = op.arg[1];
  DGEN_REQUIRE(frames > 0 && frames <= (1 << 26), "noise_table: frames %lld", (long long)frames);
  DGEN_CHECK_CELL(L, out, frames, "noise_table.out");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_noise_table, dim3(1), dim3(64), 0, L.stream, cell(L, out), (int)frames);
  DGEN_LAUNCH_CHECK("k_noise_table");
  return 0;
}

// Row schedule of a sampleRow read driven by a playhead table
// (Sources/DGen/Emit+RowSelection.swift:164-197: fmod wrap, floor/ceil with
// wrap to 0, frac, 1-frac).  Produces
//   lerp[t][8]   = lo, hi, frac, 1-frac, slot(lo), slot(hi), 0, 0
//   seg_rows[s][4] = distinct rows touched by frame segment s (-1 unused)
//   row_list[f][kRowEntries] = (segment*4 + slot) entries that touch row f (-1 unused)
//   flag[0]      = 0 ok, 1 a segment touches > 4 rows, 2 a row has > 8 entries,
//                  3 a non-finite playhead
// The gradient of a row read is then reduced per row in a fixed order.
constexpr int kSlots = 4;

__global__ void k_row_schedule(const float* play, float* lerp, float* seg_rows, float* row_list, float* flag,
                               int rows, int frames, int seg) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  const int nseg = (frames + seg - 1) / seg;
  for (int i = 0; i < nseg * kSlots; ++i) seg_rows[i] = -1.f;
  for (int i = 0; i < rows * kRowEntries; ++i) row_list[i] = -1.f;
  float status = 0.f;
  const float nr = (float)rows;
  for (int s = 0; s < nseg; ++s) {
    int srow[kSlots] = {-1, -1, -1, -1};
    int nslot = 0;
    for (int t = s * seg; t < frames && t < (s + 1) * seg; ++t) {
      float w = fmodf(play[t], nr);
      if (w < 0.f) w = w + nr;
      float fl = floorf(w);
      if (!(fl >= 0.f && fl < nr)) {  // non-finite playhead: keep every index in range
        fl = 0.f;
        w = 0.f;
        status = 3.f;
      }
      float ce = fl + 1.0f;
      if (ce >= nr) ce = 0.f;
      float frac = w - fl;
      int ids[2] = {(int)fl, (int)ce};
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
            status = 1.f;
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
    for (int j = 0; j < nslot; ++j) {
      seg_rows[s * kSlots + j] = (float)srow[j];
      float* lst = row_list + (size_t)srow[j] * kRowEntries;
      int q = 0;
      while (q < kRowEntries && lst[q] >= 0.f) ++q;
      if (q < kRowEntries)
        lst[q] = (float)(s * kSlots + j);
      else
        status = 2.f;
    }
  }
  flag[0] = status;
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
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_row_schedule, dim3(1), dim3(64), 0, L.stream, cell(L, play), cell(L, lerp), cell(L, segr),
                     cell(L, rowl), cell(L, flag), (int)rows, (int)frames, (int)seg);
  DGEN_LAUNCH_CHECK("k_row_schedule");
  return 0;
}

// Spectral-loss tables for one FFT size (Sources/DGen/HigherOps.swift:71-99):
// symmetric Hann 0.5*(1-cos(2*pi*i/(N-1))) and twiddles cos/sin(2*pi*k/(2h))
// at offset h-1, all evaluated in double and rounded to float.
// out = hann[N] | twre[N-1] | twim[N-1].
__global__ void k_fft_tables(float* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const double two_pi = 6.283185307179586476925286766559;
  if (i < n) out[i] = (float)(0.5 * (1.0 - cos(two_pi * (double)i / (double)(n - 1))));
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
  const int64_t out = op.arg[0], n = op.arg[1];
  DGEN_REQUIRE(n >= 2 && n <= 65536 && (n & (n - 1)) == 0, "fft_tables: N=%lld must be a power of two", (long long)n);
  DGEN_CHECK_CELL(L, out, 3 * n - 2, "fft_tables.out");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_fft_tables, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, L.stream, cell(L, out), (int)n);
  DGEN_LAUNCH_CHECK("k_fft_tables");
  return 0;
}

}  // namespace dgen
