// Batched harmonic + FIR-noise synth (HarmonicSynth.renderBatchedSignal,
// Examples/HarmonicE2E/Synth.swift:47-102) and its adjoint.
//
// Time is cut into segments of `seg` (<= 64) frames.  The only true
// recurrence is the tensor phasor (Sources/DGen/Emit+State.swift:322-369):
// one lane per (batch, harmonic) accumulates phase sequentially in fp32.
// k_phasor_carry runs that chain once over the whole signal (lane = wave
// lane, phase in a VGPR) and stores the phase at each segment start; every
// other kernel restarts the chain from those checkpoints, so all remaining
// work is parallel over (segment, batch) and bit-identical to the sequential
// evaluation.  The chain, the sampleRow interpolation and every sum are
// evaluated in the reference's operation order with contraction disabled.
//
// Layouts: ctrl rows [B*F][ldc] (row = b*F + f); f0, uv [F][B]; y, dy
// [B][T]; lerp table [T][8] = lo, hi, frac, 1-frac, slot(lo), slot(hi);
// checkpoints [nseg][B][K]; noise [T].
#pragma clang fp contract(off)

#include "internal.h"

namespace dgen {

constexpr int kMaxSeg = 64;   // frames per segment (one thread per frame)
constexpr int kMaxK = 64;     // harmonics (one lane per harmonic)
constexpr int kMaxNC = 128;   // control columns (one thread per column)
constexpr int kSlots = 4;     // distinct control rows a segment may touch
constexpr float kTwoPi = 2.0f * 3.14159265358979323846f;  // 2*Float.pi

__device__ __forceinline__ float phasor_wrap(float next) {
  float w = next - floorf(next);
  return w >= 1.0f ? w - 1.0f : w;
}

// ------------------------------------------------------------ carry pass
__global__ __launch_bounds__(64) void k_phasor_carry(const float* __restrict__ lerp, const float* __restrict__ f0,
                                                     float* __restrict__ ckpt, int B, int K, int T, int seg, float sr) {
  const int lane = blockIdx.x * blockDim.x + threadIdx.x;
  if (lane >= B * K) return;
  const int b = lane / K;
  const float kf = (float)(lane % K + 1);
  const int BK = B * K;
  float ph = 0.f;
  int until = 0, s = 0;
  for (int t = 0; t < T; ++t) {
    if (t == until) {
      ckpt[(size_t)s * BK + lane] = ph;
      ++s;
      until += seg;
    }
    const float* e = lerp + (size_t)t * 8;
    const int lo = (int)e[0], hi = (int)e[1];
    const float f0i = e[3] * f0[lo * B + b] + e[2] * f0[hi * B + b];
    const float freq = kf * f0i;
    ph = phasor_wrap(ph + freq / sr);
  }
}

int launch_phasor_carry(const Launch& L, const dgen_hip_op& op) {
  const int64_t lerp = op.arg[0], f0 = op.arg[1], ck = op.arg[2], B = op.arg[3], K = op.arg[4], F = op.arg[5],
                T = op.arg[6], seg = op.arg[7];
  DGEN_REQUIRE(B > 0 && K > 0 && F > 0 && T > 0 && seg > 0 && B * K <= (1 << 24) && T <= (1 << 26),
               "phasor_carry: B %lld K %lld F %lld T %lld seg %lld", (long long)B, (long long)K, (long long)F,
               (long long)T, (long long)seg);
  const int64_t nseg = (T + seg - 1) / seg;
  DGEN_CHECK_CELL(L, lerp, T * 8, "phasor_carry.lerp");
  DGEN_CHECK_CELL(L, f0, F * B, "phasor_carry.f0");
  DGEN_CHECK_CELL(L, ck, nseg * B * K, "phasor_carry.checkpoints");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_phasor_carry, dim3((unsigned)((B * K + 63) / 64)), dim3(64), 0, L.stream, cell(L, lerp),
                     cell(L, f0), cell(L, ck), (int)B, (int)K, (int)T, (int)seg, op.farg[0]);
  DGEN_LAUNCH_CHECK("k_phasor_carry");
  return 0;
}

// ------------------------------------------------------------ shared per-frame prologue
struct FrameRow {
  int lo, hi, slo, shi;
  float frac, omf;
};

__device__ __forceinline__ FrameRow frame_row(const float* __restrict__ lerp, int t) {
  const float* e = lerp + (size_t)t * 8;
  FrameRow r;
  r.lo = (int)e[0];
  r.hi = (int)e[1];
  r.frac = e[2];
  r.omf = e[3];
  r.slo = (int)e[4];
  r.shi = (int)e[5];
  return r;
}

struct SynthArgs {
  const float* ctrl;
  int ldc;
  const float* f0;
  const float* uv;
  const float* lerp;
  const float* noise;
  const float* ckpt;
  int B, K, NF, F, T, seg;
  float sr, hscale, nscale;
};

// ------------------------------------------------------------ forward
__global__ __launch_bounds__(64) void k_synth_fwd(SynthArgs a, float* __restrict__ y) {
  __shared__ float s_den[kMaxSeg], s_f0[kMaxSeg], s_omf[kMaxSeg], s_frac[kMaxSeg];
  __shared__ int s_lo[kMaxSeg], s_hi[kMaxSeg];
  __shared__ float s_contrib[kMaxSeg][kMaxK + 1];
  const int s = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int t0 = s * a.seg, nt = min(a.seg, a.T - t0);
  const float nyq = a.sr * 0.5f;

  if (tid < nt) {  // phase A: per-frame interpolation and harmonic normaliser
    const int t = t0 + tid;
    const FrameRow r = frame_row(a.lerp, t);
    const float f0i = r.omf * a.f0[r.lo * a.B + b] + r.frac * a.f0[r.hi * a.B + b];
    const float* c0 = a.ctrl + (size_t)(b * a.F + r.lo) * a.ldc;
    const float* c1 = a.ctrl + (size_t)(b * a.F + r.hi) * a.ldc;
    float den = 0.f;
    for (int k = 0; k < a.K; ++k) {
      const float freq = (float)(k + 1) * f0i;
      const float amp = r.omf * c0[k] + r.frac * c1[k];
      den = den + amp * (freq < nyq ? 1.0f : 0.0f);
    }
    s_den[tid] = den + 1e-8f;
    s_f0[tid] = f0i;
    s_omf[tid] = r.omf;
    s_frac[tid] = r.frac;
    s_lo[tid] = r.lo;
    s_hi[tid] = r.hi;
  }
  __syncthreads();
  if (tid < a.K) {  // phase B: one lane per harmonic runs the phasor from the checkpoint
    const float kf = (float)(tid + 1);
    float ph = a.ckpt[((size_t)s * a.B + b) * a.K + tid];
    for (int i = 0; i < nt; ++i) {
      const float freq = kf * s_f0[i];
      const float p = ph;
      ph = phasor_wrap(ph + freq / a.sr);
      const float sn = sinf(p * kTwoPi);
      const float* c0 = a.ctrl + (size_t)(b * a.F + s_lo[i]) * a.ldc;
      const float* c1 = a.ctrl + (size_t)(b * a.F + s_hi[i]) * a.ldc;
      const float masked = (s_omf[i] * c0[tid] + s_frac[i] * c1[tid]) * (freq < nyq ? 1.0f : 0.0f);
      s_contrib[i][tid] = sn * (masked / s_den[i]);
    }
  }
  __syncthreads();
  if (tid < nt) {  // phase C: sum over harmonics, FIR noise, mix
    const int t = t0 + tid;
    const float omf = s_omf[tid], frac = s_frac[tid];
    const float* c0 = a.ctrl + (size_t)(b * a.F + s_lo[tid]) * a.ldc;
    const float* c1 = a.ctrl + (size_t)(b * a.F + s_hi[tid]) * a.ldc;
    float hsum = 0.f;
    for (int k = 0; k < a.K; ++k) hsum = hsum + s_contrib[tid][k];
    const float gain = omf * c0[a.K] + frac * c1[a.K];
    const float ngain = omf * c0[a.K + 1] + frac * c1[a.K + 1];
    const float uvi = omf * a.uv[s_lo[tid] * a.B + b] + frac * a.uv[s_hi[tid] * a.B + b];
    float filt = 0.f;
    for (int i = 0; i < a.NF; ++i) {
      const int tt = t - (a.NF - 1) + i;
      const float w = tt >= 0 ? a.noise[tt] : 0.f;
      filt = filt + w * (omf * c0[a.K + 2 + i] + frac * c1[a.K + 2 + i]);
    }
    const float hout = ((hsum * gain) * uvi) * a.hscale;
    const float nout = ((filt * ngain) * 0.12f) * a.nscale;
    const float v = hout + nout;
    y[(size_t)b * a.T + t] = isfinite(v) ? v : 0.f;  // dgen_runtime.h:58-85 containment
  }
}

// ------------------------------------------------------------ backward
// Per (segment, batch): recompute the forward quantities, then one thread
// per control column accumulates its gradient into <= 4 row slots.
__global__ __launch_bounds__(128) void k_synth_bwd(SynthArgs a, const float* __restrict__ dy,
                                                   float* __restrict__ part) {
  __shared__ float s_den[kMaxSeg], s_f0[kMaxSeg], s_omf[kMaxSeg], s_frac[kMaxSeg];
  __shared__ int s_lo[kMaxSeg], s_hi[kMaxSeg], s_slo[kMaxSeg], s_shi[kMaxSeg];
  __shared__ float s_dhsum[kMaxSeg], s_dot[kMaxSeg], s_dgain[kMaxSeg], s_dngain[kMaxSeg], s_dfilt[kMaxSeg];
  __shared__ float s_sin[kMaxSeg][kMaxK + 1];
  __shared__ float s_amp[kMaxSeg][kMaxK + 1];
  const int s = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int t0 = s * a.seg, nt = min(a.seg, a.T - t0);
  const int nseg = (a.T + a.seg - 1) / a.seg;
  const float nyq = a.sr * 0.5f;

  if (tid < nt) {
    const int t = t0 + tid;
    const FrameRow r = frame_row(a.lerp, t);
    const float f0i = r.omf * a.f0[r.lo * a.B + b] + r.frac * a.f0[r.hi * a.B + b];
    const float* c0 = a.ctrl + (size_t)(b * a.F + r.lo) * a.ldc;
    const float* c1 = a.ctrl + (size_t)(b * a.F + r.hi) * a.ldc;
    float den = 0.f;
    for (int k = 0; k < a.K; ++k) {
      const float freq = (float)(k + 1) * f0i;
      den = den + (r.omf * c0[k] + r.frac * c1[k]) * (freq < nyq ? 1.0f : 0.0f);
    }
    s_den[tid] = den + 1e-8f;
    s_f0[tid] = f0i;
    s_omf[tid] = r.omf;
    s_frac[tid] = r.frac;
    s_lo[tid] = r.lo;
    s_hi[tid] = r.hi;
    s_slo[tid] = r.slo;
    s_shi[tid] = r.shi;
  }
  __syncthreads();
  if (tid < a.K) {
    const float kf = (float)(tid + 1);
    float ph = a.ckpt[((size_t)s * a.B + b) * a.K + tid];
    for (int i = 0; i < nt; ++i) {
      const float freq = kf * s_f0[i];
      const float p = ph;
      ph = phasor_wrap(ph + freq / a.sr);
      s_sin[i][tid] = sinf(p * kTwoPi);
      const float* c0 = a.ctrl + (size_t)(b * a.F + s_lo[i]) * a.ldc;
      const float* c1 = a.ctrl + (size_t)(b * a.F + s_hi[i]) * a.ldc;
      const float masked = (s_omf[i] * c0[tid] + s_frac[i] * c1[tid]) * (freq < nyq ? 1.0f : 0.0f);
      s_amp[i][tid] = masked / s_den[i];
    }
  }
  __syncthreads();
  if (tid < nt) {
    const int t = t0 + tid;
    const float omf = s_omf[tid], frac = s_frac[tid];
    const float* c0 = a.ctrl + (size_t)(b * a.F + s_lo[tid]) * a.ldc;
    const float* c1 = a.ctrl + (size_t)(b * a.F + s_hi[tid]) * a.ldc;
    float hsum = 0.f;
    for (int k = 0; k < a.K; ++k) hsum = hsum + s_sin[tid][k] * s_amp[tid][k];
    const float gain = omf * c0[a.K] + frac * c1[a.K];
    const float ngain = omf * c0[a.K + 1] + frac * c1[a.K + 1];
    const float uvi = omf * a.uv[s_lo[tid] * a.B + b] + frac * a.uv[s_hi[tid] * a.B + b];
    float filt = 0.f;
    for (int i = 0; i < a.NF; ++i) {
      const int tt = t - (a.NF - 1) + i;
      const float w = tt >= 0 ? a.noise[tt] : 0.f;
      filt = filt + w * (omf * c0[a.K + 2 + i] + frac * c1[a.K + 2 + i]);
    }
    const float g = dy[(size_t)b * a.T + t];
    const float dhsum = g * gain * uvi * a.hscale;
    float dot = 0.f;
    for (int k = 0; k < a.K; ++k) dot = dot + dhsum * s_sin[tid][k] * s_amp[tid][k];
    s_dhsum[tid] = dhsum;
    s_dot[tid] = dot;
    s_dgain[tid] = g * hsum * uvi * a.hscale;
    s_dfilt[tid] = g * ngain * 0.12f * a.nscale;
    s_dngain[tid] = g * filt * 0.12f * a.nscale;
  }
  __syncthreads();
  const int NC = a.K + 2 + a.NF;
  if (tid < NC) {
    float acc[kSlots] = {0.f, 0.f, 0.f, 0.f};
    const float kf = (float)(tid + 1);
    for (int i = 0; i < nt; ++i) {
      float dm;
      if (tid < a.K) {
        const float mk = kf * s_f0[i] < nyq ? 1.0f : 0.0f;
        dm = (s_dhsum[i] * s_sin[i][tid] - s_dot[i]) / s_den[i] * mk;
      } else if (tid == a.K) {
        dm = s_dgain[i];
      } else if (tid == a.K + 1) {
        dm = s_dngain[i];
      } else {
        const int tt = t0 + i - (a.NF - 1) + (tid - a.K - 2);
        dm = s_dfilt[i] * (tt >= 0 ? a.noise[tt] : 0.f);
      }
      acc[s_slo[i]] += s_omf[i] * dm;
      acc[s_shi[i]] += s_frac[i] * dm;
    }
    float* out = part + ((size_t)b * nseg + s) * kSlots * a.ldc;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) out[(size_t)j * a.ldc + tid] = acc[j];
  }
}

// d ctrl[b*F+f][c] = sum over the (segment, slot) entries listed for row f.
__global__ void k_synth_bwd_reduce(const float* __restrict__ part, const float* __restrict__ row_list,
                                   float* __restrict__ dctrl, int B, int NC, int ldc, int F, int nseg) {
  const int c = threadIdx.x;
  const int f = blockIdx.x, b = blockIdx.y;
  if (c >= ldc) return;
  float s = 0.f;
  if (c < NC) {
    const float* lst = row_list + (size_t)f * 8;
    for (int q = 0; q < 8; ++q) {
      const float e = lst[q];
      if (e < 0.f) break;
      const int ent = (int)e;
      const int seg = ent / kSlots, slot = ent % kSlots;
      s += part[(((size_t)b * nseg + seg) * kSlots + slot) * ldc + c];
    }
  }
  dctrl[((size_t)b * F + f) * ldc + c] = s;
}

static int synth_args(const Launch& L, const dgen_hip_op& op, SynthArgs& a, const char* who) {
  // arg: [0]=ctrl [1]=f0 [2]=uv [3]=lerp [4]=checkpoints [5]=y/dy [6]=B [7]=K [8]=NF [9]=F [10]=T [11]=seg
  //      [12]=partials (bwd) [13]=noise [14]=ldc
  const int64_t B = op.arg[6], K = op.arg[7], NF = op.arg[8], F = op.arg[9], T = op.arg[10], seg = op.arg[11];
  const int64_t ldc = op.arg[14];
  DGEN_REQUIRE(B > 0 && B <= 65535 && K > 0 && K <= kMaxK && NF > 0 && F > 0 && T > 0 && T <= (1 << 26) &&
                   seg > 0 && seg <= kMaxSeg && K + 2 + NF <= kMaxNC && ldc >= K + 2 + NF,
               "%s: B %lld K %lld NF %lld F %lld T %lld seg %lld ldc %lld", who, (long long)B, (long long)K,
               (long long)NF, (long long)F, (long long)T, (long long)seg, (long long)ldc);
  const int64_t nseg = (T + seg - 1) / seg;
  DGEN_REQUIRE(nseg <= 2147483647ll, "%s: too many segments", who);
  DGEN_CHECK_CELL(L, op.arg[0], B * F * ldc, "synth.ctrl");
  DGEN_CHECK_CELL(L, op.arg[1], F * B, "synth.f0");
  DGEN_CHECK_CELL(L, op.arg[2], F * B, "synth.uv");
  DGEN_CHECK_CELL(L, op.arg[3], T * 8, "synth.lerp");
  DGEN_CHECK_CELL(L, op.arg[4], nseg * B * K, "synth.checkpoints");
  DGEN_CHECK_CELL(L, op.arg[5], B * T, "synth.y");
  DGEN_CHECK_CELL(L, op.arg[13], T, "synth.noise");
  if (L.dry) return 0;
  a.ctrl = cell(L, op.arg[0]);
  a.ldc = (int)ldc;
  a.f0 = cell(L, op.arg[1]);
  a.uv = cell(L, op.arg[2]);
  a.lerp = cell(L, op.arg[3]);
  a.ckpt = cell(L, op.arg[4]);
  a.noise = cell(L, op.arg[13]);
  a.B = (int)B;
  a.K = (int)K;
  a.NF = (int)NF;
  a.F = (int)F;
  a.T = (int)T;
  a.seg = (int)seg;
  a.sr = op.farg[0];
  a.hscale = op.farg[1];
  a.nscale = op.farg[2];
  return 0;
}

int launch_synth_fwd(const Launch& L, const dgen_hip_op& op) {
  SynthArgs a{};
  int rc = synth_args(L, op, a, "synth_fwd");
  if (rc || L.dry) return rc;
  const int nseg = (a.T + a.seg - 1) / a.seg;
  hipLaunchKernelGGL(k_synth_fwd, dim3((unsigned)nseg, (unsigned)a.B), dim3(64), 0, L.stream, a, cell(L, op.arg[5]));
  DGEN_LAUNCH_CHECK("k_synth_fwd");
  return 0;
}

int launch_synth_bwd(const Launch& L, const dgen_hip_op& op) {
  SynthArgs a{};
  int rc = synth_args(L, op, a, "synth_bwd");
  if (rc) return rc;
  const int64_t T = op.arg[10], seg = op.arg[11], B = op.arg[6], ldc = op.arg[14];
  const int64_t nseg = (T + seg - 1) / seg;
  DGEN_CHECK_CELL(L, op.arg[12], B * nseg * kSlots * ldc, "synth_bwd.partials");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_synth_bwd, dim3((unsigned)nseg, (unsigned)a.B), dim3(128), 0, L.stream, a,
                     cell(L, op.arg[5]), cell(L, op.arg[12]));
  DGEN_LAUNCH_CHECK("k_synth_bwd");
  return 0;
}

int launch_synth_bwd_reduce(const Launch& L, const dgen_hip_op& op) {
  // arg: [0]=partials [1]=row_list [2]=dctrl [3]=B [4]=NC [5]=F [6]=T [7]=seg [8]=ldc
  const int64_t part = op.arg[0], rl = op.arg[1], dc = op.arg[2], B = op.arg[3], NC = op.arg[4], F = op.arg[5],
                T = op.arg[6], seg = op.arg[7], ldc = op.arg[8];
  DGEN_REQUIRE(B > 0 && B <= 65535 && NC > 0 && ldc >= NC && ldc <= 1024 && F > 0 && T > 0 && seg > 0,
               "synth_bwd_reduce: B %lld NC %lld F %lld T %lld seg %lld ldc %lld", (long long)B, (long long)NC,
               (long long)F, (long long)T, (long long)seg, (long long)ldc);
  const int64_t nseg = (T + seg - 1) / seg;
  DGEN_CHECK_CELL(L, part, B * nseg * kSlots * ldc, "synth_bwd_reduce.partials");
  DGEN_CHECK_CELL(L, rl, F * 8, "synth_bwd_reduce.row_list");
  DGEN_CHECK_CELL(L, dc, B * F * ldc, "synth_bwd_reduce.dctrl");
  if (L.dry) return 0;
  hipLaunchKernelGGL(k_synth_bwd_reduce, dim3((unsigned)F, (unsigned)B), dim3((unsigned)((ldc + 63) / 64 * 64)), 0,
                     L.stream, cell(L, part), cell(L, rl), cell(L, dc), (int)B, (int)NC, (int)ldc, (int)F, (int)nseg);
  DGEN_LAUNCH_CHECK("k_synth_bwd_reduce");
  return 0;
}

}  // namespace dgen
