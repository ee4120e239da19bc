// Device arithmetic shared by the recurrence kernels: fp32 reciprocal and
// quotient rounded like IEEE division (hardware estimate + one correction).
#pragma once

#include <hip/hip_runtime.h>

namespace dgen {

// RN(1/d): v_rcp_f32 (1 ulp) refined by one Newton step in fma.
__device__ __forceinline__ float rcp_rn(float d) {
  const float r = __builtin_amdgcn_rcpf(d);
  return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
}

// x / d with rd = RN(1/d): one Markstein correction of x*rd.
__device__ __forceinline__ float div_rn(float x, float d, float rd) {
  const float q = x * rd;
  return __builtin_fmaf(__builtin_fmaf(-q, d, x), rd, q);
}

}  // namespace dgen
