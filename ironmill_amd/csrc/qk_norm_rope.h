// qk_norm_rope.h -- per-head RMSNorm + rotary embedding at head_dim =
// rotary_dim = 128 (fused_qk_norm_rope.metal:43-124, pairs (d, d + 64)), held
// by one wave: lane l has elements l and l + 64, which are exactly the two
// members of rotation pair l.  Shared by the stand-alone kernel
// (glue_kernels.hip), the TurboQuant cache write (K) and the TurboQuant
// attention prologue (Q), so every path rounds the same f32 operations.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "dpp_reduce.h"

namespace imh_qk {

constexpr int kHd = 128;

// Sum over the 64 lanes of a wave (DPP rows, then two xor shuffles).
__device__ __forceinline__ float wave_sum64(float v) {
    v = imh_dpp::row16_sum(v);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// Table row of a position: positions clamp into [0, max_pos).
__device__ __forceinline__ long clamp_pos(long pos, int max_pos) {
    return pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
}

// x0 = element lane, x1 = element lane + 64 of one head; w0 / w1 the norm
// weights of those elements, c / s the cos / sin of pair lane at the
// position.  Writes back the normalised, rotated pair rounded to f16
// (returned as f32).
__device__ __forceinline__ void norm_rope_128(float &x0, float &x1, float w0, float w1, float c, float s,
                                              float eps) {
    const float ss = wave_sum64(__builtin_fmaf(x1, x1, x0 * x0));
    const float rms_inv = 1.0f / sqrtf(ss / (float)kHd + eps);
    const float lo = x0 * rms_inv * w0;
    const float hi = x1 * rms_inv * w1;
    x0 = __half2float(__float2half(__builtin_fmaf(lo, c, -(hi * s))));
    x1 = __half2float(__float2half(__builtin_fmaf(lo, s, hi * c)));
}

// The same with the norm weight [128] and the cos / sin table rows [64] of
// the position given as pointers.
__device__ __forceinline__ void norm_rope_128(float &x0, float &x1, int lane, const __half *__restrict__ nw,
                                              const __half *__restrict__ cs, const __half *__restrict__ sn,
                                              float eps) {
    norm_rope_128(x0, x1, __half2float(nw[lane]), __half2float(nw[lane + 64]), __half2float(cs[lane]),
                  __half2float(sn[lane]), eps);
}

}  // namespace imh_qk
