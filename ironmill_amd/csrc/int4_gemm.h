// int4_gemm.h -- host entry points of the prefill INT4 GEMM (int4_gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "imh_internal.h"

namespace imh_int4 {

// Token counts from which the INT4 ops run the GEMM instead of the matvec.
constexpr int kGemmMinTokens = 32;

// K splits the GEMM uses for this shape (1 when the tile grid fills the GPU);
// nmat = 2 for a gate/up pair
int gemm_splits(int M, int N, int K, int nmat, int cus);
// bytes of f32 split partials encode_gemm needs (0 without a split)
size_t gemm_workspace_bytes(int M, int N, int K, int nmat, int cus);
// y0 [M][N] f16 = f16(x [M][K] / awq0) . W0^T with W0's dequantized f16
// values; with w1 (a gate/up pair sharing x and awq0): epi 0 also stores
// y1 = x . W1^T, epi 2 / 3 stores y0 = f16(silu / gelu(x . W0^T) * (x . W1^T))
// from the f32 results
int encode_gemm(imh_stream *s, const __half *x, int M, const imh_affine_int4_weight *w0,
                const imh_affine_int4_weight *w1, int epi, __half *y0, __half *y1, void *workspace);

// Sum of squares of a 256-thread workgroup's per-thread partials, in the
// order of a halving tree over red[] (t + 128, then + 64, ... + 1): wave 0
// forms the first two levels from red[], shuffles do the rest.  Two barriers
// where an LDS tree takes nine; every thread gets rms_inv.
__device__ __forceinline__ float block_rms_inv(float sq, float *red, float *bcast, int K, float eps) {
    const int t = threadIdx.x;
    red[t] = sq;
    __syncthreads();
    if (t < 64) {
        float v = (red[t] + red[t + 128]) + (red[t + 64] + red[t + 192]);
#pragma unroll
        for (int st = 32; st >= 1; st >>= 1) v += __shfl_down(v, st);
        if (t == 0) *bcast = 1.0f / __builtin_sqrtf(v / (float)K + eps);
    }
    __syncthreads();
    return *bcast;
}

// Register chunks per thread of the residual-norm row kernels (256 threads
// per row): 1, 2, 4 or 8.
inline int resnorm_cpt(int K) {
    const int c = (K / 8 + 255) / 256;
    return c <= 1 ? 1 : c <= 2 ? 2 : c <= 4 ? 4 : 8;
}

// residual_out = f16(a + b), normed_out = f16((a + b) * rms_inv * gamma) per row
int encode_resnorm_rows(imh_stream *s, const __half *a, const __half *b, const __half *gamma, float eps,
                        __half *residual_out, __half *normed_out, int B, int K);

}  // namespace imh_int4
