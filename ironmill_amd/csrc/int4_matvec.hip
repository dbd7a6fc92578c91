// int4_matvec.hip -- INT4-affine (group 128) decode matvec family for gfx950.
//
// Semantics (dequantize-then-compute, core/dequant.rs:85-180 + the f32 dot of
// the reference kernels, affine_batched.metal:51-90):
//     y[m][r] = sum_k xe[m][k] * (q[r][k] - z[r][g]) * s[r][g],  g = k / 128
// where xe = x / awq (affine_batched.metal:70-79) or, for the fused residual
// norm, xe = (a + b) * gamma / awq and the epilogue multiplies by rms_inv
// (superblock_fused_norm.metal:37-124).
//
// MI355X design:
//  * the contraction runs on the matrix cores (v_mfma_f32_16x16x32_f16), with
//    each group split as
//        y_g = s * (sum_k xe_k q_k - z * sum_k xe_k)
//    so the raw codes enter the MFMA with no per-element zero-point work.  A
//    code byte in the low byte of an f16 whose high byte is zero is the f16
//    denormal byte * 2^-24, exactly, and the matrix cores multiply f16
//    denormals at full precision.  For the 8 codes n0..n7 of one weight dword
//    (byte i = n_2i + 16 n_2i+1) two v_perm_b32 spread the bytes into f16 lanes
//    and two masks keep 16 n_2i+1, giving the B operand
//        {b0, b1, b2, b3, 16 n1, 16 n3, 16 n5, 16 n7} * 2^-24;
//    the activation operand
//        {x0, x2, x4, x6, x1/16 - x0, x3/16 - x2, x5/16 - x4, x7/16 - x6}
//    makes the products sum to x0 n0 + x1 n1 + ... + x7 n7: 4 VALU per 8
//    weights, every product exact, f32 accumulation.
//  * the activation operand values are split into f16 hi + lo halves
//    (~22-bit operands).  In an MFMA tile, A rows 0-7 carry the hi halves of 8
//    batch rows and rows 8-15 their lo halves: one MFMA covers both, and the
//    two halves of a row are added at the end.
//  * the activation image carries the per-group sums of the operand values
//    (hi and lo apart, prescaled by 2^-24); the zero-point correction is two
//    FMAs per output per group.
//  * one workgroup owns one 16-row tile (of each matrix of a gate/up pair);
//    its waves split K, each holding its slice's weights in registers (one
//    16-byte load per lane per group, issued up front), and reduce through
//    LDS in a fixed order: deterministic, no cross-workgroup synchronisation.
//  * activation, scales/zeros and group sums are staged into LDS by the whole
//    workgroup, their loads issued before the weight loads and followed by an
//    LDS-only barrier, so the weights stay in flight while the first groups
//    compute.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <string>

#include "imh_internal.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGS = 128;         // group size the kernels are built for
constexpr int kMaxGroups = 8;    // groups one wave holds per stage (weights stay in registers)
constexpr int kMaxWaves = 16;    // waves per workgroup
constexpr int kSZChunks = 2;     // scale/zero elements per thread loaded ahead of the weights
constexpr int kSXChunks = 2;     // group-sum elements per thread loaded ahead of the weights
constexpr int kLdsBudget = 64 * 1024;
constexpr float kTwoM24 = 5.9604644775390625e-08f;  // 2^-24
constexpr float kTwo24 = 16777216.0f;               // 2^24

enum Epi : int { EPI_STORE = IMH_EPI_STORE, EPI_SILU = IMH_EPI_SILU, EPI_GELU = IMH_EPI_GELU };

struct MatPtrs {
    const uint8_t *data[2];
    const __half *scales[2];
    const __half *zeros[2];
    __half *out[2];
};

// Split v into f16 hi + lo with hi + lo == v to ~22 bits.
__device__ __forceinline__ void split_hilo(float v, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// Operand image of one 8-element chunk v[0..7] of xe (natural order): slots
// {v0, v2, v4, v6, v1/16 - v0, v3/16 - v2, v5/16 - v4, v7/16 - v6}, split into
// hi/lo halves.  sh / sl get the chunk's share of the group sums: the codes
// q == z everywhere give sum_i a_i (z + 16 z) + c_i (16 z), so the sum that the
// zero point multiplies is sum_i 17 a_i + 16 c_i, per half.
__device__ __forceinline__ void chunk_operands(const float v[8], half8_t &hi, half8_t &lo, float &sh,
                                               float &sl) {
    sh = 0.0f;
    sl = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = v[2 * i];
        const float c = v[2 * i + 1] * 0.0625f - a;
        _Float16 ah, al, ch, cl;
        split_hilo(a, ah, al);
        split_hilo(c, ch, cl);
        hi[i] = ah;
        lo[i] = al;
        hi[4 + i] = ch;
        lo[4 + i] = cl;
        sh += 17.0f * (float)ah + 16.0f * (float)ch;
        sl += 17.0f * (float)al + 16.0f * (float)cl;
    }
}

// Sum over the 16 lanes of a group (16 consecutive lanes, fixed order) and
// store the group sums (prescaled by 2^-24) from the group's first lane.
__device__ __forceinline__ void store_group_sums(float sh, float sl, bool live, float *gs_row, int G,
                                                 int g) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
        sh += __shfl_xor(sh, o, 16);
        sl += __shfl_xor(sl, o, 16);
    }
    if (live && (threadIdx.x & 15) == 0) {
        gs_row[g] = sh * kTwoM24;
        gs_row[G + g] = sl * kTwoM24;
    }
}

// ---------------------------------------------------------------------------
// prep: activation -> MFMA operand image
// ---------------------------------------------------------------------------
// Plain mode.  grid (ceil(K/8/256), B), block 256; thread = one 8-element
// chunk; the 16 chunks of a group are 16 consecutive lanes (K % 128 == 0).
__global__ void __launch_bounds__(256) int4_prep_plain(const __half *__restrict__ x,
                                                        const __half *__restrict__ awq,
                                                        _Float16 *__restrict__ xa_hi,
                                                        _Float16 *__restrict__ xa_lo,
                                                        float *__restrict__ gsum, int K) {
    const int m = blockIdx.y;
    const int c_raw = blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = c_raw * 8 < K;
    const int c = live ? c_raw : 0;
    const int G = K / kGS;
    const size_t base = (size_t)m * K + (size_t)c * 8;
    uint4 xv = *reinterpret_cast<const uint4 *>(x + base);
    const _Float16 *xh = reinterpret_cast<const _Float16 *>(&xv);
    float v[8];
    if (awq) {
        uint4 av = *reinterpret_cast<const uint4 *>(awq + (size_t)c * 8);
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&av);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (float)xh[i] / (float)ah[i];
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (float)xh[i];
    }
    half8_t hi, lo;
    float sh, sl;
    chunk_operands(v, hi, lo, sh, sl);
    if (live) {
        *reinterpret_cast<half8_t *>(xa_hi + base) = hi;
        *reinterpret_cast<half8_t *>(xa_lo + base) = lo;
    }
    store_group_sums(sh, sl, live, gsum + (size_t)m * 2 * G, G, c / 16);
}

// Residual + RMSNorm mode.  grid (B), block 256: r = a + b, rms_inv, writes
// residual_out / normed_out and the operand image of r * gamma / awq.
__global__ void __launch_bounds__(256) int4_prep_resnorm(
    const __half *__restrict__ a, const __half *__restrict__ b, const __half *__restrict__ gamma,
    const __half *__restrict__ awq, float eps, __half *__restrict__ residual_out,
    __half *__restrict__ normed_out, _Float16 *__restrict__ xa_hi, _Float16 *__restrict__ xa_lo,
    float *__restrict__ gsum, float *__restrict__ rms_out, int K) {
    const int m = blockIdx.x;
    const int G = K / kGS;
    const size_t row = (size_t)m * K;
    __shared__ float red[256];
    float sq = 0.0f;
    for (int c = threadIdx.x; c * 8 < K; c += blockDim.x) {
        uint4 av = *reinterpret_cast<const uint4 *>(a + row + (size_t)c * 8);
        uint4 bv = *reinterpret_cast<const uint4 *>(b + row + (size_t)c * 8);
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&av);
        const _Float16 *bh = reinterpret_cast<const _Float16 *>(&bv);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float r = (float)ah[i] + (float)bh[i];
            sq = __builtin_fmaf(r, r, sq);
        }
    }
    red[threadIdx.x] = sq;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    const float rms_inv = 1.0f / __builtin_sqrtf(red[0] / (float)K + eps);
    if (threadIdx.x == 0) rms_out[m] = rms_inv;
    // every thread runs the same number of iterations (K / 8 is a multiple of
    // 16), so the 16 lanes of a group always meet in store_group_sums
    const int iters = (K / 8 + blockDim.x - 1) / blockDim.x;
    for (int it = 0; it < iters; it++) {
        const int c_raw = it * blockDim.x + threadIdx.x;
        const bool live = c_raw * 8 < K;
        const int c = live ? c_raw : 0;
        const size_t off = row + (size_t)c * 8;
        uint4 av = *reinterpret_cast<const uint4 *>(a + off);
        uint4 bv = *reinterpret_cast<const uint4 *>(b + off);
        uint4 gv = *reinterpret_cast<const uint4 *>(gamma + (size_t)c * 8);
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&av);
        const _Float16 *bh = reinterpret_cast<const _Float16 *>(&bv);
        const _Float16 *gh = reinterpret_cast<const _Float16 *>(&gv);
        float v[8];
        half8_t res, nrm;
        for (int i = 0; i < 8; i++) {
            float r = (float)ah[i] + (float)bh[i];
            res[i] = (_Float16)r;
            nrm[i] = (_Float16)(r * rms_inv * (float)gh[i]);
            v[i] = r * (float)gh[i];
        }
        if (awq) {
            uint4 wv = *reinterpret_cast<const uint4 *>(awq + (size_t)c * 8);
            const _Float16 *wh = reinterpret_cast<const _Float16 *>(&wv);
            for (int i = 0; i < 8; i++) v[i] = v[i] / (float)wh[i];
        }
        half8_t hi, lo;
        float sh, sl;
        chunk_operands(v, hi, lo, sh, sl);
        if (live) {
            *reinterpret_cast<half8_t *>(residual_out + off) = res;
            *reinterpret_cast<half8_t *>(normed_out + off) = nrm;
            *reinterpret_cast<half8_t *>(xa_hi + off) = hi;
            *reinterpret_cast<half8_t *>(xa_lo + off) = lo;
        }
        store_group_sums(sh, sl, live, gsum + (size_t)m * 2 * G, G, c / 16);
    }
}

// ---------------------------------------------------------------------------
// main matvec kernel
// ---------------------------------------------------------------------------
// grid (ceil(N/16), ceil(B/16)), block 64 * NMAT * parts.  The workgroup's
// batch rows (up to 16) form MT MFMA tiles of 8 rows.  Wave w works on matrix
// w / parts and, in every K stage, on part w % parts of the stage's groups (at
// most NG of them).  A stage is the range of groups whose activation image
// fits the LDS budget (normally all of K: one stage).  XC activation chunks
// per thread are loaded ahead of the weights (the rest, if any, after them).
//
// Issue order matters: vector-memory loads of a wave complete in order, so
// the small loads the LDS staging needs are issued first and the weight loads
// right after them, before anything waits.  The first stage is peeled so no
// loop-carried wait sits ahead of the first weight loads.
template <int NMAT, int EPI, int MT, int NG, int XC>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu((NG <= 5 && (MT == 1 || XC == 1)) ? 6 : 5)))
int4_matvec_kernel(MatPtrs mp, const _Float16 *__restrict__ xa_hi, const _Float16 *__restrict__ xa_lo,
                   const float *__restrict__ gsum, const float *__restrict__ row_scale, int N, int K,
                   int B, int parts, int SG) {
    // dynamic LDS: [NMAT][G][16] u32 (scale | zero << 16); [G][MT][16] f32
    // group sums per A row; then one region holding the activation planes
    // ([2][bc][SG*128 + 8] f16: hi rows, then lo rows) during the stages and
    // the [MT][waves][64] float4 partial sums after them
    extern __shared__ __attribute__((aligned(16))) uint32_t lds_dyn[];

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int waves = nthr >> 6;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int mat = wave / parts;
    const int part = wave - mat * parts;
    const int G = K / kGS;
    const int m0 = blockIdx.y * 16;
    const int bc = min(16, B - m0);
    const int RSX = SG * kGS + 8;        // LDS row stride in halfs (16-byte pad)

    const int n_l = lane & 15;           // weight row within the tile (B column) and A row
    const int kq = lane >> 4;            // 16-byte quarter of a group this lane reads
    const int row0 = blockIdx.x * 16;
    const int row = row0 + n_l;
    const int row_c = row < N ? row : N - 1;

    // matrix pointers by select: a dynamic index into the kernel-argument
    // struct would turn into dependent memory loads
    const uint8_t *wdata = (NMAT == 2 && mat) ? mp.data[1] : mp.data[0];
    const uint8_t *wrow = wdata + (size_t)row_c * (K / 2) + kq * 16;

    uint32_t *szs = lds_dyn;
    float *sxs = reinterpret_cast<float *>(lds_dyn + NMAT * G * 16);
    _Float16 *xs = reinterpret_cast<_Float16 *>(sxs + G * MT * 16);
    float4_t *red = reinterpret_cast<float4_t *>(xs);

    // scales/zeros of the tile: per matrix one contiguous run of 16 * G halfs
    // from row0 * G (elements past the last row clamp to it; their rows are
    // never stored); LDS slot [mat][g][row]
    const int per_mat = 16 * G;
    const int sz_total = NMAT * per_mat;
    const size_t sz_last = (size_t)N * G - 1;
    auto sz_elem = [&](int e, const uint16_t *&sp, const uint16_t *&zp, int &dst) {
        const bool second = NMAT == 2 && e >= per_mat;
        const int el = second ? e - per_mat : e;
        sp = reinterpret_cast<const uint16_t *>(second ? mp.scales[1] : mp.scales[0]);
        zp = reinterpret_cast<const uint16_t *>(second ? mp.zeros[1] : mp.zeros[0]);
        const int rr = el / G;
        dst = ((second ? G : 0) + (el - rr * G)) * 16 + rr;
        return min((size_t)row0 * G + el, sz_last);
    };
    // group sums: LDS slot e = (g * MT + t) * 16 + a holds A row a of tile t:
    // the hi (a < 8) or lo (a >= 8) sum of batch row 8t + (a & 7), rows past
    // the batch reusing row 0
    const int sx_total = G * MT * 16;
    auto sx_src = [&](int e) {
        const int a = e & 15;
        const int gt = e >> 4;
        const int g = gt / MT;
        const int t = gt - g * MT;
        const int r = 8 * t + (a & 7);
        const int rc = r < bc ? r : 0;
        return (size_t)(m0 + rc) * 2 * G + (a >> 3) * G + g;
    };
    uint32_t sv[kSZChunks], zv[kSZChunks];
    int sd[kSZChunks];
#pragma unroll
    for (int i = 0; i < kSZChunks; i++) {
        const uint16_t *sp, *zp;
        const size_t src = sz_elem(min(i * nthr + tid, sz_total - 1), sp, zp, sd[i]);
        sv[i] = sp[src];
        zv[i] = zp[src];
    }
    float xsum[kSXChunks];
#pragma unroll
    for (int i = 0; i < kSXChunks; i++) xsum[i] = gsum[sx_src(min(i * nthr + tid, sx_total - 1))];

    // A rows of this lane in each tile: plane n_l >> 3, batch row 8t + (n_l & 7)
    int arow[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int r = 8 * t + (n_l & 7);
        arow[t] = (n_l >> 3) * bc + (r < bc ? r : 0);
    }

    float4_t acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};

    auto stage = [&](const int gs0, const bool first) __attribute__((always_inline)) {
        const int SGs = min(SG, G - gs0);
        // (a) activation loads of this stage
        const int cpr = SGs * 16;                  // 8-half chunks per batch row
        const int total = bc * cpr;
        u32x4_t xv[XC], lv[XC];
#pragma unroll
        for (int i = 0; i < XC; i++) {
            const int c = min(i * nthr + tid, total - 1);
            const int r = c / cpr;
            const size_t src = (size_t)(m0 + r) * K + (size_t)gs0 * kGS + (size_t)(c - r * cpr) * 8;
            xv[i] = *reinterpret_cast<const u32x4_t *>(xa_hi + src);
            lv[i] = *reinterpret_cast<const u32x4_t *>(xa_lo + src);
        }
        // (b) this wave's weights for the stage: unconditional, clamped loads
        const int wg0 = gs0 + (part * SGs) / parts;
        const int ng = gs0 + ((part + 1) * SGs) / parts - wg0;
        u32x4_t wq[NG];
#pragma unroll
        for (int i = 0; i < NG; i++) {
            const int g = min(max(wg0 + min(i, ng - 1), 0), G - 1);
            wq[i] = *reinterpret_cast<const u32x4_t *>(wrow + (size_t)g * 64);
        }
        // (c) scales/zeros and group sums -> LDS (first stage only).  The
        // writes are unconditional -- threads past the end rewrite the last
        // element with its own value -- so the compiler has no branch to sink
        // the loads into behind a wait for the weights.
        if (first) {
#pragma unroll
            for (int i = 0; i < kSZChunks; i++) szs[sd[i]] = sv[i] | (zv[i] << 16);
            for (int e = kSZChunks * nthr + tid; e < sz_total; e += nthr) {
                const uint16_t *sp, *zp;
                int dst;
                const size_t src = sz_elem(e, sp, zp, dst);
                szs[dst] = (uint32_t)sp[src] | ((uint32_t)zp[src] << 16);
            }
#pragma unroll
            for (int i = 0; i < kSXChunks; i++) sxs[min(i * nthr + tid, sx_total - 1)] = xsum[i];
            for (int e = kSXChunks * nthr + tid; e < sx_total; e += nthr) sxs[e] = gsum[sx_src(e)];
        } else {
            // the previous stage is done with the activation planes
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        }
        // (d) activation -> LDS (plane 0 rows 0..bc-1, plane 1 rows bc..2bc-1)
#pragma unroll
        for (int i = 0; i < XC; i++) {
            const int c = min(i * nthr + tid, total - 1);
            const int r = c / cpr;
            const int off = r * RSX + (c - r * cpr) * 8;
            *reinterpret_cast<u32x4_t *>(xs + off) = xv[i];
            *reinterpret_cast<u32x4_t *>(xs + bc * RSX + off) = lv[i];
        }
        for (int c = XC * nthr + tid; c < total; c += nthr) {  // activation beyond XC chunks
            const int r = c / cpr;
            const size_t src = (size_t)(m0 + r) * K + (size_t)gs0 * kGS + (size_t)(c - r * cpr) * 8;
            const int off = r * RSX + (c - r * cpr) * 8;
            *reinterpret_cast<u32x4_t *>(xs + off) = *reinterpret_cast<const u32x4_t *>(xa_hi + src);
            *reinterpret_cast<u32x4_t *>(xs + bc * RSX + off) = *reinterpret_cast<const u32x4_t *>(xa_lo + src);
        }
        // LDS-only barrier: the weight loads stay in flight across it
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

        // (e) MFMA over the wave's groups
#pragma unroll
        for (int i = 0; i < NG; i++) {
            if (i < ng) {
                const int g = wg0 + i;
                const uint32_t sz = szs[(mat * G + g) * 16 + n_l];
                const float s24 = (float)__builtin_bit_cast(_Float16, (uint16_t)(sz & 0xFFFFu)) * kTwo24;
                const float z = (float)__builtin_bit_cast(_Float16, (uint16_t)(sz >> 16));
                u32x4_t bq[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t w = wq[i][j];
                    const uint32_t p0 = __builtin_amdgcn_perm(w, 0u, 0x0C050C04u);  // b0, b1
                    const uint32_t p1 = __builtin_amdgcn_perm(w, 0u, 0x0C070C06u);  // b2, b3
                    bq[j] = (u32x4_t){p0, p1, p0 & 0x00F000F0u, p1 & 0x00F000F0u};
                }
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const _Float16 *xa = xs + arow[t] * RSX + (g - gs0) * kGS + kq * 32;
                    float4_t accg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const half8_t av = *reinterpret_cast<const half8_t *>(xa + j * 8);
                        accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            av, __builtin_bit_cast(half8_t, bq[j]), accg, 0, 0, 0);
                    }
                    // D rows 4*kq + r of tile t
                    const float4_t sx = *reinterpret_cast<const float4_t *>(sxs + (g * MT + t) * 16 + 4 * kq);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc[t][r] = __builtin_fmaf(s24, __builtin_fmaf(-z, sx[r], accg[r]), acc[t][r]);
                }
            }
        }
    };
    stage(0, true);
    for (int gs0 = SG; gs0 < G; gs0 += SG) stage(gs0, false);

    // reduce: the partial-sum region overlays the activation planes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
    for (int t = 0; t < MT; t++) red[(t * waves + wave) * 64 + lane] = acc[t];
    __syncthreads();
    if (wave != 0) return;
    // wave 0: lanes 32t..32t+31 finish tile t.  Lane l of a tile holds D rows
    // 4*(l>>4) + r, r < 4; rows < 8 are hi halves, row + 8 (lane l + 32) the lo
    // halves of the same batch rows.  Parts are summed in part order.
    const int t = lane >> 5;
    if (t >= MT) return;
    const int l2 = lane & 31;
    float4_t sum[NMAT];
#pragma unroll
    for (int mt = 0; mt < NMAT; mt++) {
        const float4_t *rp = red + (t * waves + mt * parts) * 64;
        sum[mt] = rp[l2] + rp[l2 + 32];
        for (int p = 1; p < parts; p++) sum[mt] += rp[p * 64 + l2] + rp[p * 64 + l2 + 32];
    }
    if (row >= N) return;
    const int mrow = m0 + 8 * t + 4 * (l2 >> 4);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = mrow + r;
        if (m >= B) break;
        const float scale = row_scale ? row_scale[m] : 1.0f;
        if (EPI == EPI_SILU || EPI == EPI_GELU) {
            const float g = sum[0][r], u = sum[NMAT - 1][r];
            float act;
            if (EPI == EPI_SILU) {
                act = g / (1.0f + __expf(-g));
            } else {
                float inner = 0.7978845608f * (g + 0.044715f * g * g * g);
                inner = fminf(fmaxf(inner, -10.0f), 10.0f);
                act = 0.5f * g * (1.0f + tanhf(inner));
            }
            mp.out[0][(size_t)m * N + row] = __float2half(act * u * scale);
        } else {
#pragma unroll
            for (int mt = 0; mt < NMAT; mt++)
                mp.out[mt][(size_t)m * N + row] = __float2half(sum[mt][r] * scale);
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

int check_weight(const imh_affine_int4_weight *w, const char *who) {
    if (!w || !w->data || !w->scales || !w->zeros)
        return imh::fail(IMH_EINVAL, std::string(who) + ": weight or one of its arrays is NULL");
    if (w->group_size != kGS)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": group_size " +
                                               std::to_string(w->group_size) +
                                               " not supported (built for 128)");
    if (w->n == 0 || w->k == 0 || w->k % kGS != 0)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": k=" + std::to_string(w->k) +
                                               " must be a non-zero multiple of 128, n=" +
                                               std::to_string(w->n) + " non-zero");
    if ((reinterpret_cast<uintptr_t>(w->data) & 15) != 0)
        return imh::fail(IMH_EINVAL, std::string(who) + ": weight data must be 16-byte aligned");
    return IMH_OK;
}

bool misaligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

// image layout in caller storage: hi [B][K] f16, lo [B][K] f16, group sums
// [B][2][K/128] f32, row scales [B] f32
size_t act_bytes(uint32_t B, uint32_t K) {
    return (size_t)B * K * 4 + (size_t)B * 2 * (K / kGS) * 4 + (size_t)B * 4 + 256;
}

void act_layout(void *storage, uint32_t B, uint32_t K, imh_int4_activation *act, float **rms) {
    _Float16 *hi = static_cast<_Float16 *>(storage);
    _Float16 *lo = hi + (size_t)B * K;
    float *gs = reinterpret_cast<float *>(lo + (size_t)B * K);
    *rms = gs + (size_t)B * 2 * (K / kGS);
    act->hi = reinterpret_cast<const uint16_t *>(hi);
    act->lo = reinterpret_cast<const uint16_t *>(lo);
    act->group_sums = gs;
    act->row_scale = nullptr;
    act->token_count = B;
    act->k = K;
}

// Waves per tile.  Each wave holds at most kMaxGroups groups per stage, and
// the whole grid should be resident at once -- one round of workgroups, so
// every weight load is in flight together.  The kernels run 6 waves per SIMD
// (24 per CU); within that, ~6 waves per SIMD in total is enough to cover
// HBM latency.
int pick_parts(int tiles, int nmat, int G, int cus) {
    const int need = (G + kMaxGroups - 1) / kMaxGroups;
    const int per_cu = (tiles + cus - 1) / cus;              // workgroups each CU must hold
    const int resident = 24 / per_cu / nmat;
    const int total = 6 * 4 * cus / std::max(1, tiles * nmat);
    const int cap = std::min(kMaxWaves / nmat, G);
    return std::max(1, std::min(cap, std::max(need, std::min(resident, total))));
}

int prep_plain(imh_stream *s, const uint16_t *x, uint32_t B, uint32_t K, const uint16_t *awq,
               void *storage, imh_int4_activation *act) {
    if (misaligned16(x) || misaligned16(awq) || misaligned16(storage))
        return imh::fail(IMH_EINVAL, "int4 activation: x, awq and storage must be 16-byte aligned");
    float *rms;
    act_layout(storage, B, K, act, &rms);
    dim3 grid((K / 8 + 255) / 256, B);
    hipLaunchKernelGGL(int4_prep_plain, grid, dim3(256), 0, s->stream,
                       reinterpret_cast<const __half *>(x), reinterpret_cast<const __half *>(awq),
                       const_cast<_Float16 *>(reinterpret_cast<const _Float16 *>(act->hi)),
                       const_cast<_Float16 *>(reinterpret_cast<const _Float16 *>(act->lo)),
                       const_cast<float *>(act->group_sums), (int)K);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

template <int NMAT, int EPI, int MT, int NG>
void launch_xc(bool one_chunk, dim3 grid, dim3 block, size_t lds, hipStream_t st, const MatPtrs &mp,
               const imh_int4_activation *act, int N, int K, int B, int parts, int SG) {
    const _Float16 *hi = reinterpret_cast<const _Float16 *>(act->hi);
    const _Float16 *lo = reinterpret_cast<const _Float16 *>(act->lo);
    if (one_chunk)
        hipLaunchKernelGGL((int4_matvec_kernel<NMAT, EPI, MT, NG, 1>), grid, block, lds, st, mp, hi, lo,
                           act->group_sums, act->row_scale, N, K, B, parts, SG);
    else
        hipLaunchKernelGGL((int4_matvec_kernel<NMAT, EPI, MT, NG, 2>), grid, block, lds, st, mp, hi, lo,
                           act->group_sums, act->row_scale, N, K, B, parts, SG);
}

template <int NMAT, int EPI, int MT>
void launch_ng(int ng, bool one_chunk, dim3 grid, dim3 block, size_t lds, hipStream_t st,
               const MatPtrs &mp, const imh_int4_activation *act, int N, int K, int B, int parts, int SG) {
    if (ng <= 2) launch_xc<NMAT, EPI, MT, 2>(one_chunk, grid, block, lds, st, mp, act, N, K, B, parts, SG);
    else if (ng <= 3) launch_xc<NMAT, EPI, MT, 3>(one_chunk, grid, block, lds, st, mp, act, N, K, B, parts, SG);
    else if (ng <= 4) launch_xc<NMAT, EPI, MT, 4>(one_chunk, grid, block, lds, st, mp, act, N, K, B, parts, SG);
    else if (ng <= 5) launch_xc<NMAT, EPI, MT, 5>(one_chunk, grid, block, lds, st, mp, act, N, K, B, parts, SG);
    else if (ng <= 6) launch_xc<NMAT, EPI, MT, 6>(one_chunk, grid, block, lds, st, mp, act, N, K, B, parts, SG);
    else launch_xc<NMAT, EPI, MT, 8>(one_chunk, grid, block, lds, st, mp, act, N, K, B, parts, SG);
}

template <int NMAT, int EPI>
int launch_main(imh_stream *s, const MatPtrs &mp, const imh_int4_activation *act, int N, const char *who) {
    const int K = (int)act->k, B = (int)act->token_count;
    const int G = K / kGS;
    const int rows = std::min(B, 16);
    const int MT = rows > 8 ? 2 : 1;
    const int tiles = (N + 15) / 16;
    const int btiles = (B + 15) / 16;
    const int parts = pick_parts(tiles * btiles, NMAT, G, s->dev->props.multiProcessorCount);
    const int waves = NMAT * parts;
    // LDS: scales/zeros + group sums, then max(activation planes, partial sums)
    const size_t fixed = (size_t)NMAT * G * 16 * 4 + (size_t)G * MT * 16 * 4;
    const size_t red_bytes = (size_t)MT * waves * 64 * sizeof(float4_t);
    const size_t per_group = (size_t)2 * rows * kGS * sizeof(_Float16);
    const size_t pad = (size_t)2 * rows * 8 * sizeof(_Float16);
    if (fixed + pad + per_group > (size_t)kLdsBudget || fixed + red_bytes > (size_t)kLdsBudget)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": k=" + std::to_string(K) +
                                               " too large for the LDS staging of this kernel");
    int SG = (int)((kLdsBudget - fixed - pad) / per_group);
    SG = std::min(std::min(SG, parts * kMaxGroups), G);
    const int ng = (SG + parts - 1) / parts;  // most groups a wave takes in one stage
    const size_t lds = fixed + std::max(pad + (size_t)SG * per_group, red_bytes);
    const bool one_chunk = rows * SG * 16 <= 64 * waves;
    dim3 grid(tiles, btiles), block(64 * waves);
    if (MT == 1)
        launch_ng<NMAT, EPI, 1>(ng, one_chunk, grid, block, lds, s->stream, mp, act, N, K, B, parts, SG);
    else
        launch_ng<NMAT, EPI, 2>(ng, one_chunk, grid, block, lds, s->stream, mp, act, N, K, B, parts, SG);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

int run_matvec(imh_stream *s, const imh_int4_activation *act, const imh_affine_int4_weight *w0,
               const imh_affine_int4_weight *w1, int epi, uint16_t *out0, uint16_t *out1,
               const char *who) {
    int rc = check_weight(w0, who);
    if (rc) return rc;
    if (w1) {
        rc = check_weight(w1, who);
        if (rc) return rc;
        if (w1->n != w0->n || w1->k != w0->k)  // D7: the reference assumes N_up == N_gate
            return imh::fail(IMH_EINVAL, std::string(who) + ": gate and up shapes differ");
    }
    if (!act || !act->hi || !act->lo || !act->group_sums || !out0 || (w1 && epi == EPI_STORE && !out1))
        return imh::fail(IMH_EINVAL, std::string(who) + ": NULL activation array or output");
    if (act->k != w0->k)
        return imh::fail(IMH_EINVAL, std::string(who) + ": activation k differs from the weight's");
    if (epi != EPI_STORE && epi != EPI_SILU && epi != EPI_GELU)
        return imh::fail(IMH_EINVAL, std::string(who) + ": unknown epilogue");
    if (epi != EPI_STORE && !w1)
        return imh::fail(IMH_EINVAL, std::string(who) + ": activation epilogues need a gate/up pair");
    if (misaligned16(act->hi) || misaligned16(act->lo))
        return imh::fail(IMH_EINVAL, std::string(who) + ": activation image must be 16-byte aligned");
    if (act->token_count == 0) return IMH_OK;
    rc = imh::use_device(s->dev);
    if (rc) return rc;
    MatPtrs mp = {};
    const imh_affine_int4_weight *ws[2] = {w0, w1};
    for (int i = 0; i < (w1 ? 2 : 1); i++) {
        mp.data[i] = ws[i]->data;
        mp.scales[i] = reinterpret_cast<const __half *>(ws[i]->scales);
        mp.zeros[i] = reinterpret_cast<const __half *>(ws[i]->zeros);
    }
    mp.out[0] = reinterpret_cast<__half *>(out0);
    mp.out[1] = reinterpret_cast<__half *>(out1);
    const int N = (int)w0->n;
    if (!w1) return launch_main<1, EPI_STORE>(s, mp, act, N, who);
    if (epi == EPI_SILU) return launch_main<2, EPI_SILU>(s, mp, act, N, who);
    if (epi == EPI_GELU) return launch_main<2, EPI_GELU>(s, mp, act, N, who);
    return launch_main<2, EPI_STORE>(s, mp, act, N, who);
}

// prep into the stream's scratch, then the matvec
int plain_op(imh_stream *s, const uint16_t *x, uint32_t B, const imh_affine_int4_weight *w0,
             const imh_affine_int4_weight *w1, int epi, uint16_t *out0, uint16_t *out1,
             const char *who) {
    if (!s || !x) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_weight(w0, who);
    if (rc) return rc;
    if (B == 0) return IMH_OK;
    rc = imh::use_device(s->dev);
    if (rc) return rc;
    void *scr = nullptr;
    rc = imh::stream_scratch(s, 0, act_bytes(B, w0->k), &scr);
    if (rc) return rc;
    imh_int4_activation act;
    rc = prep_plain(s, x, B, w0->k, w0->awq_scales, scr, &act);
    if (rc) return rc;
    return run_matvec(s, &act, w0, w1, epi, out0, out1, who);
}

}  // namespace

extern "C" {

size_t imh_int4_activation_bytes(uint32_t token_count, uint32_t k) { return act_bytes(token_count, k); }

int imh_encode_int4_activation(imh_stream *stream, const uint16_t *x, uint32_t token_count, uint32_t k,
                               const uint16_t *awq, void *storage, imh_int4_activation *out) {
    const char *who = "imh_encode_int4_activation";
    if (!stream || !x || !storage || !out) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    if (k == 0 || k % kGS != 0)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": k must be a non-zero multiple of 128");
    float *rms;
    act_layout(storage, token_count, k, out, &rms);
    if (token_count == 0) return IMH_OK;
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    return prep_plain(stream, x, token_count, k, awq, storage, out);
}

int imh_encode_int4_matvec_prepared(imh_stream *stream, const imh_int4_activation *act,
                                    const imh_affine_int4_weight *w0, const imh_affine_int4_weight *w1,
                                    int epilogue, uint16_t *out0, uint16_t *out1) {
    if (!stream) return imh::fail(IMH_EINVAL, "imh_encode_int4_matvec_prepared: NULL stream");
    return run_matvec(stream, act, w0, w1, epilogue, out0, out1, "imh_encode_int4_matvec_prepared");
}

int imh_encode_affine_projection_int4(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                      const imh_affine_int4_weight *w, uint16_t *y) {
    return plain_op(stream, x, token_count, w, nullptr, EPI_STORE, y, nullptr,
                    "imh_encode_affine_projection_int4");
}

int imh_encode_batched_affine_matvec_int4(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                          const imh_affine_int4_weight *gate, uint16_t *gate_out,
                                          const imh_affine_int4_weight *up, uint16_t *up_out) {
    const char *who = "imh_encode_batched_affine_matvec_int4";
    if (!gate_out || !up_out || !up) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    return plain_op(stream, x, token_count, gate, up, EPI_STORE, gate_out, up_out, who);
}

int imh_encode_fused_ffn_gate_up_act_int4(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                          const imh_affine_int4_weight *gate,
                                          const imh_affine_int4_weight *up, uint16_t *out,
                                          int use_gelu) {
    const char *who = "imh_encode_fused_ffn_gate_up_act_int4";
    if (!out || !up) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    return plain_op(stream, x, token_count, gate, up, use_gelu ? EPI_GELU : EPI_SILU, out, nullptr, who);
}

int imh_encode_fused_residual_norm_affine_matvec_int4(imh_stream *stream,
                                                      const imh_fused_residual_norm_params *p) {
    const char *who = "imh_encode_fused_residual_norm_affine_matvec_int4";
    if (!stream || !p || !p->a || !p->b || !p->norm_weight || !p->residual_output || !p->output ||
        !p->normed_output)
        return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_weight(p->weight, who);
    if (rc) return rc;
    if (p->token_count == 0) return IMH_OK;
    if (misaligned16(p->a) || misaligned16(p->b) || misaligned16(p->norm_weight) ||
        misaligned16(p->residual_output) || misaligned16(p->normed_output) ||
        misaligned16(p->weight->awq_scales))
        return imh::fail(IMH_EINVAL, std::string(who) + ": vectors must be 16-byte aligned");
    rc = imh::use_device(stream->dev);
    if (rc) return rc;
    const uint32_t B = p->token_count, K = p->weight->k;
    void *scr = nullptr;
    rc = imh::stream_scratch(stream, 0, act_bytes(B, K), &scr);
    if (rc) return rc;
    imh_int4_activation act;
    float *rms;
    act_layout(scr, B, K, &act, &rms);
    hipLaunchKernelGGL(int4_prep_resnorm, dim3(B), dim3(256), 0, stream->stream,
                       reinterpret_cast<const __half *>(p->a), reinterpret_cast<const __half *>(p->b),
                       reinterpret_cast<const __half *>(p->norm_weight),
                       reinterpret_cast<const __half *>(p->weight->awq_scales), p->eps,
                       reinterpret_cast<__half *>(p->residual_output),
                       reinterpret_cast<__half *>(p->normed_output),
                       const_cast<_Float16 *>(reinterpret_cast<const _Float16 *>(act.hi)),
                       const_cast<_Float16 *>(reinterpret_cast<const _Float16 *>(act.lo)),
                       const_cast<float *>(act.group_sums), rms, (int)K);
    IMH_HIP(hipGetLastError());
    act.row_scale = rms;
    return run_matvec(stream, &act, p->weight, nullptr, EPI_STORE, p->output, nullptr, who);
}

}  // extern "C"
