// int8_matvec.hip -- the INT8 "sensitive-layer" weight matvec and the
// INT4 x Q8 decode variant:
//
//  * INT8 weights (superblock_matvec_int8, affine_matvec.metal:123-189, over
//    quantize_tensor_int8, quantized.rs:852-901): codes [N][K] bytes 0..255,
//    f16 scales / zero-points per 128-group,
//        y[m][n] = f16( sum_g s * sum_{k in g} (x[m][k] / awq[k]) * (q - z) ).
//    The matrix cores multiply the raw code bytes as f16 denormals (byte *
//    2^-24, exact) against the activation split into f16 hi + lo (~22 bits);
//    zero-point and scale are applied in f32 per group to the group sums, as
//    in the INT4 matvec.
//  * INT4 x Q8 (superblock_affine_matvec_int4xq8, affine_fused.metal:115-176,
//    with quantize_input_q8, quantize.metal:21-52): the activation is first
//    quantized to int8 per 128-group (scale = absmax / 127, q = rint(x * 127 /
//    absmax) clamped to +-127), then
//        y[m][n] = f16( sum_g ws * as * sum_{k in g} q8 * (q - rint(z)) ).
//    On MI355X the group's dot product runs on the integer matrix cores
//    (v_mfma_i32_16x16x64_i8): exact in int32, sum q8 q minus z sum q8, the
//    two scales applied in f32.
//
// The tile kernels: one workgroup per 16 weight rows, waves splitting the K
// groups of each stage, the activation staged in LDS per stage (all of K when
// it fits), each wave's weights loaded into registers before the staging so
// they are in flight meanwhile; wave partials reduced through LDS in a fixed
// order (deterministic).  INT8 weights at 1-4 batch rows take the band kernel
// (int8w_band_kernel) instead, and INT4 x Q8 at 1-8 rows int4xq8_band_kernel:
// a grid of one row band per compute unit.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <string>

#include "dpp_reduce.h"
#include "imh_internal.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGS = 128;
constexpr int kMaxWaves = 8;
constexpr int kNG = 8;                    // groups one wave holds per stage
constexpr int kStageBytes = 48 * 1024;    // LDS for one stage's activation
constexpr float kTwoM24 = 5.9604644775390625e-08f;
constexpr float kTwo24 = 16777216.0f;

// ---------------------------------------------------------------------------
// INT8 weights x f16 activations
// ---------------------------------------------------------------------------
// grid (ceil(N / 16)), block 64 * waves; B <= 8 batch rows.  LDS: hi [B][SG *
// 128] f16, lo [B][SG * 128] f16, group sums [SG][16] (A rows: hi sums of the
// B rows, then lo sums, prescaled by 2^-24), then the wave partials.
__global__ void __launch_bounds__(64 * kMaxWaves) int8w_matvec_kernel(
    const __half *__restrict__ x, const __half *__restrict__ awq, const uint8_t *__restrict__ w,
    const __half *__restrict__ scales, const __half *__restrict__ zeros, __half *__restrict__ y, int N, int K, int B,
    int SG) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, waves = nthr >> 6;
    const int n_l = lane & 15, kq = lane >> 4;
    const int G = K / kGS;
    const int row0 = blockIdx.x * 16;
    const int row = row0 + n_l;
    const int row_c = min(row, N - 1);
    const int RS = SG * kGS + 8;                         // LDS row stride (halfs), 16-byte pad
    _Float16 *img = reinterpret_cast<_Float16 *>(lds8);  // hi rows, then lo rows
    float *gsx = reinterpret_cast<float *>(lds8 + (size_t)2 * B * RS * 2);
    // A row of this lane: plane n_l >> 3, batch row (n_l & 7) (rows past B reuse row 0)
    const int ab = (n_l & 7) < B ? (n_l & 7) : 0;
    const int arow = (n_l >> 3) * B + ab;

    float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < G; s0 += SG) {
        const int SGs = min(SG, G - s0);
        // (a) this wave's weights for its share of the stage's groups
        const int g0 = s0 + (wave * SGs) / waves;
        const int ng = s0 + ((wave + 1) * SGs) / waves - g0;
        u32x4_t wq[kNG][2];
#pragma unroll
        for (int i = 0; i < kNG; i++) {
            const int g = min(g0 + min(i, max(ng - 1, 0)), G - 1);
            const uint8_t *p = w + (size_t)row_c * K + (size_t)g * kGS + kq * 32;
            wq[i][0] = *reinterpret_cast<const u32x4_t *>(p);
            wq[i][1] = *reinterpret_cast<const u32x4_t *>(p + 16);
        }
        // (b) the stage's activation image: chunk c (8 elements) of batch row b
        const int cpr = SGs * 16;
        for (int c = tid; c < B * cpr + (16 - (B * cpr) % 16) % 16; c += nthr) {
            const bool live = c < B * cpr;
            const int cc = live ? c : 0;
            const int b = cc / cpr, ci = cc - b * cpr;
            const size_t k = (size_t)s0 * kGS + (size_t)ci * 8;
            const u32x4_t xv = *reinterpret_cast<const u32x4_t *>(x + (size_t)b * K + k);
            const _Float16 *xh = reinterpret_cast<const _Float16 *>(&xv);
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = (float)xh[i];
            if (awq) {
                const u32x4_t av = *reinterpret_cast<const u32x4_t *>(awq + k);
                const _Float16 *ah = reinterpret_cast<const _Float16 *>(&av);
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = v[i] * __builtin_amdgcn_rcpf((float)ah[i]);
            }
            half8_t hi, lo;
            float sh = 0.0f, sl = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                hi[i] = (_Float16)v[i];
                lo[i] = (_Float16)(v[i] - (float)hi[i]);
                sh += (float)hi[i];
                sl += (float)lo[i];
            }
            if (live) {
                *reinterpret_cast<half8_t *>(img + (size_t)b * RS + ci * 8) = hi;
                *reinterpret_cast<half8_t *>(img + (size_t)(B + b) * RS + ci * 8) = lo;
            }
            // the 16 chunks of a group are 16 consecutive lanes (cpr is a multiple of 16)
            sh = imh_dpp::row16_sum(sh);
            sl = imh_dpp::row16_sum(sl);
            if (live && (tid & 15) == 0) {
                const int g = ci / 16;
                gsx[g * 16 + b] = sh * kTwoM24;
                gsx[g * 16 + 8 + b] = sl * kTwoM24;
            }
        }
        __syncthreads();
        // (c) MFMA over the wave's groups: B = 8 code bytes of row n_l as f16
        // denormals, A = 8 operand values of A row n_l (same k: 32 kq + 8 j)
#pragma unroll
        for (int i = 0; i < kNG; i++) {
            if (i < ng) {
                const int g = g0 + i;
                const float s24 = __half2float(scales[(size_t)row_c * G + g]) * kTwo24;
                const float z = __half2float(zeros[(size_t)row_c * G + g]);
                const _Float16 *xa = img + (size_t)arow * RS + (g - s0) * kGS + kq * 32;
                float4_t accg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t w0 = wq[i][j >> 1][2 * (j & 1)], w1 = wq[i][j >> 1][2 * (j & 1) + 1];
                    const u32x4_t bq = {__builtin_amdgcn_perm(0u, w0, 0x0C010C00u), __builtin_amdgcn_perm(0u, w0, 0x0C030C02u),
                                        __builtin_amdgcn_perm(0u, w1, 0x0C010C00u), __builtin_amdgcn_perm(0u, w1, 0x0C030C02u)};
                    const half8_t av = *reinterpret_cast<const half8_t *>(xa + j * 8);
                    accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, __builtin_bit_cast(half8_t, bq), accg, 0, 0, 0);
                }
                // D rows 4 kq + r: hi rows (< 8) and lo rows share the group's sums per A row
                const float4_t sx = *reinterpret_cast<const float4_t *>(gsx + (g - s0) * 16 + 4 * kq);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(s24, __builtin_fmaf(-z, sx[r], accg[r]), acc[r]);
            }
        }
        __syncthreads();
    }
    // reduce the waves (partials overlay the image), wave 0 stores: lane l < 32
    // holds D rows 4 (l >> 4) + r (hi of batch rows), lane l + 32 the lo rows
    float4_t *red = reinterpret_cast<float4_t *>(lds8);
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave != 0 || lane >= 32 || row >= N) return;
    float4_t s = red[lane] + red[lane + 32];
    for (int wv = 1; wv < waves; wv++) s += red[wv * 64 + lane] + red[wv * 64 + lane + 32];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int b = 4 * (lane >> 4) + r;
        if (b < B) y[(size_t)b * N + row] = __float2half(s[r]);
    }
}

// ---------------------------------------------------------------------------
// INT8 weights, 1-4 batch rows, over a grid balanced on the compute units
// ---------------------------------------------------------------------------
// The tile kernel above gives each workgroup 16 rows, so the Qwen3-4B down
// shape (2560 rows) fills 160 of 256 compute units.  Here workgroup b of NWG
// owns the row band [N b / NWG, N (b+1) / NWG), cut into TM tiles of 8 rows
// (the last one masked); W waves split the K groups of every tile, each wave
// issuing all of its weight loads (TM x NPW x 16 bytes per lane) before the
// activation is staged.  Same arithmetic per group as the tile kernel (codes
// as f16 denormals, activation as f16 hi + lo, zero point on the group sums,
// f32 accumulation); the group's two 64-code halves are summed separately.
//  * B column j = r + 8h: row r of the tile, half h of the group; lane l loads
//    16 codes of row r at 64 h + 16 kq (kq = l >> 4), so a wave reads 8 rows
//    x 128 contiguous bytes.  MFMA u takes its bytes 8u .. 8u + 7.
//  * A row i = 8h + 4 plane + b: batch row b (rows past B read row 0), f16 hi
//    (plane 0) or lo (plane 1) of the activation at the same offsets.  Only
//    result entries whose row and column share h are used: lane l holds D
//    rows 4 (l >> 4) .. + 3 of column l & 15, used when (l >> 5) == ((l >> 3) & 1).
//  * LDS: image [2 B][K + 8] f16 (plane-major), half-group sums [G][16] f32
//    (entry 4 (2h + plane) + b, prescaled by 2^-24), the band's scales and zero
//    points [rows][G] f16 (coalesced loads issued with the activation's, ahead
//    of the weights); the wave partials overlay
//    the image after the last MFMA and are summed in (wave, h, plane) order.
__host__ __device__ inline size_t int8_band_img_bytes(int K, int B) { return (size_t)2 * B * (K + 8) * 2; }
constexpr int PX = 2;   // activation chunks per thread loaded ahead of the weights

template <int TM, int NPW>
__global__ void __launch_bounds__(1024) int8w_band_kernel(const __half *__restrict__ x, const __half *__restrict__ awq,
                                                          const uint8_t *__restrict__ w, const __half *__restrict__ scales,
                                                          const __half *__restrict__ zeros, __half *__restrict__ y, int N,
                                                          int K, int B) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63, waves = nthr >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = K / kGS;
    const int rb = (int)((long long)N * blockIdx.x / gridDim.x);
    const int re = (int)((long long)N * (blockIdx.x + 1) / gridDim.x);
    const int j = lane & 15, kq = lane >> 4, r = j & 7, h = j >> 3;
    const int g0 = (G * wave) / waves, ng = (G * (wave + 1)) / waves - g0;
    const int RS = K + 8;
    _Float16 *img = reinterpret_cast<_Float16 *>(lds8);
    float *gsx = reinterpret_cast<float *>(lds8 + int8_band_img_bytes(K, B));
    __half *szl = reinterpret_cast<__half *>(gsx + G * 16);   // [band row][G] scales, then zero points
    const int nsz = (re - rb) * G;

    // (a) the first PX chunks of the activation, then this wave's weights,
    // scales and zero points, all issued before any of them is used (the
    // loads complete in order, so the staging then waits for the activation
    // alone)
    const int cpr = K / 8, nch = B * cpr;
    u32x4_t xr[PX], ar[PX];
#pragma unroll
    for (int p = 0; p < PX; p++) {
        const int c = min(tid + p * nthr, nch - 1);
        const int b = c / cpr, ci = c - b * cpr;
        xr[p] = *reinterpret_cast<const u32x4_t *>(x + (size_t)b * K + (size_t)ci * 8);
        if (awq) ar[p] = *reinterpret_cast<const u32x4_t *>(awq + (size_t)ci * 8);
    }
    // the band's scales and zero points (rows rb .. re - 1 are consecutive),
    // stored to LDS after the activation is staged
    __half sr[PX], zr[PX];
#pragma unroll
    for (int p = 0; p < PX; p++) {
        const int e = min(tid + p * nthr, nsz - 1);
        sr[p] = scales[(size_t)rb * G + e];
        zr[p] = zeros[(size_t)rb * G + e];
    }
    // weights of the band's rows only: a buffer resource over rows rb .. re - 1,
    // so the lanes of rows past the band read zeros without touching memory.
    // Group i of every tile is issued one group ahead of its MFMAs (the first
    // before the staging): a wave whose next load cannot issue waits there, so
    // loads issued all at once held the MFMAs until the whole band was asked
    // for.  (An execution barrier between every wave's small loads and the
    // weights, which the INT4 band kernel takes, measured slower here.)
    constexpr uint32_t kRsrcWord3 = 0x00020000u;
    const __amdgpu_buffer_rsrc_t w_r =
        __builtin_amdgcn_make_buffer_rsrc((void *)(w + (size_t)rb * K), 0, (re - rb) * K, kRsrcWord3);
    u32x4_t wq[TM][NPW];
    auto load_group = [&](int i) __attribute__((always_inline)) {
        const int g = g0 + min(i, ng - 1);
#pragma unroll
        for (int t = 0; t < TM; t++)
            wq[t][i] = __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(w_r, (8 * t + r) * K + g * kGS + h * 64 + kq * 16, 0, 0));
    };
    load_group(0);
    // (b) the activation image of all of K: chunk c (8 elements) of batch row
    // b; the 8 chunks of a half group are 8 consecutive lanes
    auto stage = [&](int c, const u32x4_t &xv, const u32x4_t &av) {
        const int b = c / cpr, ci = c - b * cpr;
        const size_t k = (size_t)ci * 8;
        const _Float16 *xh = reinterpret_cast<const _Float16 *>(&xv);
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (float)xh[i];
        if (awq) {
            const _Float16 *ah = reinterpret_cast<const _Float16 *>(&av);
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = v[i] * __builtin_amdgcn_rcpf((float)ah[i]);
        }
        half8_t hi, lo;
        float sh = 0.0f, sl = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            hi[i] = (_Float16)v[i];
            lo[i] = (_Float16)(v[i] - (float)hi[i]);
            sh += (float)hi[i];
            sl += (float)lo[i];
        }
        *reinterpret_cast<half8_t *>(img + (size_t)b * RS + k) = hi;
        *reinterpret_cast<half8_t *>(img + (size_t)(B + b) * RS + k) = lo;
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
            sh += __shfl_xor(sh, o);
            sl += __shfl_xor(sl, o);
        }
        if ((ci & 7) == 0) {
            const int g = ci >> 4, hh = (ci >> 3) & 1;
            gsx[g * 16 + 4 * (2 * hh) + b] = sh * kTwoM24;
            gsx[g * 16 + 4 * (2 * hh + 1) + b] = sl * kTwoM24;
        }
    };
    // nch is a multiple of 16: the 8 lanes of a half group pass or fail each bound together
#pragma unroll
    for (int p = 0; p < PX; p++)
        if (tid + p * nthr < nch) stage(tid + p * nthr, xr[p], ar[p]);
    for (int c = tid + PX * nthr; c < nch; c += nthr) {
        const int b = c / cpr, ci = c - b * cpr;
        const u32x4_t xv = *reinterpret_cast<const u32x4_t *>(x + (size_t)b * K + (size_t)ci * 8);
        u32x4_t av = xv;
        if (awq) av = *reinterpret_cast<const u32x4_t *>(awq + (size_t)ci * 8);
        stage(c, xv, av);
    }
    // then the scales and zero points (their wait may cover the weights)
#pragma unroll
    for (int p = 0; p < PX; p++)
        if (tid + p * nthr < nsz) {
            szl[tid + p * nthr] = sr[p];
            szl[nsz + tid + p * nthr] = zr[p];
        }
    for (int e = tid + PX * nthr; e < nsz; e += nthr) {
        szl[e] = scales[(size_t)rb * G + e];
        szl[nsz + e] = zeros[(size_t)rb * G + e];
    }
    __syncthreads();
    // (c) MFMAs: A row of this lane (i = j): half j >> 3, plane (j >> 2) & 1, batch row j & 3
    const int ab = (j & 3) < B ? (j & 3) : 0;
    const _Float16 *xa = img + (size_t)(((j >> 2) & 1) * B + ab) * RS + (j >> 3) * 64 + kq * 16;
    float4_t acc[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) acc[t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NPW; i++) {
        if (i + 1 < NPW) load_group(i + 1);
        if (i < ng) {
            const int g = g0 + i;
            const half8_t a0 = *reinterpret_cast<const half8_t *>(xa + (size_t)g * kGS);
            const half8_t a1 = *reinterpret_cast<const half8_t *>(xa + (size_t)g * kGS + 8);
            const float4_t sx = *reinterpret_cast<const float4_t *>(gsx + g * 16 + 4 * kq);
#pragma unroll
            for (int t = 0; t < TM; t++) {
                float4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const uint32_t w0 = wq[t][i][2 * u], w1 = wq[t][i][2 * u + 1];
                    const u32x4_t bq = {__builtin_amdgcn_perm(0u, w0, 0x0C010C00u), __builtin_amdgcn_perm(0u, w0, 0x0C030C02u),
                                        __builtin_amdgcn_perm(0u, w1, 0x0C010C00u), __builtin_amdgcn_perm(0u, w1, 0x0C030C02u)};
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(u ? a1 : a0, __builtin_bit_cast(half8_t, bq), d, 0, 0, 0);
                }
                const int lr = min(8 * t + r, re - rb - 1);
                const float s24 = __half2float(szl[lr * G + g]) * kTwo24, z = __half2float(szl[nsz + lr * G + g]);
#pragma unroll
                for (int q = 0; q < 4; q++) acc[t][q] = __builtin_fmaf(s24, __builtin_fmaf(-z, sx[q], d[q]), acc[t][q]);
            }
        }
    }
    __syncthreads();
    // (d) partials over the image; thread (t, r, b) sums waves, halves and planes in order
    float4_t *red = reinterpret_cast<float4_t *>(lds8);
#pragma unroll
    for (int t = 0; t < TM; t++) red[(wave * TM + t) * 64 + lane] = acc[t];
    __syncthreads();
    // the block is sized from K, so it may hold fewer threads than outputs
    for (int o = tid; o < TM * 8 * B; o += nthr) {
        const int t = o / (8 * B), rr = (o / B) & 7, b = o % B;
        const int row = rb + 8 * t + rr;
        if (row >= re) continue;
        float s = 0.0f;
        for (int wv = 0; wv < waves; wv++) {
            const float4_t *p = red + (wv * TM + t) * 64;
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
                for (int pl = 0; pl < 2; pl++) s += p[16 * (2 * hh + pl) + rr + 8 * hh][b];
        }
        y[(size_t)b * N + row] = __float2half(s);
    }
}

// false (nothing launched) if the runtime refuses LDS above 64 KB (gfx950 has 160 KB per CU)
template <int TM, int NPW>
bool launch_int8_band(hipStream_t st, int nwg, int waves, size_t lds, const __half *x, const __half *awq, const uint8_t *w,
                      const __half *sc, const __half *zr, __half *y, int N, int K, int B) {
    if (lds > 64 * 1024 && hipFuncSetAttribute(reinterpret_cast<const void *>(int8w_band_kernel<TM, NPW>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    hipLaunchKernelGGL((int8w_band_kernel<TM, NPW>), dim3(nwg), dim3(64 * waves), lds, st, x, awq, w, sc, zr, y, N, K, B);
    return true;
}

// Picks the band shape: bands of at most 5 tiles, waves holding at most
// 10 / TM groups per tile (10 for one row in 2-tile bands over more than 40
// groups), 1-4 batch rows whose image fits 156 KB of LDS.
// Returns false (nothing launched) when the shape is outside those limits.
bool int8_band_launch(hipStream_t st, int cus, const __half *x, const __half *awq, const uint8_t *w, const __half *sc,
                      const __half *zr, __half *y, int N, int K, int B) {
    const int G = K / kGS;
    if (B < 1 || B > 4) return false;
    int nwg = std::min(cus, (N + 7) / 8);
    while ((N + nwg - 1) / nwg > 40) nwg += cus;
    const int TM = ((N + nwg - 1) / nwg + 7) / 8;
    const size_t img = int8_band_img_bytes(K, B) + (size_t)G * 16 * 4 + (size_t)TM * 8 * G * 4;
    if (img > 156 * 1024) return false;
    // one row over more than 40 groups in 2-tile bands (down): eight waves of
    // up to 10 groups -- B=1 9.28 -> 8.85 us against sixteen of 5; at 2-3
    // rows that measured ~7 % slower
    const int npw = TM == 2 && G > 40 && B == 1 ? 10 : std::min(8, 10 / TM);
    const int waves = std::max(1, (G + npw - 1) / npw);
    if (waves > 16) return false;
    const size_t lds = std::max(img, (size_t)waves * TM * 64 * sizeof(float4_t));
    switch (TM) {
        case 1: return launch_int8_band<1, 8>(st, nwg, waves, lds, x, awq, w, sc, zr, y, N, K, B);
        case 2:
            if (npw == 10) return launch_int8_band<2, 10>(st, nwg, waves, lds, x, awq, w, sc, zr, y, N, K, B);
            return launch_int8_band<2, 5>(st, nwg, waves, lds, x, awq, w, sc, zr, y, N, K, B);
        case 3: return launch_int8_band<3, 3>(st, nwg, waves, lds, x, awq, w, sc, zr, y, N, K, B);
        case 4: return launch_int8_band<4, 2>(st, nwg, waves, lds, x, awq, w, sc, zr, y, N, K, B);
        default: return launch_int8_band<5, 2>(st, nwg, waves, lds, x, awq, w, sc, zr, y, N, K, B);
    }
}

// ---------------------------------------------------------------------------
// quantize_input_q8: grid (K / 128, B), block 128 (one thread per element)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kGS) q8_quantize_kernel(const __half *__restrict__ x, int8_t *__restrict__ q8,
                                                          float *__restrict__ q8_scales, int K) {
    __shared__ float wmax[2];
    const int g = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const size_t i = (size_t)b * K + (size_t)g * kGS + t;
    const float v = __half2float(x[i]);
    float m = fabsf(v);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((t & 63) == 0) wmax[t >> 6] = m;
    __syncthreads();
    m = fmaxf(wmax[0], wmax[1]);
    const float scale = m / 127.0f;
    const float inv = m > 0.0f ? 127.0f / m : 0.0f;
    if (t == 0) q8_scales[(size_t)b * (K / kGS) + g] = scale;
    q8[i] = (int8_t)fminf(fmaxf(rintf(v * inv), -127.0f), 127.0f);
}

// ---------------------------------------------------------------------------
// INT4 weights x Q8 activations on the integer matrix cores
// ---------------------------------------------------------------------------
// grid (ceil(N / 16), ceil(B / 16)), block 64 * waves.  LDS per stage: q8
// rows [16][SG * 128] (batch rows of the tile; rows past B read row 0), the
// rows' group sums of q8 [SG][16] (int32) and scales [SG][16]; then partials.
// Lane (n_l, kq) holds codes 32 kq .. 32 kq + 31 of its row's group (one
// 16-byte load), MFMA j takes codes 32 kq + 16 j .. + 15 as int8 in natural
// order, against the same 16 q8 bytes of A row n_l.
__global__ void __launch_bounds__(64 * kMaxWaves) int4xq8_matvec_kernel(
    const int8_t *__restrict__ q8, const float *__restrict__ q8_scales, const uint8_t *__restrict__ w,
    const __half *__restrict__ scales, const __half *__restrict__ zeros, __half *__restrict__ y, int N, int K, int B,
    int SG) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, waves = nthr >> 6;
    const int n_l = lane & 15, kq = lane >> 4;
    const int G = K / kGS;
    const int row0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
    const int bc = min(16, B - m0);
    const int row = row0 + n_l, row_c = min(row, N - 1);
    const int RS = SG * kGS + 16;                       // LDS row stride (bytes)
    int8_t *img = reinterpret_cast<int8_t *>(lds8);
    int *gsum = reinterpret_cast<int *>(lds8 + (size_t)16 * RS);
    float *gscl = reinterpret_cast<float *>(gsum + SG * 16);

    float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < G; s0 += SG) {
        const int SGs = min(SG, G - s0);
        const int g0 = s0 + (wave * SGs) / waves;
        const int ng = s0 + ((wave + 1) * SGs) / waves - g0;
        u32x4_t wq[kNG];
#pragma unroll
        for (int i = 0; i < kNG; i++) {
            const int g = min(g0 + min(i, max(ng - 1, 0)), G - 1);
            wq[i] = *reinterpret_cast<const u32x4_t *>(w + (size_t)row_c * (K / 2) + (size_t)g * 64 + kq * 16);
        }
        // q8 rows of the stage: 16-byte chunks, 8 per group row; the 8 chunks
        // of a (row, group) are 8 consecutive lanes
        const int cpr = SGs * 8;
        for (int c = tid; c < 16 * cpr; c += nthr) {
            const int r = c / cpr, ci = c - r * cpr;
            const int rb = r < bc ? r : 0;
            const size_t k = (size_t)s0 * kGS + (size_t)ci * 16;
            const u32x4_t v = *reinterpret_cast<const u32x4_t *>(q8 + (size_t)(m0 + rb) * K + k);
            *reinterpret_cast<u32x4_t *>(img + (size_t)r * RS + ci * 16) = v;
            int sum = 0;
#pragma unroll
            for (int d = 0; d < 4; d++) sum = __builtin_amdgcn_sdot4((int)v[d], 0x01010101, sum, false);
            sum += __shfl_xor(sum, 1);
            sum += __shfl_xor(sum, 2);
            sum += __shfl_xor(sum, 4);
            if ((ci & 7) == 0) {
                const int g = ci / 8;
                gsum[g * 16 + r] = sum;
                gscl[g * 16 + r] = q8_scales[(size_t)(m0 + rb) * G + s0 + g];
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kNG; i++) {
            if (i < ng) {
                const int g = g0 + i;
                const float ws = __half2float(scales[(size_t)row_c * G + g]);
                const float iz = rintf(__half2float(zeros[(size_t)row_c * G + g]));
                i32x4_t ai = {0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    // codes 32 kq + 16 j .. + 15 in natural order: dword pairs (2 j, 2 j + 1)
                    u32x4_t bq;
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const uint32_t wd = wq[i][2 * j + h];
                        const uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
                        bq[2 * h] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
                        bq[2 * h + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
                    }
                    const u32x4_t av =
                        *reinterpret_cast<const u32x4_t *>(img + (size_t)n_l * RS + (g - s0) * kGS + kq * 32 + j * 16);
                    ai = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, av), __builtin_bit_cast(i32x4_t, bq),
                                                               ai, 0, 0, 0);
                }
                // D rows 4 kq + r are batch rows; column n_l is this lane's weight row
                const i32x4_t gs4 = *reinterpret_cast<const i32x4_t *>(gsum + (g - s0) * 16 + 4 * kq);
                const float4_t as4 = *reinterpret_cast<const float4_t *>(gscl + (g - s0) * 16 + 4 * kq);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc[r] = __builtin_fmaf(ws * as4[r], (float)(ai[r] - (int)iz * gs4[r]), acc[r]);
            }
        }
        __syncthreads();
    }
    float4_t *red = reinterpret_cast<float4_t *>(lds8);
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave != 0 || row >= N) return;
    float4_t s = red[lane];
    for (int wv = 1; wv < waves; wv++) s += red[wv * 64 + lane];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int b = 4 * kq + r;
        if (b < bc) y[(size_t)(m0 + b) * N + row] = __float2half(s[r]);
    }
}

// ---------------------------------------------------------------------------
// INT4 x Q8, 1-8 batch rows, over a grid balanced on the compute units
// ---------------------------------------------------------------------------
// Row bands as in int8w_band_kernel.  Lane (r, h, kq) loads 16 bytes (32
// codes) of row r at byte 64 (2p + h) + 16 kq of the band's group pair p, so
// a wave reads 8 rows x 128 contiguous bytes; B column j = r + 8h, A row i =
// 8h + b (batch row b, rows past B read row 0); MFMA u takes codes 32 kq + 16u
// .. + 15 of group 2p + h against the same q8 bytes.  Only result entries
// whose row and column share h are used (lane l: (l >> 5) == ((l >> 3) & 1)).
// Per group: ws * as * (sum q8 q - rint(z) sum q8) in f32 from the exact
// int32 sums.  LDS: q8 image [B][K + 16], per-group q8 sums [G][8] int32 and
// activation scales [G][8] f32, the band's scales and zero points [rows][G]
// f16; the wave partials overlay them, summed in (wave, h) order.
// FQ: the activation arrives as f16 and every workgroup quantizes it while it
// stages it, with quantize_input_q8's arithmetic (q8_quantize_kernel: the
// group's absmax over its 8 chunk lanes, scale = m / 127, q = clamp(rint(v *
// (127 / m)), -127, 127)), so the codes and scales are those the separate
// launch writes; workgroup 0 also stores them when q8_out is set.
__host__ __device__ inline size_t q8_band_lds(int K, int B, int G, int TM) {
    return (size_t)B * (K + 16) + (size_t)G * 8 * 8 + (size_t)TM * 8 * G * 4;
}

// 16 f16 activations (two 16-byte halves) -> 16 Q8 codes packed little-endian,
// and the group's scale; the 8 chunks of a group are 8 consecutive lanes
__device__ __forceinline__ u32x4_t q8_chunk(const u32x4_t &xa, const u32x4_t &xb, float &scale) {
    const _Float16 *h0 = reinterpret_cast<const _Float16 *>(&xa);
    const _Float16 *h1 = reinterpret_cast<const _Float16 *>(&xb);
    float v[16];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        v[i] = (float)h0[i];
        v[8 + i] = (float)h1[i];
    }
#pragma unroll
    for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, __shfl_xor(m, 1));
    m = fmaxf(m, __shfl_xor(m, 2));
    m = fmaxf(m, __shfl_xor(m, 4));
    scale = m / 127.0f;
    const float inv = m > 0.0f ? 127.0f / m : 0.0f;
    u32x4_t out;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int qv = (int)fminf(fmaxf(rintf(v[4 * d + e] * inv), -127.0f), 127.0f);
            word |= ((uint32_t)qv & 0xFFu) << (8 * e);
        }
        out[d] = word;
    }
    return out;
}

template <int TM, int NPW, bool FQ>
__global__ void __launch_bounds__(1024) int4xq8_band_kernel(const int8_t *__restrict__ q8, const float *__restrict__ q8_scales,
                                                            const __half *__restrict__ x16, int8_t *__restrict__ q8_out,
                                                            float *__restrict__ q8s_out,
                                                            const uint8_t *__restrict__ w, const __half *__restrict__ scales,
                                                            const __half *__restrict__ zeros, __half *__restrict__ y, int N,
                                                            int K, int B) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63, waves = nthr >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = K / kGS, GP = (G + 1) / 2;
    const int rb = (int)((long long)N * blockIdx.x / gridDim.x);
    const int re = (int)((long long)N * (blockIdx.x + 1) / gridDim.x);
    const int j = lane & 15, kq = lane >> 4, r = j & 7, h = j >> 3;
    const int p0 = (GP * wave) / waves, np = (GP * (wave + 1)) / waves - p0;
    const int RS = K + 16;
    int8_t *img = reinterpret_cast<int8_t *>(lds8);
    int *gsum = reinterpret_cast<int *>(lds8 + (size_t)B * RS);
    float *gscl = reinterpret_cast<float *>(gsum + G * 8);
    __half *szl = reinterpret_cast<__half *>(gscl + G * 8);
    const int nsz = (re - rb) * G;
    const bool store_q8 = FQ && q8_out && blockIdx.x == 0;

    // (a) the first activation chunk per thread (16 q8 codes, or FQ: their 16
    // f16 values), the band's scales / zero points, then this wave's weights
    // (a buffer resource over the band's rows: lanes past it, or past the
    // row's last group, read zeros or are discarded)
    const int cpr = K / 16, nch = B * cpr;
    const int c0 = min(tid, nch - 1);
    u32x4_t x0, x0b;
    if constexpr (FQ) {
        const __half *src = x16 + (size_t)(c0 / cpr) * K + (size_t)(c0 % cpr) * 16;
        x0 = *reinterpret_cast<const u32x4_t *>(src);
        x0b = *reinterpret_cast<const u32x4_t *>(src + 8);
    } else {
        x0 = *reinterpret_cast<const u32x4_t *>(q8 + (size_t)(c0 / cpr) * K + (size_t)(c0 % cpr) * 16);
        x0b = x0;
    }
    const int e0 = min(tid, nsz - 1);
    const __half s0 = scales[(size_t)rb * G + e0], z0 = zeros[(size_t)rb * G + e0];
    constexpr uint32_t kRsrcWord3 = 0x00020000u;
    const __amdgpu_buffer_rsrc_t w_r =
        __builtin_amdgcn_make_buffer_rsrc((void *)(w + (size_t)rb * (K / 2)), 0, (re - rb) * (K / 2), kRsrcWord3);
    // pair i of every tile issued one pair ahead of its MFMAs (the first now),
    // as in the INT8 band kernel
    u32x4_t wq[TM][NPW];
    auto load_pair = [&](int i) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TM; t++)
            wq[t][i] = __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                             w_r, (8 * t + r) * (K / 2) + (2 * (p0 + min(i, np - 1)) + h) * 64 + kq * 16, 0, 0));
    };
    load_pair(0);
    // (b) q8 rows into LDS with each group's sum (8 consecutive lanes per group)
    auto stage = [&](int c, const u32x4_t &xa, const u32x4_t &xb) {
        const int b = c / cpr, ci = c - b * cpr;
        float scl = 0.0f;
        u32x4_t v = xa;
        if constexpr (FQ) v = q8_chunk(xa, xb, scl);
        *reinterpret_cast<u32x4_t *>(img + (size_t)b * RS + ci * 16) = v;
        if (store_q8) *reinterpret_cast<u32x4_t *>(q8_out + (size_t)b * K + ci * 16) = v;
        int sum = 0;
#pragma unroll
        for (int d = 0; d < 4; d++) sum = __builtin_amdgcn_sdot4((int)v[d], 0x01010101, sum, false);
        sum += __shfl_xor(sum, 1);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 4);
        if ((ci & 7) == 0) {
            gsum[(ci >> 3) * 8 + b] = sum;
            if constexpr (!FQ) scl = q8_scales[(size_t)b * G + (ci >> 3)];
            gscl[(ci >> 3) * 8 + b] = scl;
            if (store_q8) q8s_out[(size_t)b * G + (ci >> 3)] = scl;
        }
    };
    // nch is a multiple of 8: the 8 lanes of a group pass or fail each bound together
    if (tid < nch) stage(tid, x0, x0b);
    for (int c = tid + nthr; c < nch; c += nthr) {
        u32x4_t xa, xb;
        if constexpr (FQ) {
            const __half *src = x16 + (size_t)(c / cpr) * K + (size_t)(c % cpr) * 16;
            xa = *reinterpret_cast<const u32x4_t *>(src);
            xb = *reinterpret_cast<const u32x4_t *>(src + 8);
        } else {
            xa = *reinterpret_cast<const u32x4_t *>(q8 + (size_t)(c / cpr) * K + (size_t)(c % cpr) * 16);
            xb = xa;
        }
        stage(c, xa, xb);
    }
    if (tid < nsz) {
        szl[tid] = s0;
        szl[nsz + tid] = z0;
    }
    for (int e = tid + nthr; e < nsz; e += nthr) {
        szl[e] = scales[(size_t)rb * G + e];
        szl[nsz + e] = zeros[(size_t)rb * G + e];
    }
    __syncthreads();
    // (c) integer MFMAs; A row of this lane: half j >> 3, batch row j & 7
    const int ab = (j & 7) < B ? (j & 7) : 0;
    const int8_t *xa = img + (size_t)ab * RS + (j >> 3) * kGS + kq * 32;
    const int bq0 = 4 * ((lane >> 4) & 1);   // batch rows of this lane's D rows
    float4_t acc[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) acc[t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NPW; i++) {
        if (i + 1 < NPW) load_pair(i + 1);
        if (i < np) {
            const int pg = 2 * (p0 + i);   // first group of the pair
            const u32x4_t a0 = *reinterpret_cast<const u32x4_t *>(xa + (size_t)pg * kGS);
            const u32x4_t a1 = *reinterpret_cast<const u32x4_t *>(xa + (size_t)pg * kGS + 16);
            const int g = pg + h;          // this lane's column group
            const int gc = min(g, G - 1);
            const i32x4_t gs4 = *reinterpret_cast<const i32x4_t *>(gsum + gc * 8 + bq0);
            const float4_t as4 = *reinterpret_cast<const float4_t *>(gscl + gc * 8 + bq0);
#pragma unroll
            for (int t = 0; t < TM; t++) {
                i32x4_t ai = {0, 0, 0, 0};
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    u32x4_t bq;
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        const uint32_t wd = wq[t][i][2 * u + hh];
                        const uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
                        bq[2 * hh] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
                        bq[2 * hh + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
                    }
                    ai = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, u ? a1 : a0),
                                                               __builtin_bit_cast(i32x4_t, bq), ai, 0, 0, 0);
                }
                if (g < G) {
                    const int lr = min(8 * t + r, re - rb - 1);
                    const float ws = __half2float(szl[lr * G + g]);
                    const int iz = (int)rintf(__half2float(szl[nsz + lr * G + g]));
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        acc[t][q] = __builtin_fmaf(ws * as4[q], (float)(ai[q] - iz * gs4[q]), acc[t][q]);
                }
            }
        }
    }
    __syncthreads();
    // (d) partials over the image; thread (t, r, b) sums waves and halves in order
    float4_t *red = reinterpret_cast<float4_t *>(lds8);
#pragma unroll
    for (int t = 0; t < TM; t++) red[(wave * TM + t) * 64 + lane] = acc[t];
    __syncthreads();
    // the block is sized from K, so it may hold fewer threads than outputs
    for (int o = tid; o < TM * 8 * B; o += nthr) {
        const int t = o / (8 * B), rr = (o / B) & 7, b = o % B;
        const int row = rb + 8 * t + rr;
        if (row >= re) continue;
        float s = 0.0f;
        for (int wv = 0; wv < waves; wv++) {
            const float4_t *p = red + (wv * TM + t) * 64;
#pragma unroll
            for (int hh = 0; hh < 2; hh++) s += p[16 * (2 * hh + (b >> 2)) + rr + 8 * hh][b & 3];
        }
        y[(size_t)b * N + row] = __float2half(s);
    }
}

// The activation of the band launch: Q8 codes and scales, or (FQ) f16 rows
// quantized in the launch, optionally writing the codes and scales.
struct Q8Src {
    const int8_t *q8;
    const float *q8s;
    const __half *x16;
    int8_t *q8_out;
    float *q8s_out;
};

template <int TM, int NPW, bool FQ>
bool launch_q8_band_t(hipStream_t st, int nwg, int waves, size_t lds, const Q8Src &src, const uint8_t *w,
                      const __half *sc, const __half *zr, __half *y, int N, int K, int B) {
    if (lds > 64 * 1024 && hipFuncSetAttribute(reinterpret_cast<const void *>(int4xq8_band_kernel<TM, NPW, FQ>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    hipLaunchKernelGGL((int4xq8_band_kernel<TM, NPW, FQ>), dim3(nwg), dim3(64 * waves), lds, st, src.q8, src.q8s,
                       src.x16, src.q8_out, src.q8s_out, w, sc, zr, y, N, K, B);
    return true;
}

template <int TM, int NPW>
bool launch_q8_band(hipStream_t st, int nwg, int waves, size_t lds, const Q8Src &src, const uint8_t *w,
                    const __half *sc, const __half *zr, __half *y, int N, int K, int B) {
    return src.x16 ? launch_q8_band_t<TM, NPW, true>(st, nwg, waves, lds, src, w, sc, zr, y, N, K, B)
                   : launch_q8_band_t<TM, NPW, false>(st, nwg, waves, lds, src, w, sc, zr, y, N, K, B);
}

// Band shape as for the INT8 band kernel, over group pairs; 1-8 batch rows.
// Returns false (nothing launched) outside its limits.
bool q8_band_launch(hipStream_t st, int cus, const Q8Src &src, const uint8_t *w, const __half *sc, const __half *zr,
                    __half *y, int N, int K, int B) {
    const int G = K / kGS, GP = (G + 1) / 2;
    if (B < 1 || B > 8) return false;
    int nwg = std::min(cus, (N + 7) / 8);
    while ((N + nwg - 1) / nwg > 40) nwg += cus;
    const int TM = ((N + nwg - 1) / nwg + 7) / 8;
    // 5-tile bands (the gate shape): one group pair per wave, as many waves
    // as pairs -- B=1 / 2 / 4 7.96 / 8.01 / 8.94 -> 6.97 / 7.25 / 7.64 us
    // against five waves of two (four of three: 8.02 / 8.78 / 9.82 us)
    const int npw = TM == 5 ? 1 : std::min(8, 10 / TM);
    const int waves = std::max(1, (GP + npw - 1) / npw);
    if (waves > 16) return false;
    const size_t lds = std::max(q8_band_lds(K, B, G, TM), (size_t)waves * TM * 64 * sizeof(float4_t));
    if (lds > 156 * 1024) return false;
    switch (TM) {
        case 1: return launch_q8_band<1, 8>(st, nwg, waves, lds, src, w, sc, zr, y, N, K, B);
        case 2: return launch_q8_band<2, 5>(st, nwg, waves, lds, src, w, sc, zr, y, N, K, B);
        case 3: return launch_q8_band<3, 3>(st, nwg, waves, lds, src, w, sc, zr, y, N, K, B);
        case 4: return launch_q8_band<4, 2>(st, nwg, waves, lds, src, w, sc, zr, y, N, K, B);
        default: return launch_q8_band<5, 1>(st, nwg, waves, lds, src, w, sc, zr, y, N, K, B);
    }
}

int check_w(const imh_affine_int4_weight *w, const char *who) {
    if (!w || !w->data || !w->scales || !w->zeros)
        return imh::fail(IMH_EINVAL, std::string(who) + ": weight or one of its arrays is NULL");
    if (w->group_size != kGS)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": group_size " + std::to_string(w->group_size) +
                                               " not supported (built for 128)");
    if (w->n == 0 || w->k == 0 || w->k % kGS)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": k must be a non-zero multiple of 128, n non-zero");
    if ((reinterpret_cast<uintptr_t>(w->data) & 15) != 0)
        return imh::fail(IMH_EINVAL, std::string(who) + ": weight data must be 16-byte aligned");
    return IMH_OK;
}

int waves_for(int G) { return std::max(1, std::min(kMaxWaves, (G + 3) / 4)); }

}  // namespace

extern "C" {

int imh_encode_affine_projection_int8(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                      const imh_affine_int8_weight *w8, uint16_t *y) {
    const char *who = "imh_encode_affine_projection_int8";
    if (!stream || !x || !y || !w8) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    const imh_affine_int4_weight *w = reinterpret_cast<const imh_affine_int4_weight *>(w8);
    int rc = check_w(w, who);
    if (rc) return rc;
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w->awq_scales)) & 15)
        return imh::fail(IMH_EINVAL, std::string(who) + ": x and awq_scales must be 16-byte aligned");
    if (token_count == 0) return IMH_OK;
    rc = imh::use_device(stream->dev);
    if (rc) return rc;
    const int N = (int)w->n, K = (int)w->k, G = K / kGS;
    if (token_count <= 4 &&
        int8_band_launch(stream->stream, stream->dev->props.multiProcessorCount, reinterpret_cast<const __half *>(x),
                         reinterpret_cast<const __half *>(w->awq_scales), w->data,
                         reinterpret_cast<const __half *>(w->scales), reinterpret_cast<const __half *>(w->zeros),
                         reinterpret_cast<__half *>(y), N, K, (int)token_count)) {
        IMH_HIP(hipGetLastError());
        return IMH_OK;
    }
    const int waves = waves_for(G);
    // batch rows in launches of up to 8 (rows 0-7 of the MFMA tile hi, 8-15 lo)
    for (uint32_t b0 = 0; b0 < token_count; b0 += 8) {
        const int B = (int)std::min<uint32_t>(8, token_count - b0);
        int SG = std::max(1, std::min(G, kStageBytes / (2 * B * (kGS + 8) * 2)));
        SG = std::min(SG, waves * kNG);
        const size_t lds = std::max((size_t)2 * B * (SG * kGS + 8) * 2 + (size_t)SG * 16 * 4,
                                    (size_t)waves * 64 * sizeof(float4_t));
        hipLaunchKernelGGL(int8w_matvec_kernel, dim3((N + 15) / 16), dim3(64 * waves), lds, stream->stream,
                           reinterpret_cast<const __half *>(x) + (size_t)b0 * K,
                           reinterpret_cast<const __half *>(w->awq_scales), w->data,
                           reinterpret_cast<const __half *>(w->scales), reinterpret_cast<const __half *>(w->zeros),
                           reinterpret_cast<__half *>(y) + (size_t)b0 * N, N, K, B, SG);
        IMH_HIP(hipGetLastError());
    }
    return IMH_OK;
}

int imh_encode_quantize_input_q8(imh_stream *stream, const uint16_t *x, uint32_t token_count, uint32_t k,
                                 int8_t *q8, float *q8_scales) {
    const char *who = "imh_encode_quantize_input_q8";
    if (!stream || !x || !q8 || !q8_scales) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    if (k == 0 || k % kGS) return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": k must be a multiple of 128");
    if (token_count == 0) return IMH_OK;
    if (token_count > 65535) return imh::fail(IMH_EINVAL, std::string(who) + ": token_count above 65535");
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    hipLaunchKernelGGL(q8_quantize_kernel, dim3(k / kGS, token_count), dim3(kGS), 0, stream->stream,
                       reinterpret_cast<const __half *>(x), q8, q8_scales, (int)k);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

int imh_encode_affine_matvec_int4xq8(imh_stream *stream, const int8_t *q8, const float *q8_scales,
                                     uint32_t token_count, const imh_affine_int4_weight *w, uint16_t *y) {
    const char *who = "imh_encode_affine_matvec_int4xq8";
    if (!stream || !q8 || !q8_scales || !y) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_w(w, who);
    if (rc) return rc;
    if (reinterpret_cast<uintptr_t>(q8) & 15) return imh::fail(IMH_EINVAL, std::string(who) + ": q8 must be 16-byte aligned");
    if (w->awq_scales)
        return imh::fail(IMH_EINVAL, std::string(who) + ": the Q8 path has no AWQ division (pipeline.rs:639-664)");
    if (token_count == 0) return IMH_OK;
    if (token_count > 65535u * 16) return imh::fail(IMH_EINVAL, std::string(who) + ": token_count too large");
    rc = imh::use_device(stream->dev);
    if (rc) return rc;
    const int N = (int)w->n, K = (int)w->k, G = K / kGS;
    const Q8Src src = {q8, q8_scales, nullptr, nullptr, nullptr};
    if (token_count <= 8 &&
        q8_band_launch(stream->stream, stream->dev->props.multiProcessorCount, src, w->data,
                       reinterpret_cast<const __half *>(w->scales), reinterpret_cast<const __half *>(w->zeros),
                       reinterpret_cast<__half *>(y), N, K, (int)token_count)) {
        IMH_HIP(hipGetLastError());
        return IMH_OK;
    }
    const int waves = waves_for(G);
    int SG = std::max(1, std::min(G, kStageBytes / (16 * (kGS + 16))));
    SG = std::min(SG, waves * kNG);
    const size_t lds = std::max((size_t)16 * (SG * kGS + 16) + (size_t)SG * 16 * 8, (size_t)waves * 64 * sizeof(float4_t));
    hipLaunchKernelGGL(int4xq8_matvec_kernel, dim3((N + 15) / 16, (token_count + 15) / 16), dim3(64 * waves), lds,
                       stream->stream, q8, q8_scales, w->data, reinterpret_cast<const __half *>(w->scales),
                       reinterpret_cast<const __half *>(w->zeros), reinterpret_cast<__half *>(y), N, K,
                       (int)token_count, SG);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

int imh_encode_affine_projection_int4_q8(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                         const imh_affine_int4_weight *w, uint16_t *y, int8_t *q8_out,
                                         float *q8_scales_out) {
    const char *who = "imh_encode_affine_projection_int4_q8";
    if (!stream || !x || !y) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_w(w, who);
    if (rc) return rc;
    if (w->awq_scales)
        return imh::fail(IMH_EINVAL, std::string(who) + ": the Q8 path has no AWQ division (pipeline.rs:639-664)");
    if ((q8_out == nullptr) != (q8_scales_out == nullptr))
        return imh::fail(IMH_EINVAL, std::string(who) + ": q8_out and q8_scales_out are both given or both NULL");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(q8_out)) & 15)
        return imh::fail(IMH_EINVAL, std::string(who) + ": x and q8_out must be 16-byte aligned");
    if (token_count == 0) return IMH_OK;
    if (token_count > 65535) return imh::fail(IMH_EINVAL, std::string(who) + ": token_count above 65535");
    rc = imh::use_device(stream->dev);
    if (rc) return rc;
    const int N = (int)w->n, K = (int)w->k, G = K / kGS;
    const Q8Src src = {nullptr, nullptr, reinterpret_cast<const __half *>(x), q8_out, q8_scales_out};
    if (token_count <= 8 &&
        q8_band_launch(stream->stream, stream->dev->props.multiProcessorCount, src, w->data,
                       reinterpret_cast<const __half *>(w->scales), reinterpret_cast<const __half *>(w->zeros),
                       reinterpret_cast<__half *>(y), N, K, (int)token_count)) {
        IMH_HIP(hipGetLastError());
        return IMH_OK;
    }
    // outside the band kernel's shapes: the two launches, the codes in the
    // caller's buffers or the stream's scratch memory
    int8_t *q8 = q8_out;
    float *q8s = q8_scales_out;
    if (!q8) {
        void *scr = nullptr;
        const size_t code_bytes = ((size_t)token_count * K + 255) & ~(size_t)255;
        rc = imh::stream_scratch(stream, 0, code_bytes + (size_t)token_count * G * sizeof(float), &scr);
        if (rc) return rc;
        q8 = static_cast<int8_t *>(scr);
        q8s = reinterpret_cast<float *>(static_cast<uint8_t *>(scr) + code_bytes);
    }
    rc = imh_encode_quantize_input_q8(stream, x, token_count, (uint32_t)K, q8, q8s);
    return rc ? rc : imh_encode_affine_matvec_int4xq8(stream, q8, q8s, token_count, w, y);
}

}  // extern "C"
