// int4_gemm.hip -- INT4-affine (group 128) GEMM for prefill-sized token counts
// (superblock_matmul_int4, affine_matmul.metal:10-152, reached from
// encode_projection at token_count > 1, projection.rs:227-312).
//
//     C[m][n] = f16( sum_g s[n][g] * sum_{k in g} (x[m][k] / awq[k]) * (q[n][k] - z[n][g]) ),  f32 accumulate
//
// (q - z) is exact in f16 (integer zero-points, as the quantizer produces)
// and the scale is applied in f32 once per group, so no weight is rounded;
// x / awq keeps ~22 bits (f16 hi + lo).  The reference's prefill kernel
// instead rounds both the dequantized weight and a / awq to f16 (affine_matmul
// B dequant -> half, A rows = half(a / awq)), which costs several fp16 steps
// against the CPU path where terms cancel.
//
// MI355X design: one workgroup (4 waves) computes a 128 x 128 tile of C over
// 64-wide K stages (32-wide with AWQ, see the kernel), double-buffered in LDS.  Each stage the workgroup loads the
// next stage's activation (128 x 64 f16) and codes (128 x 64 nibbles + the
// group's scale/zero) into registers before the current stage's MFMAs, then
// turns the codes into q - z (nibbles -> f16 with a 0x64 exponent byte, one
// packed subtract of 1024 + z) and stores both operands into the other LDS
// buffer: one barrier per stage.  Each wave owns a 64 x 64 quarter of the
// tile: 4 x 4 v_mfma_f32_16x16x32_f16 tiles accumulating the group's partial
// sums, folded into the f32 result with the group's scale at every group end.  Within every 8-element chunk both operands sit in the slot order
// {0, 2, 4, 6, 1, 3, 5, 7} that the nibble unpack produces.  When the tile
// grid is smaller than the CU count, K is split over workgroups; the f32
// partials are summed in split order by a second kernel (deterministic).
//
// A gate/up pair runs as one GEMM: the B tile's first 64 rows come from the
// gate matrix and the last 64 from up (same output columns), so a workgroup
// holds both results of its 128 x 64 output tile in f32 and applies SiLU /
// GELU (or stores both) before rounding -- the fused epilogue of
// affine_fused.metal:89-107 at prefill sizes, with no f16 intermediate.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <string>

#include "imh_internal.h"
#include "int4_gemm.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGS = 128;
constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;         // K per stage without AWQ (32 with)
constexpr int kThreads = 256;

__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

enum GemmEpi : int { GE_STORE, GE_SILU, GE_GELU };

struct GemmMats {
    const uint8_t *data[2];
    const __half *scales[2];
    const __half *zeros[2];
    __half *out[2];
};

__device__ __forceinline__ float gate_act(float g, float u, int epi) {
    float act;
    if (epi == GE_GELU) {
        float inner = 0.7978845608f * (g + 0.044715f * g * g * g);
        inner = fminf(fmaxf(inner, -10.0f), 10.0f);
        act = 0.5f * g * (1.0f + tanhf(inner));
    } else {
        act = g / (1.0f + __expf(-g));
    }
    return act * u;
}

// grid (ceil(N / (128 / NMAT)), ceil(M/128), splits), block 256.  Split z
// covers K stages [z * stages_per_split, ...).  NMAT == 1: a 128 x 128 tile of
// C = x . W0^T.  NMAT == 2: a 128 x 64 tile of both x . W0^T (B rows 0-63,
// waves wn = 0) and x . W1^T (B rows 64-127, waves wn = 1).  Without a split
// the epilogue stores f16 results (EPI); with one it writes f32 partials
// [splits][M][NMAT * N] for int4_gemm_reduce_kernel.
//
// Without AWQ the activation is f16 already and enters the MFMA exactly
// (64-wide K stages).  With AWQ, x / awq is split into f16 hi + lo planes
// (~22-bit operands, two MFMAs per step, 32-wide K stages so two workgroups
// still fit a CU's LDS): rounding x / awq to f16 alone moves outputs by
// several fp16 steps where terms cancel.  The planes are built once, in slot
// order, by int4_gemm_prep_kernel (x = the hi plane, xlo = the lo plane):
// built per workgroup they were redone by every column tile and made the
// kernel VALU-bound.
template <bool AWQ, int NMAT>
__global__ void __launch_bounds__(kThreads, 2) int4_gemm_kernel(
    const __half *__restrict__ x, const __half *__restrict__ xlo, GemmMats mats, int epi,
    float *__restrict__ part, int M, int N, int K, int stages_per_split) {
    constexpr int kTN = kBN / NMAT;          // output columns per matrix
    constexpr int BK = AWQ ? 32 : 64;        // K per stage
    constexpr int ROW = BK + 8;              // LDS row stride in halfs (16-byte pad)
    constexpr int NPL = AWQ ? 2 : 1;         // activation planes (hi, lo)
    constexpr int ACH = kBM * BK / 8 / kThreads;  // activation chunks of 8 per thread
    constexpr int BDW = BK / 16;             // code dwords per thread
    constexpr int SPG = kGS / BK;            // stages per quantization group
    __shared__ __attribute__((aligned(16))) _Float16 As[2][NPL][kBM * ROW];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][kBN * ROW];
    __shared__ float Ss[2][kBN];             // the stage's group scale per B row

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kTN;
    const int G = K / kGS;
    const int total_stages = K / BK;
    const int s_begin = blockIdx.z * stages_per_split;
    const int s_end = min(s_begin + stages_per_split, total_stages);

    // staging roles: A -- ACH chunks of 8 halfs per thread (chunk c = i*256 +
    // tid: row c / (BK/8), column chunk c % (BK/8)); B -- row tid / 2, BDW code
    // dwords at half tid % 2 of the stage
    const int b_row = tid >> 1, b_half = tid & 1;
    const int b_mat = NMAT == 2 ? b_row / kTN : 0;
    const int b_n = min(n0 + b_row - b_mat * kTN, N - 1);
    // matrix by select: a dynamic index into the argument struct would turn
    // into memory loads
    const uint8_t *b_data = b_mat ? mats.data[1] : mats.data[0];
    const __half *scales = b_mat ? mats.scales[1] : mats.scales[0];
    const __half *zeros = b_mat ? mats.zeros[1] : mats.zeros[0];
    const uint8_t *b_src = b_data + (size_t)b_n * (K / 2) + b_half * (BK / 4);

    // one stage's global loads, held in registers until stored to LDS
    struct StageRegs {
        u32x4_t a[ACH], w[ACH];
        uint32_t b[BDW];
        uint32_t sz;
    };

    auto load_stage = [&](int st, StageRegs &rg) __attribute__((always_inline)) {
        u32x4_t *a_reg = rg.a, *a_w = rg.w;
        uint32_t *b_reg = rg.b;
        const int k0 = st * BK;
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int c = i * kThreads + tid;
            const int r = c / (BK / 8), kc = c % (BK / 8);
            const int m = min(m0 + r, M - 1);
            a_reg[i] = *reinterpret_cast<const u32x4_t *>(x + (size_t)m * K + k0 + kc * 8);
            if (AWQ) a_w[i] = *reinterpret_cast<const u32x4_t *>(xlo + (size_t)m * K + k0 + kc * 8);
        }
        const uint32_t *bp = reinterpret_cast<const uint32_t *>(b_src + (size_t)k0 / 2);
        if (BDW == 4) {
            const u32x4_t v = *reinterpret_cast<const u32x4_t *>(bp);
#pragma unroll
            for (int j = 0; j < BDW; j++) b_reg[j] = v[j];
        } else {
            const uint2 v = *reinterpret_cast<const uint2 *>(bp);
            b_reg[0] = v.x;
            b_reg[BDW - 1] = v.y;
        }
        const size_t gi = (size_t)b_n * G + k0 / kGS;
        rg.sz = (uint32_t)reinterpret_cast<const uint16_t *>(scales)[gi] |
                ((uint32_t)reinterpret_cast<const uint16_t *>(zeros)[gi] << 16);
    };

    // (e0 e1)(e2 e3)(e4 e5)(e6 e7) -> (e0 e2)(e4 e6)(e1 e3)(e5 e7)
    auto slot_order = [](u32x4_t v) __attribute__((always_inline)) {
        return (u32x4_t){__builtin_amdgcn_perm(v[1], v[0], 0x05040100u), __builtin_amdgcn_perm(v[3], v[2], 0x05040100u),
                         __builtin_amdgcn_perm(v[1], v[0], 0x07060302u), __builtin_amdgcn_perm(v[3], v[2], 0x07060302u)};
    };

    auto store_stage = [&](int buf, const StageRegs &rg) __attribute__((always_inline)) {
        const u32x4_t *a_reg = rg.a, *a_w = rg.w;
        const uint32_t *b_reg = rg.b;
        const uint32_t b_sz = rg.sz;
        // activation: x, or x / awq as hi + lo; slots {0,2,4,6,1,3,5,7} within each chunk
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int c = i * kThreads + tid;
            const int r = c / (BK / 8), kc = c % (BK / 8);
            if (AWQ) {   // planes already in slot order
                *reinterpret_cast<u32x4_t *>(&As[buf][0][r * ROW + kc * 8]) = a_reg[i];
                *reinterpret_cast<u32x4_t *>(&As[buf][NPL - 1][r * ROW + kc * 8]) = a_w[i];
            } else {
                *reinterpret_cast<u32x4_t *>(&As[buf][0][r * ROW + kc * 8]) = slot_order(a_reg[i]);
            }
        }
        // weights: q - z, exact in f16 (nibble beside a 0x64 exponent byte is
        // 1024 + q; one packed add of -(1024 + z)), same slot order; the
        // group's scale goes to LDS for the fold at the group's end
        const _Float16 z = __builtin_bit_cast(_Float16, (uint16_t)(b_sz >> 16));
        const _Float16 nb = (_Float16)(-(1024.0f + (float)z));
        const half2_t bias = {nb, nb};
        const uint32_t c64 = 0x64646464u;
#pragma unroll
        for (int j = 0; j < BDW; j++) {
            const uint32_t w = b_reg[j];
            const uint32_t lo = w & 0x0F0F0F0Fu;          // q0 q2 q4 q6
            const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // q1 q3 q5 q7
            const u32x4_t o = {as_u32(as_h2(__builtin_amdgcn_perm(lo, c64, 0x00050004u)) + bias),
                               as_u32(as_h2(__builtin_amdgcn_perm(lo, c64, 0x00070006u)) + bias),
                               as_u32(as_h2(__builtin_amdgcn_perm(hi, c64, 0x00050004u)) + bias),
                               as_u32(as_h2(__builtin_amdgcn_perm(hi, c64, 0x00070006u)) + bias)};
            *reinterpret_cast<u32x4_t *>(&Bs[buf][b_row * ROW + b_half * (BK / 2) + j * 8]) = o;
        }
        if (b_half == 0) Ss[buf][b_row] = (float)__builtin_bit_cast(_Float16, (uint16_t)(b_sz & 0xFFFFu));
    };

    // acc: the result; accg: the current group's sum of x * (q - z), folded
    // into acc with the group's scale when the group ends
    float4_t acc[4][4], accg[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc[i][j] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
            accg[i][j] = acc[i][j];
        }

    const int fr = lane & 15, fk = (lane >> 4) * 8;
    // the MFMAs of stage st from LDS buffer buf, and the group-end fold
    auto compute_stage = [&](int st, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < BK; ks += 32) {
            half8_t bf[4];
#pragma unroll
            for (int t = 0; t < 4; t++)
                bf[t] = *reinterpret_cast<const half8_t *>(&Bs[buf][(wn * 64 + t * 16 + fr) * ROW + ks + fk]);
#pragma unroll
            for (int pl = 0; pl < NPL; pl++) {
                half8_t af[4];
#pragma unroll
                for (int t = 0; t < 4; t++)
                    af[t] = *reinterpret_cast<const half8_t *>(&As[buf][pl][(wm * 64 + t * 16 + fr) * ROW + ks + fk]);
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        accg[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], accg[i][j], 0, 0, 0);
            }
        }
        if ((st + 1) % SPG == 0) {   // group end: acc += s * accg (column lane & 15 of tile j)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float sj = Ss[buf][wn * 64 + j * 16 + fr];
#pragma unroll
                for (int i = 0; i < 4; i++) {
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][j][r] = __builtin_fmaf(sj, accg[i][j][r], acc[i][j][r]);
                    accg[i][j] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
        }
    };
    StageRegs rg;
    if (s_begin < s_end) {
        load_stage(s_begin, rg);
        store_stage(0, rg);
        __syncthreads();
    }
    for (int st = s_begin; st < s_end; st++) {
        const int buf = (st - s_begin) & 1;
        const bool more = st + 1 < s_end;
        if (more) load_stage(st + 1, rg);
        compute_stage(st, buf);
        if (more) store_stage(buf ^ 1, rg);
        __syncthreads();
    }

    // D of tile (i, j): lane holds rows 4*(lane>>4) + r, column lane & 15
    const int rbase = m0 + wm * 64 + 4 * (lane >> 4);
    const int mat = NMAT == 2 ? wn : 0;
    const int cbase = n0 + (NMAT == 2 ? 0 : wn * 64) + (lane & 15);
    if (part) {   // split-K partials, both matrices side by side
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int n = cbase + j * 16;
                if (n >= N) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = rbase + i * 16 + r;
                    if (m < M) part[((size_t)blockIdx.z * M + m) * NMAT * N + (size_t)mat * N + n] = acc[i][j][r];
                }
            }
        return;
    }
    if (NMAT == 2 && epi != GE_STORE) {
        // up (waves wn = 1) hands its accumulators to gate (wn = 0) through
        // LDS, which the stages no longer use
        float4_t *xch = reinterpret_cast<float4_t *>(&As[0][0][0]);
        if (wn == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) xch[((wm * 16) + i * 4 + j) * 64 + lane] = acc[i][j];
        }
        __syncthreads();
        if (wn == 1) return;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4_t u = xch[((wm * 16) + i * 4 + j) * 64 + lane];
                const int n = cbase + j * 16;
                if (n >= N) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = rbase + i * 16 + r;
                    if (m < M) mats.out[0][(size_t)m * N + n] = __float2half(gate_act(acc[i][j][r], u[r], epi));
                }
            }
        return;
    }
    __half *o = mat ? mats.out[1] : mats.out[0];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = cbase + j * 16;
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = rbase + i * 16 + r;
                if (m < M) o[(size_t)m * N + n] = __float2half(acc[i][j][r]);
            }
        }
}

// The AWQ activation planes: hi = f16(x / awq), lo = f16(x / awq - hi), each
// 8-element chunk in slot order {0, 2, 4, 6, 1, 3, 5, 7}.  grid (M,
// ceil(K/8 / 256)), block 256: one chunk per thread.
__global__ void __launch_bounds__(256) int4_gemm_prep_kernel(const __half *__restrict__ x,
                                                             const __half *__restrict__ awq,
                                                             __half *__restrict__ hi_out,
                                                             __half *__restrict__ lo_out, int K) {
    const int c = blockIdx.y * blockDim.x + threadIdx.x;
    if (c * 8 >= K) return;
    const size_t off = (size_t)blockIdx.x * K + (size_t)c * 8;
    const u32x4_t xv = *reinterpret_cast<const u32x4_t *>(x + off);
    const u32x4_t wv = *reinterpret_cast<const u32x4_t *>(awq + (size_t)c * 8);
    const _Float16 *xh = reinterpret_cast<const _Float16 *>(&xv);
    const _Float16 *wh = reinterpret_cast<const _Float16 *>(&wv);
    half8_t hi, lo;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float v = (float)xh[j] * __builtin_amdgcn_rcpf((float)wh[j]);
        hi[j] = (_Float16)v;
        lo[j] = (_Float16)(v - (float)hi[j]);
    }
    auto slot_order = [](u32x4_t v) {
        return (u32x4_t){__builtin_amdgcn_perm(v[1], v[0], 0x05040100u), __builtin_amdgcn_perm(v[3], v[2], 0x05040100u),
                         __builtin_amdgcn_perm(v[1], v[0], 0x07060302u), __builtin_amdgcn_perm(v[3], v[2], 0x07060302u)};
    };
    *reinterpret_cast<u32x4_t *>(hi_out + off) = slot_order(__builtin_bit_cast(u32x4_t, hi));
    *reinterpret_cast<u32x4_t *>(lo_out + off) = slot_order(__builtin_bit_cast(u32x4_t, lo));
}

// Sum the split partials in split order, then store (or, for a gate/up pair,
// apply the activation): grid ceil(M*N / 256), block 256.
__global__ void __launch_bounds__(256) int4_gemm_reduce_kernel(const float *__restrict__ part, int splits,
                                                               int M, int N, int nmat, int epi,
                                                               __half *__restrict__ out0,
                                                               __half *__restrict__ out1) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t count = (size_t)M * N;
    if (i >= count) return;
    const size_t m = i / N, n = i - m * N;
    const size_t stride = (size_t)M * nmat * N;
    float v[2] = {0.0f, 0.0f};
    for (int t = 0; t < nmat; t++) {
        const size_t at = m * nmat * N + (size_t)t * N + n;
        float s = part[at];
        for (int z = 1; z < splits; z++) s += part[(size_t)z * stride + at];
        v[t] = s;
    }
    if (nmat == 2 && epi != GE_STORE) {
        out0[i] = __float2half(gate_act(v[0], v[1], epi));
    } else {
        out0[i] = __float2half(v[0]);
        if (nmat == 2) out1[i] = __float2half(v[1]);
    }
}

// Residual + RMSNorm rows (the prefill path and the 3-8-row decode FFN):
// grid (B), block 256.  residual_out = f16(a + b), normed_out = f16((a + b) *
// rms_inv * gamma).  Thread t takes chunks t, t + 256, ..: the first CPT of
// them are loaded before the reduction and stay in registers (all of them for
// K <= 2048 CPT); chunks past those are read again after it.
template <int CPT>
__global__ void __launch_bounds__(256) resnorm_rows_kernel(const __half *__restrict__ a,
                                                           const __half *__restrict__ b,
                                                           const __half *__restrict__ gamma, float eps,
                                                           __half *__restrict__ residual_out,
                                                           __half *__restrict__ normed_out, int K) {
    __shared__ float red[256];
    __shared__ float rms_s;
    const size_t row = (size_t)blockIdx.x * K;
    const int nchunk = K / 8;
    const int iters = (nchunk + 255) / 256;
    uint4 av[CPT], bv[CPT], gv[CPT];
#pragma unroll
    for (int it = 0; it < CPT; it++) {
        const int c_raw = it * 256 + (int)threadIdx.x;
        const int c = c_raw < nchunk ? c_raw : 0;
        av[it] = *reinterpret_cast<const uint4 *>(a + row + (size_t)c * 8);
        bv[it] = *reinterpret_cast<const uint4 *>(b + row + (size_t)c * 8);
        gv[it] = *reinterpret_cast<const uint4 *>(gamma + (size_t)c * 8);
    }
    float sq = 0.0f;
    auto add_sq = [&](const uint4 &x, const uint4 &y) __attribute__((always_inline)) {
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&x);
        const _Float16 *bh = reinterpret_cast<const _Float16 *>(&y);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float r = (float)ah[i] + (float)bh[i];
            sq = __builtin_fmaf(r, r, sq);
        }
    };
#pragma unroll
    for (int it = 0; it < CPT; it++)
        if (it * 256 + (int)threadIdx.x < nchunk) add_sq(av[it], bv[it]);
    for (int it = CPT; it < iters; it++) {
        const int c = it * 256 + (int)threadIdx.x;
        if (c < nchunk)
            add_sq(*reinterpret_cast<const uint4 *>(a + row + (size_t)c * 8),
                   *reinterpret_cast<const uint4 *>(b + row + (size_t)c * 8));
    }
    const float rms_inv = imh_int4::block_rms_inv(sq, red, &rms_s, K, eps);
    auto emit = [&](int c, const uint4 &x, const uint4 &y, const uint4 &gw) __attribute__((always_inline)) {
        const size_t off = row + (size_t)c * 8;
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&x);
        const _Float16 *bh = reinterpret_cast<const _Float16 *>(&y);
        const _Float16 *gh = reinterpret_cast<const _Float16 *>(&gw);
        half8_t res, nrm;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float r = (float)ah[i] + (float)bh[i];
            res[i] = (_Float16)r;
            nrm[i] = (_Float16)(r * rms_inv * (float)gh[i]);
        }
        *reinterpret_cast<half8_t *>(residual_out + off) = res;
        *reinterpret_cast<half8_t *>(normed_out + off) = nrm;
    };
#pragma unroll
    for (int it = 0; it < CPT; it++) {
        const int c = it * 256 + (int)threadIdx.x;
        if (c < nchunk) emit(c, av[it], bv[it], gv[it]);
    }
    for (int it = CPT; it < iters; it++) {
        const int c = it * 256 + (int)threadIdx.x;
        if (c < nchunk)
            emit(c, *reinterpret_cast<const uint4 *>(a + row + (size_t)c * 8),
                 *reinterpret_cast<const uint4 *>(b + row + (size_t)c * 8),
                 *reinterpret_cast<const uint4 *>(gamma + (size_t)c * 8));
    }
}

}  // namespace

namespace imh_int4 {

// K splits (whole groups each, at least 4 per split), only as many as keep
// the grid within one round of workgroup slots (two per CU).  Each
// workgroup costs about the same per group (~3.2 us at two per CU, ~0.9 of
// that alone on a CU), and a split adds its partials' round trip (read back
// by the reduce launch at ~4.5 TB/s plus ~2 us).  The rule this replaces
// split tile grids under the CU count into as many splits as fill two per
// CU, rounded up -- a second round of a few workgroups, e.g. at K 9728 ->
// N 2560, M = 512 (80 tiles, 7 splits = 560 workgroups on 512 slots).  The
// bf16 / fp8 GEMM measured the same overfill 12-19 % slower.
int gemm_splits(int M, int N, int K, int nmat, int cus) {
    const int tiles = ((M + kBM - 1) / kBM) * ((N + kBN / nmat - 1) / (kBN / nmat));
    const int G = K / kGS;
    if (tiles >= 2 * cus || G < 8) return 1;
    constexpr double g2 = 3.2;
    auto grid_us = [&](long long W, int per) {
        double us = 0.0;
        for (; W > 2 * cus; W -= 2 * cus) us += per * g2;
        return us + per * (W > cus ? g2 : 0.9 * g2);
    };
    int best = 1;
    double best_us = grid_us(tiles, G);
    for (int sp = 2; sp <= G / 4 && (long long)tiles * sp <= 2 * cus; sp++) {
        const int per = (G + sp - 1) / sp;
        if ((G + per - 1) / per != sp) continue;
        const double us = grid_us((long long)tiles * sp, per) +
                          ((double)sp * M * nmat * N * 4 + (double)M * nmat * N * 2) / 4.5e6 + 2.0;
        if (us < best_us * 0.98) {
            best_us = us;
            best = sp;
        }
    }
    return best;
}

size_t gemm_workspace_bytes(int M, int N, int K, int nmat, int cus) {
    const int splits = gemm_splits(M, N, K, nmat, cus);
    return splits > 1 ? (size_t)splits * M * nmat * N * sizeof(float) : 0;
}

int encode_gemm(imh_stream *s, const __half *x, int M, const imh_affine_int4_weight *w0,
                const imh_affine_int4_weight *w1, int epi, __half *y0, __half *y1, void *workspace) {
    const int N = (int)w0->n, K = (int)w0->k;
    const int nmat = w1 ? 2 : 1;
    const int cus = s->dev->props.multiProcessorCount;
    const int splits = gemm_splits(M, N, K, nmat, cus);
    const int bk = w0->awq_scales ? kBK / 2 : kBK;
    const int stages = K / bk;
    const int spg = kGS / bk;                                   // splits end on group boundaries
    const int per = ((stages + splits - 1) / splits + spg - 1) / spg * spg;
    dim3 grid((N + kBN / nmat - 1) / (kBN / nmat), (M + kBM - 1) / kBM, splits);
    float *part = splits == 1 ? nullptr : static_cast<float *>(workspace);
    if (splits > 1 && !part) return imh::fail(IMH_EINVAL, "int4 gemm: split-K workspace missing");
    GemmMats mats = {};
    const imh_affine_int4_weight *ws[2] = {w0, w1 ? w1 : w0};
    for (int i = 0; i < 2; i++) {
        mats.data[i] = ws[i]->data;
        mats.scales[i] = reinterpret_cast<const __half *>(ws[i]->scales);
        mats.zeros[i] = reinterpret_cast<const __half *>(ws[i]->zeros);
    }
    mats.out[0] = y0;
    mats.out[1] = y1;
    // both matrices of a pair divide x by the first one's awq scales; the
    // hi / lo planes of x / awq are built once, into stream scratch slot 0
    const __half *awq = reinterpret_cast<const __half *>(w0->awq_scales);
    const __half *xa = x, *xlo = nullptr;
    if (awq) {
        void *planes = nullptr;
        int rc = imh::stream_scratch(s, 0, (size_t)M * K * 2 * sizeof(__half), &planes);
        if (rc) return rc;
        __half *hi = static_cast<__half *>(planes), *lo = hi + (size_t)M * K;
        hipLaunchKernelGGL(int4_gemm_prep_kernel, dim3(M, (K / 8 + 255) / 256), dim3(256), 0, s->stream, x, awq, hi,
                           lo, K);
        IMH_HIP(hipGetLastError());
        xa = hi;
        xlo = lo;
    }
    const int ge = epi == 2 ? GE_SILU : epi == 3 ? GE_GELU : GE_STORE;
#define IMH_GEMM(A, NM)                                                                                        \
    hipLaunchKernelGGL((int4_gemm_kernel<A, NM>), grid, dim3(kThreads), 0, s->stream, xa, xlo, mats, ge, part, M, \
                       N, K, per)
    if (awq) {
        if (nmat == 2) IMH_GEMM(true, 2);
        else IMH_GEMM(true, 1);
    } else {
        if (nmat == 2) IMH_GEMM(false, 2);
        else IMH_GEMM(false, 1);
    }
#undef IMH_GEMM
    IMH_HIP(hipGetLastError());
    if (splits > 1) {
        const size_t count = (size_t)M * N;
        hipLaunchKernelGGL(int4_gemm_reduce_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s->stream,
                           part, splits, M, N, nmat, ge, y0, y1);
        IMH_HIP(hipGetLastError());
    }
    return IMH_OK;
}

int encode_resnorm_rows(imh_stream *s, const __half *a, const __half *b, const __half *gamma, float eps,
                        __half *residual_out, __half *normed_out, int B, int K) {
    const int cpt = resnorm_cpt(K);
    auto kern = cpt == 1 ? resnorm_rows_kernel<1>
                : cpt == 2 ? resnorm_rows_kernel<2>
                : cpt == 4 ? resnorm_rows_kernel<4>
                           : resnorm_rows_kernel<8>;
    hipLaunchKernelGGL(kern, dim3(B), dim3(256), 0, s->stream, a, b, gamma, eps, residual_out, normed_out, K);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

}  // namespace imh_int4
