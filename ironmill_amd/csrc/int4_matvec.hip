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
//  * the contraction runs on the matrix cores: v_mfma_f32_16x16x32_f16 with
//    the activation as operand A (16 batch rows; rows past the batch read
//    row 0 and their results are dropped) and the weights as operand B (16
//    weight rows).  (q - z) is formed exactly in f16: nibbles are split into
//    bytes, v_perm_b32 places each beside a 0x64 exponent byte (1024 + q), and
//    one packed f16 add of -(1024 + z) gives (q - z) -- every product is exact,
//    the accumulation is f32.
//  * an activation that is not exactly f16 (x/awq, normed values) is split
//    into hi + lo f16 halves and fed through two MFMAs: ~22-bit operands.
//  * one workgroup owns one 16-row tile (of each matrix of a gate/up pair);
//    its waves split K, each holding all of its slice's weights in registers
//    (one 16-byte load per lane per 128-element group, issued up front), and
//    reduce through LDS in a fixed order: deterministic, no cross-workgroup
//    synchronisation.
//  * the activation image is staged into LDS by the whole workgroup, with its
//    loads issued before the weight loads and an LDS-only barrier, so the
//    weights stay in flight while the first groups compute.
//  * a small prep kernel writes the activation in MFMA operand order: slot i
//    of each 8-element chunk holds element {0,2,4,6,1,3,5,7}[i], the order in
//    which the nibble unpack produces weights.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <string>

#include "imh_internal.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGS = 128;       // group size the kernels are built for
constexpr int kMaxGroups = 8;    // groups one wave holds per stage (weights stay in registers)
constexpr int kMaxWaves = 16;    // waves per workgroup
constexpr int kSZChunks = 2;     // scale/zero pairs per thread loaded ahead of the weights
constexpr int kLdsBudget = 64 * 1024;

enum Epi : int { EPI_STORE = IMH_EPI_STORE, EPI_SILU = IMH_EPI_SILU, EPI_GELU = IMH_EPI_GELU };

struct MatPtrs {
    const uint8_t *data[2];
    const __half *scales[2];
    const __half *zeros[2];
    __half *out[2];
};

__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

// Split v into f16 hi + lo with hi + lo == v to ~22 bits.
__device__ __forceinline__ void split_hilo(float v, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// ---------------------------------------------------------------------------
// prep: activation -> MFMA operand image
// ---------------------------------------------------------------------------
// Plain mode.  grid (ceil(K/8/256), B), block 256; thread = one 8-element chunk.
__global__ void __launch_bounds__(256) int4_prep_plain(const __half *__restrict__ x,
                                                        const __half *__restrict__ awq,
                                                        _Float16 *__restrict__ xa_hi,
                                                        _Float16 *__restrict__ xa_lo, int K) {
    const int m = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c * 8 >= K) return;
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
    constexpr int perm[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    half8_t hi, lo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        _Float16 h, l;
        split_hilo(v[perm[i]], h, l);
        hi[i] = h;
        lo[i] = l;
    }
    *reinterpret_cast<half8_t *>(xa_hi + base) = hi;
    if (xa_lo) *reinterpret_cast<half8_t *>(xa_lo + base) = lo;
}

// Residual + RMSNorm mode.  grid (B), block 256: r = a + b, rms_inv, writes
// residual_out / normed_out and the operand image of r * gamma / awq.
__global__ void __launch_bounds__(256) int4_prep_resnorm(
    const __half *__restrict__ a, const __half *__restrict__ b, const __half *__restrict__ gamma,
    const __half *__restrict__ awq, float eps, __half *__restrict__ residual_out,
    __half *__restrict__ normed_out, _Float16 *__restrict__ xa_hi, _Float16 *__restrict__ xa_lo,
    float *__restrict__ rms_out, int K) {
    const int m = blockIdx.x;
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
    constexpr int perm[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    for (int c = threadIdx.x; c * 8 < K; c += blockDim.x) {
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
        *reinterpret_cast<half8_t *>(residual_out + off) = res;
        *reinterpret_cast<half8_t *>(normed_out + off) = nrm;
        half8_t hi, lo;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            _Float16 h, l;
            split_hilo(v[perm[i]], h, l);
            hi[i] = h;
            lo[i] = l;
        }
        *reinterpret_cast<half8_t *>(xa_hi + off) = hi;
        *reinterpret_cast<half8_t *>(xa_lo + off) = lo;
    }
}

// ---------------------------------------------------------------------------
// main matvec kernel
// ---------------------------------------------------------------------------
// grid (ceil(N/16), ceil(B/16)), block 64 * NMAT * parts.  Wave w works on
// matrix w / parts and, in every K stage, on part w % parts of the stage's
// groups (at most NG of them).  A stage is the range of groups whose
// activation image fits the LDS budget (normally all of K: one stage).
// XC activation chunks per thread are loaded ahead of the weights (the rest,
// if any, after them).
//
// Issue order matters: vector-memory loads of a wave complete in order, so
// the small loads the LDS staging needs (scales/zeros, activation) are issued
// first and the weight loads right after them, before anything waits.  The
// first stage is peeled so that no loop-carried wait sits ahead of the first
// weight loads.
template <int NMAT, int EPI, bool HAS_LO, int NG, int XC>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu((NG < 5 || (NG == 5 && XC == 1)) ? 6 : 5)))
int4_matvec_kernel(
    MatPtrs mp, const _Float16 *__restrict__ xa_hi, const _Float16 *__restrict__ xa_lo,
    const float *__restrict__ rms_inv, int N, int K, int B, int parts, int SG) {
    // dynamic LDS: [NMAT][16][G + 1] u32 (scale | zero << 16), the activation
    // planes ([min(B,16)][SG*128 + 8] f16, hi then lo), then [waves][64] float4
    // partial sums
    extern __shared__ __attribute__((aligned(16))) uint32_t lds_dyn[];

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int mat = wave / parts;
    const int part = wave - mat * parts;
    const int G = K / kGS;
    const int m0 = blockIdx.y * 16;
    const int bc = min(16, B - m0);
    const int RSX = SG * kGS + 8;        // LDS row stride in halfs (16-byte pad)

    const int n_l = lane & 15;           // weight row within the tile (B operand column)
    const int kq = lane >> 4;            // 16-byte quarter of a group this lane reads
    const int row0 = blockIdx.x * 16;
    const int row = row0 + n_l;
    const int row_c = row < N ? row : N - 1;
    const int arow = n_l < bc ? n_l : 0; // rows past the batch reuse row 0; dropped below

    // matrix pointers by select: a dynamic index into the kernel-argument
    // struct would turn into dependent memory loads
    const uint8_t *wdata = (NMAT == 2 && mat) ? mp.data[1] : mp.data[0];
    const uint8_t *wrow = wdata + (size_t)row_c * (K / 2) + kq * 16;
    const uint32_t c64 = 0x64646464u;

    const int SZR = G + 1;                                   // LDS row stride (u32)
    uint32_t *szs = lds_dyn;
    _Float16 *xs = reinterpret_cast<_Float16 *>(lds_dyn + ((NMAT * 16 * SZR + 3) & ~3));
    float4_t *red = reinterpret_cast<float4_t *>(xs + (HAS_LO ? 2 : 1) * min(B, 16) * RSX);

    // scales and zeros of the tile: per matrix one contiguous run of 16 * G
    // halfs starting at row0 * G (elements past the last row clamp to it;
    // their rows are never stored)
    const int per_mat = 16 * G;
    const int sz_total = NMAT * per_mat;
    const size_t sz_last = (size_t)N * G - 1;
    // element e of the tile's scales/zeros: source offset, arrays, LDS slot
    auto sz_elem = [&](int e, const uint16_t *&sp, const uint16_t *&zp, int &dst) {
        const bool second = NMAT == 2 && e >= per_mat;
        const int el = second ? e - per_mat : e;
        sp = reinterpret_cast<const uint16_t *>(second ? mp.scales[1] : mp.scales[0]);
        zp = reinterpret_cast<const uint16_t *>(second ? mp.zeros[1] : mp.zeros[0]);
        const int rr = el / G;
        dst = ((second ? 16 : 0) + rr) * SZR + (el - rr * G);
        return min((size_t)row0 * G + el, sz_last);
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

    float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
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
            if (HAS_LO) lv[i] = *reinterpret_cast<const u32x4_t *>(xa_lo + src);
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
        // (c) scales/zeros -> LDS (first stage only; read after the barrier below)
        // Writes are unconditional: threads past the end rewrite the last
        // element with its own value, so the compiler has no branch to sink
        // the loads into (behind a wait for the weights).
        if (first) {
#pragma unroll
            for (int i = 0; i < kSZChunks; i++) szs[sd[i]] = sv[i] | (zv[i] << 16);
            for (int e = kSZChunks * nthr + tid; e < sz_total; e += nthr) {
                const uint16_t *sp, *zp;
                int dst;
                const size_t src = sz_elem(e, sp, zp, dst);
                szs[dst] = (uint32_t)sp[src] | ((uint32_t)zp[src] << 16);
            }
        } else {
            // the previous stage is done with the activation planes
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        }
        // (d) activation -> LDS
#pragma unroll
        for (int i = 0; i < XC; i++) {
            const int c = min(i * nthr + tid, total - 1);
            const int r = c / cpr;
            const int off = r * RSX + (c - r * cpr) * 8;
            *reinterpret_cast<u32x4_t *>(xs + off) = xv[i];
            if (HAS_LO) *reinterpret_cast<u32x4_t *>(xs + bc * RSX + off) = lv[i];
        }
        for (int c = XC * nthr + tid; c < total; c += nthr) {  // activation beyond XC chunks
            const int r = c / cpr;
            const size_t src = (size_t)(m0 + r) * K + (size_t)gs0 * kGS + (size_t)(c - r * cpr) * 8;
            const int off = r * RSX + (c - r * cpr) * 8;
            *reinterpret_cast<u32x4_t *>(xs + off) = *reinterpret_cast<const u32x4_t *>(xa_hi + src);
            if (HAS_LO)
                *reinterpret_cast<u32x4_t *>(xs + bc * RSX + off) = *reinterpret_cast<const u32x4_t *>(xa_lo + src);
        }
        // LDS-only barrier: the weight loads stay in flight across it
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

        // (e) MFMA over the wave's groups
        const _Float16 *xh = xs + arow * RSX + (wg0 - gs0) * kGS + kq * 32;
        const _Float16 *xl = xh + bc * RSX;
#pragma unroll
        for (int i = 0; i < NG; i++) {
            if (i < ng) {
                const uint32_t sz = szs[(mat * 16 + n_l) * SZR + wg0 + i];
                const float zf = (float)__builtin_bit_cast(_Float16, (uint16_t)(sz >> 16));
                const _Float16 nb = (_Float16)(-(1024.0f + zf));
                const half2_t bias = {nb, nb};
                float4_t accg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const half8_t ah = *reinterpret_cast<const half8_t *>(xh + i * kGS + j * 8);
                    const uint32_t w = wq[i][j];
                    const uint32_t lo = w & 0x0F0F0F0Fu;          // q0 q2 q4 q6
                    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // q1 q3 q5 q7
                    const half2_t p0 = as_h2(__builtin_amdgcn_perm(lo, c64, 0x00050004u)) + bias;
                    const half2_t p1 = as_h2(__builtin_amdgcn_perm(lo, c64, 0x00070006u)) + bias;
                    const half2_t p2 = as_h2(__builtin_amdgcn_perm(hi, c64, 0x00050004u)) + bias;
                    const half2_t p3 = as_h2(__builtin_amdgcn_perm(hi, c64, 0x00070006u)) + bias;
                    const half8_t bq = __builtin_bit_cast(
                        half8_t, (u32x4_t){as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)});
                    accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq, accg, 0, 0, 0);
                    if (HAS_LO) {
                        const half8_t al = *reinterpret_cast<const half8_t *>(xl + i * kGS + j * 8);
                        accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq, accg, 0, 0, 0);
                    }
                }
                const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)(sz & 0xFFFFu));
#pragma unroll
                for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(accg[r], s, acc[r]);
            }
        }
    };
    stage(0, true);
    for (int gs0 = SG; gs0 < G; gs0 += SG) stage(gs0, false);

    // reduce the parts of each matrix in part order.  Lane l holds
    // D[m = 4*(l>>4) + r][n = l & 15].
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    float4_t sum[NMAT];
#pragma unroll
    for (int mt = 0; mt < NMAT; mt++) {
        sum[mt] = red[mt * parts * 64 + lane];
        for (int p = 1; p < parts; p++) sum[mt] += red[(mt * parts + p) * 64 + lane];
    }
    if (row >= N) return;
    const int mrow = m0 + 4 * (lane >> 4);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = mrow + r;
        if (m >= B) break;
        const float scale = rms_inv ? rms_inv[m] : 1.0f;
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

size_t act_bytes(uint32_t B, uint32_t K) { return (size_t)B * K * 4 + (size_t)B * 4 + 256; }

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

// Groups per K stage: as many as the LDS budget holds for the batch rows.
int pick_stage(int G, int B, bool lo, int parts) {
    const int rows = std::min(B, 16);
    const int per_group = rows * kGS * 2 * (lo ? 2 : 1);
    int SG = std::max(1, (kLdsBudget - 64) / per_group);
    SG = std::min(SG, parts * kMaxGroups);
    return std::min(SG, G);
}

int prep_plain(imh_stream *s, const uint16_t *x, uint32_t B, uint32_t K, const uint16_t *awq,
               void *storage, imh_int4_activation *act) {
    if (misaligned16(x) || misaligned16(awq) || misaligned16(storage))
        return imh::fail(IMH_EINVAL, "int4 activation: x, awq and storage must be 16-byte aligned");
    _Float16 *hi = static_cast<_Float16 *>(storage);
    _Float16 *lo = awq ? hi + (size_t)B * K : nullptr;
    dim3 grid((K / 8 + 255) / 256, B);
    hipLaunchKernelGGL(int4_prep_plain, grid, dim3(256), 0, s->stream,
                       reinterpret_cast<const __half *>(x), reinterpret_cast<const __half *>(awq),
                       hi, lo, (int)K);
    IMH_HIP(hipGetLastError());
    act->hi = reinterpret_cast<const uint16_t *>(hi);
    act->lo = reinterpret_cast<const uint16_t *>(lo);
    act->row_scale = nullptr;
    act->token_count = B;
    act->k = K;
    return IMH_OK;
}

template <int NMAT, int EPI, bool HAS_LO>
int launch_main(imh_stream *s, const MatPtrs &mp, const imh_int4_activation *act, int N) {
    const int K = (int)act->k, B = (int)act->token_count;
    const int G = K / kGS;
    const int tiles = (N + 15) / 16;
    const int btiles = (B + 15) / 16;
    const int parts = pick_parts(tiles * btiles, NMAT, G, s->dev->props.multiProcessorCount);
    const int SG = pick_stage(G, B, HAS_LO, parts);
    const int ng = (SG + parts - 1) / parts;  // most groups a wave takes in one stage
    const int waves = NMAT * parts;
    const size_t sz_words = ((size_t)NMAT * 16 * (G + 1) + 3) & ~(size_t)3;
    const size_t lds = sz_words * sizeof(uint32_t) +
                       (size_t)(HAS_LO ? 2 : 1) * std::min(B, 16) * (SG * kGS + 8) * sizeof(_Float16) +
                       (size_t)waves * 64 * sizeof(float4_t);
    dim3 grid(tiles, btiles), block(64 * waves);
    const _Float16 *hi = reinterpret_cast<const _Float16 *>(act->hi);
    const _Float16 *lo = reinterpret_cast<const _Float16 *>(act->lo);
    const bool one_chunk = std::min(B, 16) * SG * 16 <= 64 * waves;  // activation chunks per thread
#define IMH_NG(NGV)                                                                                        \
    do {                                                                                                   \
        if (one_chunk)                                                                                     \
            hipLaunchKernelGGL((int4_matvec_kernel<NMAT, EPI, HAS_LO, NGV, 1>), grid, block, lds, s->stream, \
                               mp, hi, lo, act->row_scale, N, K, B, parts, SG);                           \
        else                                                                                               \
            hipLaunchKernelGGL((int4_matvec_kernel<NMAT, EPI, HAS_LO, NGV, 2>), grid, block, lds, s->stream, \
                               mp, hi, lo, act->row_scale, N, K, B, parts, SG);                           \
    } while (0)
    if (ng <= 2) IMH_NG(2);
    else if (ng <= 3) IMH_NG(3);
    else if (ng <= 4) IMH_NG(4);
    else if (ng <= 5) IMH_NG(5);
    else if (ng <= 6) IMH_NG(6);
    else IMH_NG(8);
#undef IMH_NG
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
    if (!act || !act->hi || !out0 || (w1 && epi == EPI_STORE && !out1))
        return imh::fail(IMH_EINVAL, std::string(who) + ": NULL activation or output");
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
    const bool lo = act->lo != nullptr;
#define IMH_MV(NM, EP) \
    return lo ? launch_main<NM, EP, true>(s, mp, act, N) : launch_main<NM, EP, false>(s, mp, act, N)
    if (!w1) IMH_MV(1, EPI_STORE);
    if (epi == EPI_SILU) IMH_MV(2, EPI_SILU);
    if (epi == EPI_GELU) IMH_MV(2, EPI_GELU);
    IMH_MV(2, EPI_STORE);
#undef IMH_MV
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
    out->hi = static_cast<const uint16_t *>(storage);
    out->lo = nullptr;
    out->row_scale = nullptr;
    out->token_count = token_count;
    out->k = k;
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
    _Float16 *hi = static_cast<_Float16 *>(scr);
    _Float16 *lo = hi + (size_t)B * K;
    float *rms = reinterpret_cast<float *>(lo + (size_t)B * K);
    hipLaunchKernelGGL(int4_prep_resnorm, dim3(B), dim3(256), 0, stream->stream,
                       reinterpret_cast<const __half *>(p->a), reinterpret_cast<const __half *>(p->b),
                       reinterpret_cast<const __half *>(p->norm_weight),
                       reinterpret_cast<const __half *>(p->weight->awq_scales), p->eps,
                       reinterpret_cast<__half *>(p->residual_output),
                       reinterpret_cast<__half *>(p->normed_output), hi, lo, rms, (int)K);
    IMH_HIP(hipGetLastError());
    imh_int4_activation act;
    act.hi = reinterpret_cast<const uint16_t *>(hi);
    act.lo = reinterpret_cast<const uint16_t *>(lo);
    act.row_scale = rms;
    act.token_count = B;
    act.k = K;
    return run_matvec(stream, &act, p->weight, nullptr, EPI_STORE, p->output, nullptr, who);
}

}  // extern "C"
