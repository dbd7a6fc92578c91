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
//    the activation as operand A (16 batch rows, unused rows zero) and the
//    weights as operand B (16 weight rows).  (q - z) is formed exactly in f16
//    from the nibbles with the 0x6400 exponent trick and one packed f16 add, so
//    every product is exact and the accumulation is f32.
//  * an activation that is not exactly f16 (x/awq, normed values) is split
//    into hi + lo f16 halves and fed through two MFMAs: ~22-bit operands.
//  * one 16-byte load per lane covers a whole 128-element group of one row
//    (the 4 lane groups of a wave read the 64 bytes of the group), and every
//    group a wave owns is loaded before the first MFMA, so each wave keeps its
//    whole K slice of weights in flight.
//  * a workgroup owns one 16-row tile; its waves split K (and gate/up) and
//    reduce through LDS in a fixed order, so results are deterministic and no
//    cross-workgroup synchronisation is needed.
//  * the activation is first rewritten by a small prep kernel into the MFMA
//    operand order (k-slot i of an 8-chunk holds element {0,4,1,5,2,6,3,7}[i]),
//    which matches the nibble pairs (q_i, q_{i+4}) the B operand is built from.
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
constexpr int kMaxGroups = 10; // groups one item may own (its weights stay in registers)

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
    constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
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
    constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
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
// grid (tiles * S, ceil(B/16)), block 64: one wave per item.  Item = 16 weight
// rows of each of the NMAT matrices x the K range of split `s` (kc groups).
//   1. every weight load of the item is issued (NMAT * kc 16-byte loads/lane);
//   2. the wave copies its activation slice (<= 16 batch rows x kc*128, hi and
//      lo planes) into LDS, so all activation misses overlap in one round trip;
//   3. per group: operand B from the nibbles, operand A from LDS, MFMAs, and
//      the group's f32 partial is scaled by s into the running accumulator;
//   4. with S > 1 the item stores its partial; the last item of a tile to
//      arrive (atomic counter) sums the S partials in split order -- the same
//      order on every run -- applies the epilogue and re-arms the counter.
template <int NMAT, int EPI, bool HAS_LO>
__global__ void __launch_bounds__(64) int4_matvec_kernel(
    MatPtrs mp, const _Float16 *__restrict__ xa_hi, const _Float16 *__restrict__ xa_lo,
    const float *__restrict__ rms_inv, int N, int K, int B, int S, int kc,
    float *__restrict__ partial, unsigned *__restrict__ counters) {
    extern __shared__ __attribute__((aligned(16))) _Float16 xs[];

    const int lane = threadIdx.x;
    const int G = K / kGS;
    const int item = blockIdx.x;
    const int tile = item / S;
    const int split = item - tile * S;
    const int g0 = split * kc;
    const int ng = min(g0 + kc, G) - g0;
    const int m0 = blockIdx.y * 16;
    const int bc = min(16, B - m0);
    const int RS = kc * kGS + 8;          // LDS row stride in halfs (16-byte pad)

    const int n_l = lane & 15;            // weight row within the tile (B operand column)
    const int kq = lane >> 4;             // 16-byte quarter of a group this lane reads
    const int row = tile * 16 + n_l;
    const int row_c = row < N ? row : N - 1;

    // 1. weights, scales, zeros of the whole item
    u32x4_t wq[NMAT][kMaxGroups];
    _Float16 sc[NMAT][kMaxGroups], zr[NMAT][kMaxGroups];
#pragma unroll
    for (int mt = 0; mt < NMAT; mt++) {
        const uint8_t *wrow = mp.data[mt] + (size_t)row_c * (K / 2) + kq * 16;
        const _Float16 *srow = reinterpret_cast<const _Float16 *>(mp.scales[mt]) + (size_t)row_c * G;
        const _Float16 *zrow = reinterpret_cast<const _Float16 *>(mp.zeros[mt]) + (size_t)row_c * G;
#pragma unroll
        for (int i = 0; i < kMaxGroups; i++) {
            if (i < ng) {
                const int g = g0 + i;
                wq[mt][i] = *reinterpret_cast<const u32x4_t *>(wrow + (size_t)g * 64);
                sc[mt][i] = srow[g];
                zr[mt][i] = zrow[g];
            }
        }
    }

    // 2. activation slice -> LDS (hi plane, then lo plane)
    {
        const int per_row = ng * 16;      // 8-half chunks per batch row
        const int chunks = bc * per_row;
        for (int c = lane; c < chunks; c += 64) {
            const int r = c / per_row;
            const int cc = c - r * per_row;
            const size_t src = (size_t)(m0 + r) * K + (size_t)g0 * kGS + (size_t)cc * 8;
            *reinterpret_cast<u32x4_t *>(xs + r * RS + cc * 8) =
                *reinterpret_cast<const u32x4_t *>(xa_hi + src);
            if (HAS_LO)
                *reinterpret_cast<u32x4_t *>(xs + (bc + r) * RS + cc * 8) =
                    *reinterpret_cast<const u32x4_t *>(xa_lo + src);
        }
    }
    __syncthreads();

    // 3. MFMA over the item's groups
    const bool a_on = n_l < bc;
    const _Float16 *xh = xs + n_l * RS + kq * 32;
    const _Float16 *xl = xs + (bc + n_l) * RS + kq * 32;
    float4_t acc[NMAT];
#pragma unroll
    for (int mt = 0; mt < NMAT; mt++) acc[mt] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
    const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < kMaxGroups; i++) {
        if (i < ng) {
            half8_t ah[4], al[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                ah[j] = a_on ? *reinterpret_cast<const half8_t *>(xh + i * kGS + j * 8) : zero8;
                if (HAS_LO) al[j] = a_on ? *reinterpret_cast<const half8_t *>(xl + i * kGS + j * 8) : zero8;
            }
#pragma unroll
            for (int mt = 0; mt < NMAT; mt++) {
                const _Float16 nb = (_Float16)(-(1024.0f + (float)zr[mt][i]));
                const half2_t bias = {nb, nb};
                float4_t accg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t w = wq[mt][i][j];
                    half8_t bq;
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        const uint32_t bits = ((w >> (4 * p)) & 0x000F000Fu) | 0x64006400u;
                        const half2_t d = as_h2(bits) + bias;   // (q_p - z, q_{p+4} - z), exact
                        bq[2 * p] = d[0];
                        bq[2 * p + 1] = d[1];
                    }
                    accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], bq, accg, 0, 0, 0);
                    if (HAS_LO) accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[j], bq, accg, 0, 0, 0);
                }
                const float s = (float)sc[mt][i];
#pragma unroll
                for (int r = 0; r < 4; r++) acc[mt][r] = __builtin_fmaf(accg[r], s, acc[mt][r]);
            }
        }
    }

    // 4. split reduction.  Lane l holds D[m = 4*(l>>4) + r][n = l & 15].
    const int mrow = m0 + 4 * (lane >> 4);
    const size_t NT = (size_t)NMAT * N;
    if (S > 1) {
#pragma unroll
        for (int mt = 0; mt < NMAT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = mrow + r;
                if (m < B && row < N) partial[((size_t)split * B + m) * NT + (size_t)mt * N + row] = acc[mt][r];
            }
        __threadfence();
        unsigned prev = 0;
        unsigned *ctr = counters + (size_t)tile * gridDim.y + blockIdx.y;
        if (lane == 0) prev = atomicAdd(ctr, 1u);
        prev = __shfl(prev, 0);
        if (prev != (unsigned)(S - 1)) return;
        __threadfence();
#pragma unroll
        for (int mt = 0; mt < NMAT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = mrow + r;
                float v = 0.0f;
                if (m < B && row < N) {
                    const float *src = partial + (size_t)m * NT + (size_t)mt * N + row;
                    for (int sp = 0; sp < S; sp++) v += __builtin_nontemporal_load(src + (size_t)sp * B * NT);
                }
                acc[mt][r] = v;
            }
        if (lane == 0) *ctr = 0u;
    }

    // 5. epilogue
    if (row >= N) return;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = mrow + r;
        if (m >= B) break;
        const float scale = rms_inv ? rms_inv[m] : 1.0f;
        if (EPI == EPI_SILU || EPI == EPI_GELU) {
            const float g = acc[0][r], u = acc[NMAT - 1][r];
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
                mp.out[mt][(size_t)m * N + row] = __float2half(acc[mt][r] * scale);
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

// Split of K across items: the activation slice of one item stays within
// ~12 KB of LDS and in kMaxGroups groups of registers, and there are enough
// items (>= ~1100) to spread over the 256 CUs in even rounds.
int pick_kc(int tiles, int G, int B, bool lo) {
    const int rows = std::min(B, 16);
    const int bytes_per_group = rows * kGS * 2 * (lo ? 2 : 1);
    int kc = std::max(1, std::min(kMaxGroups, (12 * 1024) / bytes_per_group));
    const int want_splits = (1100 + tiles - 1) / tiles;
    if (want_splits > 1) kc = std::min(kc, std::max(2, (G + want_splits - 1) / want_splits));
    return std::max(1, std::min(kc, G));
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
    const int kc = pick_kc(tiles, G, B, HAS_LO);
    const int S = (G + kc - 1) / kc;
    const int chunks = (B + 15) / 16;
    float *partial = nullptr;
    unsigned *counters = nullptr;
    if (S > 1) {
        void *p = nullptr;
        int rc = imh::stream_scratch(s, 1, (size_t)S * B * NMAT * N * sizeof(float), &p);
        if (rc) return rc;
        partial = static_cast<float *>(p);
        rc = imh::stream_scratch(s, 2, (size_t)tiles * chunks * sizeof(unsigned), &p);
        if (rc) return rc;
        counters = static_cast<unsigned *>(p);
    }
    const size_t lds = (size_t)(HAS_LO ? 2 : 1) * std::min(B, 16) * (kc * kGS + 8) * sizeof(_Float16);
    dim3 grid(tiles * S, chunks);
    hipLaunchKernelGGL((int4_matvec_kernel<NMAT, EPI, HAS_LO>), grid, dim3(64), lds, s->stream, mp,
                       reinterpret_cast<const _Float16 *>(act->hi),
                       reinterpret_cast<const _Float16 *>(act->lo), act->row_scale, N, K, B, S, kc,
                       partial, counters);
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
