// diag_valu_matvec.hip -- the INT4-affine decode matvec computed the way a
// wavefront-reduction design computes it, for a counter A/B against the MFMA
// kernels (int4_matvec_band.hip, int4_matvec_kernel.h).  Same semantics:
//     y[b][n] = sum_g s[n][g] * (sum_{k in g} xe[b][k] q[n][k] - z[n][g] sum xe),
// xe = x / awq split into f16 hi + lo, f32 accumulation.
//
//  * One workgroup of 8 waves per compute unit owns a band of rows (the
//    row-band kernel's grid); a wave takes slots of 4 rows, 16 lanes per row
//    (one DPP row), lane c reading 16-byte code chunks c, c + 16, ... of its
//    row (coalesced 128-bit loads), the next slot's loads issued before the
//    current slot is computed.
//  * In-register dequant: the nibbles of a code word taken as pairs
//    (e, e + 4) of f16 denormals q * 2^-24 by one shift and one mask, each
//    pair dotted with the matching (hi, lo) activation pairs by
//    v_dot2_f32_f16 (exact products, f32 sums, four independent chains); per
//    chunk the zero point and scale fold: acc += s * (2^24 * t - z * sum xe).
//  * The activation pairs and per-chunk sums of every batch row are staged in
//    LDS once per workgroup; each row's 16 lane sums end in a DPP row sum.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <string>

#include "../../include/ironmill_diag.h"
#include "dpp_reduce.h"
#include "imh_internal.h"

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kMaxB = 8;

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

// LDS: pairs [b][k / 8][hi 4 | lo 4] u32 (pair j of an 8-element block =
// elements (j, j + 4)), then chunk sums [b][k / 32] f32.  NC = k / 512 code
// chunks per lane.
template <int NC>
__global__ void __launch_bounds__(512) diag_valu_matvec_kernel(const __half *__restrict__ x,
                                                              const __half *__restrict__ awq,
                                                              const uint8_t *__restrict__ codes,
                                                              const __half *__restrict__ scales,
                                                              const __half *__restrict__ zeros, int N, int K, int B,
                                                              __half *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds_v[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = K / 128, nblk = K / 8, nchunk = K / 32;
    uint32_t *pairs = lds_v;
    float *csum = reinterpret_cast<float *>(lds_v + (size_t)B * nblk * 8);

    // band of this workgroup, in slots of 4 rows; wave w takes slots w, w + 8, ..
    const int rb = (int)(((int64_t)N * blockIdx.x) / gridDim.x);
    const int re = (int)(((int64_t)N * (blockIdx.x + 1)) / gridDim.x);
    const int nslot = (re - rb + 3) / 4;
    const int c16 = lane & 15;
    struct Slot {
        uint32_t sz[NC];   // s | z << 16
        u32x4_t wv[NC];
    };
    // a slot's scales, zeros and code chunks (rows past the band clamp to its
    // last row and are not stored)
    auto load_slot = [&](int slot, Slot &sl) __attribute__((always_inline)) {
        const int n = min(rb + 4 * min(slot, nslot - 1) + (lane >> 4), re - 1);
        const uint16_t *srow = reinterpret_cast<const uint16_t *>(scales) + (size_t)n * G;
        const uint16_t *zrow = reinterpret_cast<const uint16_t *>(zeros) + (size_t)n * G;
#pragma unroll
        for (int i = 0; i < NC; i++)
            sl.sz[i] = (uint32_t)srow[(c16 + 16 * i) >> 2] | ((uint32_t)zrow[(c16 + 16 * i) >> 2] << 16);
        const u32x4_t *wrow = reinterpret_cast<const u32x4_t *>(codes + (size_t)n * (K / 2));
#pragma unroll
        for (int i = 0; i < NC; i++) sl.wv[i] = wrow[c16 + 16 * i];
    };
    Slot cur, nxt;
    load_slot(wave, cur);

    // stage xe = x / awq: thread handles 8-element blocks; 4 consecutive
    // blocks form one 32-element chunk whose sum goes to csum
    for (int e = tid; e < B * nblk; e += blockDim.x) {
        const int b = e / nblk, blk = e - b * nblk;
        const u32x4_t xv = *reinterpret_cast<const u32x4_t *>(x + (size_t)b * K + (size_t)blk * 8);
        const _Float16 *xh = reinterpret_cast<const _Float16 *>(&xv);
        float v[8];
        if (awq) {
            const u32x4_t av = *reinterpret_cast<const u32x4_t *>(awq + (size_t)blk * 8);
            const _Float16 *ah = reinterpret_cast<const _Float16 *>(&av);
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = (float)xh[j] * __builtin_amdgcn_rcpf((float)ah[j]);
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = (float)xh[j];
        }
        _Float16 hi[8], lo[8];
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            hi[j] = (_Float16)v[j];
            lo[j] = (_Float16)(v[j] - (float)hi[j]);
            s += (float)hi[j] + (float)lo[j];
        }
        uint32_t *dst = pairs + ((size_t)b * nblk + blk) * 8;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            dst[j] = (uint32_t)__builtin_bit_cast(uint16_t, hi[j]) |
                     ((uint32_t)__builtin_bit_cast(uint16_t, hi[j + 4]) << 16);
            dst[4 + j] = (uint32_t)__builtin_bit_cast(uint16_t, lo[j]) |
                         ((uint32_t)__builtin_bit_cast(uint16_t, lo[j + 4]) << 16);
        }
        // the chunk's four blocks sit in four consecutive threads when
        // blockDim and nblk are multiples of 4
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        if ((blk & 3) == 0) csum[(size_t)b * nchunk + (blk >> 2)] = s;
    }
    __syncthreads();

    for (int slot = wave; slot < nslot; slot += 8) {
        load_slot(slot + 8, nxt);   // the next slot's loads in flight
        float acc[kMaxB];
#pragma unroll
        for (int b = 0; b < kMaxB; b++) acc[b] = 0.0f;
#pragma unroll
        for (int i = 0; i < NC; i++) {
            const int c = c16 + 16 * i;
            const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)(cur.sz[i] & 0xFFFFu));
            const float z = (float)__builtin_bit_cast(_Float16, (uint16_t)(cur.sz[i] >> 16));
            uint32_t q[4][4];   // [word][pair]
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t cw = cur.wv[i][w];
                q[w][0] = cw & 0x000F000Fu;
                q[w][1] = (cw >> 4) & 0x000F000Fu;
                q[w][2] = (cw >> 8) & 0x000F000Fu;
                q[w][3] = (cw >> 12) & 0x000F000Fu;
            }
#pragma unroll
            for (int b = 0; b < kMaxB; b++) {
                if (b >= B) break;
                const u32x4_t *xp = reinterpret_cast<const u32x4_t *>(pairs + ((size_t)b * nblk + c * 4) * 8);
                float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // one chain per word
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const u32x4_t xh = xp[2 * w], xl = xp[2 * w + 1];
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        t[w] = dot2(q[w][p], xh[p], t[w]);
                        t[w] = dot2(q[w][p], xl[p], t[w]);
                    }
                }
                const float tt = (t[0] + t[1]) + (t[2] + t[3]);
                acc[b] = __builtin_fmaf(s, __builtin_fmaf(tt, 16777216.0f, -z * csum[(size_t)b * nchunk + c]), acc[b]);
            }
        }
        const int row = rb + 4 * slot + (lane >> 4);
#pragma unroll
        for (int b = 0; b < kMaxB; b++) {
            if (b >= B) break;
            const float v = imh_dpp::row16_sum(acc[b]);
            if (c16 == 0 && row < re) y[(size_t)b * N + row] = __float2half(v);
        }
        cur = nxt;
    }
}

}  // namespace

extern "C" {

int imh_diag_valu_matvec(imh_stream *stream, const uint16_t *x, uint32_t batch, const imh_affine_int4_weight *w,
                         uint16_t *y) {
    const char *who = "imh_diag_valu_matvec";
    if (!stream || !x || !w || !y || !w->data || !w->scales || !w->zeros)
        return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    if (w->group_size != 128 || (w->k != 2560 && w->k != 4096) || w->n == 0)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": group 128 and k of 2560 or 4096 (Qwen3-4B)");
    if (batch == 0) return IMH_OK;
    if (batch > kMaxB) return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": batch above 8");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w->data) |
         reinterpret_cast<uintptr_t>(w->awq_scales)) & 15)
        return imh::fail(IMH_EINVAL, std::string(who) + ": x, data and awq_scales must be 16-byte aligned");
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    const int K = (int)w->k, N = (int)w->n, B = (int)batch;
    const size_t lds = (size_t)B * (K / 8) * 32 + (size_t)B * (K / 32) * 4;
    if (lds > stream->dev->props.sharedMemPerBlock)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": batch x k needs " + std::to_string(lds) +
                                               " bytes of LDS, above the device's per-workgroup limit");
    // one band per compute unit (bands of at least one 4-row slot)
    const int cus = stream->dev->props.multiProcessorCount;
    const dim3 grid(std::max(1, std::min(cus, (N + 3) / 4))), block(512);
    const __half *xh = reinterpret_cast<const __half *>(x);
    const __half *aw = reinterpret_cast<const __half *>(w->awq_scales);
    const __half *sc = reinterpret_cast<const __half *>(w->scales);
    const __half *zr = reinterpret_cast<const __half *>(w->zeros);
    __half *yh = reinterpret_cast<__half *>(y);
#define IMH_VALU_MV(NC)                                                                                   \
    hipLaunchKernelGGL(diag_valu_matvec_kernel<NC>, grid, block, lds, stream->stream, xh, aw, w->data, sc, zr, N, K, B, \
                       yh)
    if (K == 2560) IMH_VALU_MV(5);
    else IMH_VALU_MV(8);
#undef IMH_VALU_MV
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

}  // extern "C"
