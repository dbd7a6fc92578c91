// fp16_attention.hip -- FP16 KV cache: projection scatter and GQA decode
// attention (the non-quantized comparator of the TurboQuant path).
//
// Scatter: encode_kv_scatter (ops/kv.rs, kv_scatter.metal, called at
// attention.rs:497-525) -- token t of a sequence goes to cache row
// (pos + t) % max_seq_len.
//
// Attention: the semantics of fused_sdpa.metal:52-251 / the FlashDecoding
// split + reduce of flash_decode.metal:25-215 (encode_flash_decode,
// attention_ops.rs:346-417): softmax(attn_scale * q . k) . v.  The structure
// is this file's own: one workgroup per (KV split, kv head, sequence) serves
// every query head of the GQA group, so each K/V byte is read once per group.
// q and K are exact f16, so the scores run on the matrix cores
// (v_mfma_f32_16x16x32_f16, rows = the group's heads, columns = 16 positions)
// straight from 16-byte K loads with no operand split; the softmax is online
// with DPP row reductions, V is accumulated in f32, and each wave loads the
// next 16-position chunk while it computes the current one.  A second kernel
// combines the splits (log-sum-exp) and normalises.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cmath>
#include <string>

#include "dpp_reduce.h"
#include "imh_internal.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kD = 128;          // head_dim the kernels are built for
constexpr int kChunk = 16;       // positions per MFMA block
constexpr int kWaves = 4;        // waves per attention workgroup
constexpr int kSplitQuantum = kChunk * kWaves;

// grid (num_kv_heads, token_count, batch), block kD / 8: one 16-byte chunk of
// the head vector per thread.
// wrap = 0: positions at or past max_seq are skipped instead of wrapping.
__global__ void __launch_bounds__(kD / 8) fp16_kv_scatter_kernel(const __half *__restrict__ proj, int tokens,
                                                                 int nkv, int max_seq, int base_pos,
                                                                 const int32_t *__restrict__ positions,
                                                                 __half *__restrict__ cache, int wrap) {
    const int h = blockIdx.x, t = blockIdx.y, b = blockIdx.z;
    const int c = threadIdx.x;
    long pos = (long)(positions ? positions[b] : base_pos) + t;
    if (!wrap && (pos < 0 || pos >= max_seq)) return;
    pos %= max_seq;
    if (pos < 0) pos += max_seq;
    const size_t src = (((size_t)b * tokens + t) * nkv + h) * kD + (size_t)c * 8;
    const size_t dst = (((size_t)b * nkv + h) * max_seq + (size_t)pos) * kD + (size_t)c * 8;
    *reinterpret_cast<uint4 *>(cache + dst) = *reinterpret_cast<const uint4 *>(proj + src);
}

// grid (num_splits, num_kv_heads, batch * ceil(T / TB)), block 64 * kWaves.
// Score rows r = tb * GQA + hh (tb < TB query tokens, hh < GQA heads of the
// kv head's group), R = TB * GQA <= 4, so the rows of the MFMA result sit in
// lanes 0..15 (lane = position n, register = row).
template <int GQA, int TB>
__global__ void __launch_bounds__(64 * kWaves) fp16_attention_kernel(
    const __half *__restrict__ q, int T, int nh, int nkv, int max_seq, int seq_len,
    const int32_t *__restrict__ seq_lens, float attn_scale, const __half *__restrict__ k_cache,
    const __half *__restrict__ v_cache, int split_len, float *__restrict__ part_o,
    float *__restrict__ part_m, float *__restrict__ part_l) {
    constexpr int R = GQA * TB;
    static_assert(R <= 4, "score rows must fit the first register row block");
    __shared__ _Float16 qs[R][kD];
    __shared__ float om[kWaves][R][kD];
    __shared__ float mm[kWaves][R];
    __shared__ float ll[kWaves][R];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int split = blockIdx.x, kvh = blockIdx.y;
    const int QB = (T + TB - 1) / TB;
    const int b = blockIdx.z / QB, qb = blockIdx.z % QB;
    const int S = gridDim.x;
    const int t0 = qb * TB;

    // with seq_lens, seq_len is the bound every length is clamped to
    int L = seq_lens ? min(seq_lens[b], seq_len) : seq_len;
    L = L > max_seq ? max_seq : L;
    // causal limit of row r: positions < L - T + t + 1
    int lim[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int t = t0 + r / GQA;
        lim[r] = t < T ? L - T + t + 1 : 0;
    }
    int lim_max = 0;
#pragma unroll
    for (int r = 0; r < R; r++) lim_max = max(lim_max, lim[r]);
    const int p_begin = split * split_len;
    const int p_end = min(p_begin + split_len, lim_max);
    const size_t head_base = ((size_t)b * nkv + kvh) * (size_t)max_seq;
    const int n_l = lane & 15;
    const int kg = lane >> 4;
    const int vgrp = lane & 7;    // 16-dim slice of V this lane accumulates
    const int vpos = lane >> 3;   // position (of 8) per V round

    // chunk inputs, loaded one chunk ahead: K row of position n_l (dims
    // j*32 + kg*8 .. +7, j = 0..3), V rows of positions vpos and 8 + vpos
    // (dims vgrp*16 .. +15); positions past the end reread the last one
    struct ChunkIn {
        uint4 k[4];
        uint4 v[4];
    };
    auto load_chunk = [&](int p0, ChunkIn &c) __attribute__((always_inline)) {
        const int last = p_end - 1;
        const __half *kp = k_cache + (head_base + min(p0 + n_l, last)) * kD + kg * 8;
#pragma unroll
        for (int j = 0; j < 4; j++) c.k[j] = *reinterpret_cast<const uint4 *>(kp + j * 32);
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const __half *vp = v_cache + (head_base + min(p0 + r * 8 + vpos, last)) * kD + vgrp * 16;
            c.v[2 * r] = *reinterpret_cast<const uint4 *>(vp);
            c.v[2 * r + 1] = *reinterpret_cast<const uint4 *>(vp + 8);
        }
    };
    ChunkIn cur;
    const int p_first = p_begin + wave * kChunk;
    if (p_first < p_end) load_chunk(p_first, cur);

    for (int e = tid; e < R * kD; e += 64 * kWaves) {
        const int r = e / kD, d = e % kD;
        const int t = t0 + r / GQA;
        uint16_t bits = 0;
        if (t < T) bits = reinterpret_cast<const uint16_t *>(q)[(((size_t)b * T + t) * nh + kvh * GQA + r % GQA) * kD + d];
        qs[r][d] = __builtin_bit_cast(_Float16, bits);
    }
    __syncthreads();
    // operand A: row n_l < R holds q of score row n_l (zero beyond), k = dims
    // j*32 + kg*8 + i
    half8_t aq[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 8; i++) aq[j][i] = n_l < R ? qs[n_l][j * 32 + kg * 8 + i] : (_Float16)0.0f;

    float m_run[R], l_run[R];
    float o[R][16];
#pragma unroll
    for (int r = 0; r < R; r++) {
        m_run[r] = -INFINITY;
        l_run[r] = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e++) o[r][e] = 0.0f;
    }

    for (int p0 = p_first; p0 < p_end; p0 += kChunk * kWaves) {
        const ChunkIn c = cur;
        if (p0 + kChunk * kWaves < p_end) load_chunk(p0 + kChunk * kWaves, cur);
        float4_t d1 = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; j++)
            d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[j], __builtin_bit_cast(half8_t, c.k[j]), d1, 0, 0, 0);
        float wgt[R], corr[R];
        bool rescale = false;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float sc = (p0 + n_l) < lim[r] ? attn_scale * d1[r] : -INFINITY;
            const float cm = imh_dpp::first_lane(imh_dpp::row16_max(sc));
            const float nm = fmaxf(m_run[r], cm);
            // a row with no position yet keeps m = -inf, weights 0
            const bool live = nm != -INFINITY;
            corr[r] = live ? __expf(m_run[r] - nm) : 1.0f;
            const float w = live ? __expf(sc - nm) : 0.0f;
            const float ws = imh_dpp::first_lane(imh_dpp::row16_sum(w));
            l_run[r] = l_run[r] * corr[r] + ws;
            m_run[r] = nm;
            wgt[r] = w;
            rescale |= corr[r] != 1.0f;
        }
        if (rescale) {
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int e = 0; e < 16; e++) o[r][e] *= corr[r];
        }
        // o += w * V, one position per lane per round
#pragma unroll
        for (int rr = 0; rr < 2; rr++) {
            const int pi = rr * 8 + vpos;
            float wv[R];
#pragma unroll
            for (int r = 0; r < R; r++) wv[r] = __shfl(wgt[r], pi);
            const half8_t v0 = __builtin_bit_cast(half8_t, c.v[2 * rr]);
            const half8_t v1 = __builtin_bit_cast(half8_t, c.v[2 * rr + 1]);
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float v = (float)(e < 8 ? v0[e] : v1[e - 8]);
#pragma unroll
                for (int r = 0; r < R; r++) o[r][e] = __builtin_fmaf(wv[r], v, o[r][e]);
            }
        }
    }

    // sum the 8 position lanes that share a V slice
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            float v = o[r][e];
            v += __shfl_xor(v, 8);
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            o[r][e] = v;
        }
    if (lane < 8) {
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int e = 0; e < 16; e++) om[wave][r][lane * 16 + e] = o[r][e];
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            mm[wave][r] = m_run[r];
            ll[wave][r] = l_run[r];
        }
    }
    __syncthreads();
    for (int e = tid; e < R * kD; e += 64 * kWaves) {
        const int r = e / kD, d = e % kD;
        const int t = t0 + r / GQA;
        if (t >= T) continue;
        float M = -INFINITY;
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, mm[w][r]);
        float ov = 0.0f, lv = 0.0f;
        if (M != -INFINITY) {
            for (int w = 0; w < kWaves; w++) {
                if (mm[w][r] == -INFINITY) continue;
                const float f = __expf(mm[w][r] - M);
                ov += om[w][r][d] * f;
                lv += ll[w][r] * f;
            }
        }
        const size_t pidx = (((size_t)b * T + t) * nh + kvh * GQA + r % GQA) * S + split;
        part_o[pidx * kD + d] = ov;
        if (d == 0) {
            part_m[pidx] = M;
            part_l[pidx] = lv;
        }
    }
}

// combine splits (log-sum-exp) and normalise: grid (num_heads, batch * T),
// block kD; partials [batch][T][num_heads][splits]
__global__ void __launch_bounds__(kD) fp16_attention_reduce_kernel(const float *__restrict__ part_o,
                                                                   const float *__restrict__ part_m,
                                                                   const float *__restrict__ part_l, int nh, int S,
                                                                   __half *__restrict__ out) {
    __shared__ float fs[kD];
    __shared__ float red[kD];
    const int d = threadIdx.x;
    const int h = blockIdx.x, b = blockIdx.y;
    const size_t base = ((size_t)b * nh + h) * S;
    float mloc = -INFINITY;
    for (int s = d; s < S; s += kD) mloc = fmaxf(mloc, part_m[base + s]);
    red[d] = mloc;
    __syncthreads();
    for (int w = kD / 2; w > 0; w >>= 1) {
        if (d < w) red[d] = fmaxf(red[d], red[d + w]);
        __syncthreads();
    }
    const float M = red[0];
    __syncthreads();
    float ov = 0.0f, lloc = 0.0f;
    for (int s0 = 0; s0 < S; s0 += kD) {
        const int s = s0 + d;
        float f = 0.0f;
        if (s < S) {
            const float m = part_m[base + s];
            if (m != -INFINITY) {
                f = __expf(m - M);
                lloc += part_l[base + s] * f;
            }
        }
        fs[d] = f;
        __syncthreads();
        const int n = min(kD, S - s0);
#pragma unroll 8
        for (int i = 0; i < n; i++) ov = __builtin_fmaf(part_o[(base + s0 + i) * kD + d], fs[i], ov);
        __syncthreads();
    }
    red[d] = lloc;
    __syncthreads();
    for (int w = kD / 2; w > 0; w >>= 1) {
        if (d < w) red[d] += red[d + w];
        __syncthreads();
    }
    const float lv = red[0];
    out[((size_t)b * nh + h) * kD + d] = __float2half(M == -INFINITY ? 0.0f : ov / fmaxf(lv, 1e-10f));
}

int check_cache(const imh_fp16_kv_cache *c, const char *who) {
    if (!c || !c->k || !c->v) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL cache or cache array");
    if (c->head_dim != kD)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": kernels are built for head_dim 128");
    if (c->batch == 0 || c->num_kv_heads == 0 || c->max_seq_len == 0)
        return imh::fail(IMH_EINVAL, std::string(who) + ": empty cache shape");
    if ((reinterpret_cast<uintptr_t>(c->k) | reinterpret_cast<uintptr_t>(c->v)) & 15)
        return imh::fail(IMH_EINVAL, std::string(who) + ": cache arrays must be 16-byte aligned");
    return IMH_OK;
}

}  // namespace

extern "C" {

int imh_encode_kv_scatter(imh_stream *stream, const imh_fp16_kv_cache *cache, const uint16_t *proj,
                          uint32_t token_count, uint32_t base_pos, const int32_t *positions, int is_k) {
    const char *who = "imh_encode_kv_scatter";
    if (!stream || !proj) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_cache(cache, who);
    if (rc) return rc;
    if (reinterpret_cast<uintptr_t>(proj) & 15)
        return imh::fail(IMH_EINVAL, std::string(who) + ": projection must be 16-byte aligned");
    if (token_count == 0) return IMH_OK;
    if (token_count > 65535) return imh::fail(IMH_EINVAL, std::string(who) + ": token_count above 65535");
    rc = imh::use_device(stream->dev);
    if (rc) return rc;
    dim3 grid(cache->num_kv_heads, token_count, cache->batch);
    hipLaunchKernelGGL(fp16_kv_scatter_kernel, grid, dim3(kD / 8), 0, stream->stream,
                       reinterpret_cast<const __half *>(proj), (int)token_count, (int)cache->num_kv_heads,
                       (int)cache->max_seq_len, (int)base_pos, positions,
                       reinterpret_cast<__half *>(is_k ? cache->k : cache->v), 1);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

int imh_encode_fp16_attention(imh_stream *stream, const imh_fp16_kv_cache *cache, const uint16_t *q,
                              uint32_t num_heads, uint32_t token_count, uint32_t seq_len,
                              const int32_t *seq_lens, float attn_scale, uint16_t *out, uint32_t num_splits) {
    const char *who = "imh_encode_fp16_attention";
    if (!stream || !q || !out) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_cache(cache, who);
    if (rc) return rc;
    const uint32_t nkv = cache->num_kv_heads;
    if (num_heads == 0 || num_heads % nkv != 0)
        return imh::fail(IMH_EINVAL, std::string(who) + ": num_heads must be a multiple of num_kv_heads");
    const uint32_t gqa = num_heads / nkv;
    if (gqa != 1 && gqa != 2 && gqa != 4)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": GQA group of " + std::to_string(gqa) +
                                               " heads not built (1, 2, 4)");
    if (seq_len > cache->max_seq_len)
        return imh::fail(IMH_ERANGE, std::string(who) + ": seq_len " + std::to_string(seq_len) +
                                         " exceeds max_seq_len " + std::to_string(cache->max_seq_len));
    if (token_count == 0) return IMH_OK;
    if (!seq_lens && token_count > seq_len)
        return imh::fail(IMH_EINVAL, std::string(who) + ": token_count exceeds seq_len");
    const uint32_t B = cache->batch;
    const uint32_t tb = gqa == 4 ? 1 : (token_count == 1 ? 1 : 4 / gqa);
    const uint32_t qblocks = (token_count + tb - 1) / tb;
    if ((uint64_t)B * token_count > 65535)
        return imh::fail(IMH_EINVAL, std::string(who) + ": batch * token_count above 65535");
    rc = imh::use_device(stream->dev);
    if (rc) return rc;

    // KV split: ~512 workgroups, each split a multiple of one pass of the
    // workgroup's waves (64 positions); with per-sequence lengths the splits
    // span the bound (0 = max_seq_len)
    const uint32_t L = seq_lens && seq_len == 0 ? cache->max_seq_len : seq_len;
    uint32_t want = num_splits;
    if (want == 0) want = (512 + B * nkv * qblocks - 1) / (B * nkv * qblocks);
    const uint32_t max_splits = std::max<uint32_t>(1, (L + kSplitQuantum - 1) / kSplitQuantum);
    want = std::max<uint32_t>(1, std::min(want, max_splits));
    uint32_t split_len = (L + want - 1) / want;
    split_len = std::max<uint32_t>(kSplitQuantum, (split_len + kSplitQuantum - 1) / kSplitQuantum * kSplitQuantum);
    const uint32_t S = std::max<uint32_t>(1, (L + split_len - 1) / split_len);

    const size_t nparts = (size_t)B * token_count * num_heads * S;
    void *scr = nullptr;
    rc = imh::stream_scratch(stream, 1, nparts * kD * 4 + nparts * 8 + 512, &scr);
    if (rc) return rc;
    float *po = static_cast<float *>(scr);
    float *pm = po + nparts * kD;
    float *pl = pm + nparts;
    dim3 grid(S, nkv, B * qblocks);
    const __half *qh = reinterpret_cast<const __half *>(q);
    const __half *kc = reinterpret_cast<const __half *>(cache->k);
    const __half *vc = reinterpret_cast<const __half *>(cache->v);
#define IMH_FP16_ATTN(G, TBV)                                                                                      \
    hipLaunchKernelGGL((fp16_attention_kernel<G, TBV>), grid, dim3(64 * kWaves), 0, stream->stream, qh,             \
                       (int)token_count, (int)num_heads, (int)nkv, (int)cache->max_seq_len, (int)L, seq_lens,        \
                       attn_scale, kc, vc, (int)split_len, po, pm, pl)
    if (gqa == 4) IMH_FP16_ATTN(4, 1);
    else if (gqa == 2 && tb == 1) IMH_FP16_ATTN(2, 1);
    else if (gqa == 2) IMH_FP16_ATTN(2, 2);
    else if (tb == 1) IMH_FP16_ATTN(1, 1);
    else IMH_FP16_ATTN(1, 4);
#undef IMH_FP16_ATTN
    IMH_HIP(hipGetLastError());
    hipLaunchKernelGGL(fp16_attention_reduce_kernel, dim3(num_heads, B * token_count), dim3(kD), 0,
                       stream->stream, po, pm, pl, (int)num_heads, (int)S, reinterpret_cast<__half *>(out));
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

int imh_encode_fp16_kv_cache_and_attention(imh_stream *stream, const imh_fp16_kv_cache *cache,
                                           const uint16_t *k_proj, const uint16_t *v_proj, const uint16_t *q,
                                           uint32_t num_heads, uint32_t token_count, uint32_t seq_pos,
                                           float attn_scale, uint16_t *out) {
    const char *who = "imh_encode_fp16_kv_cache_and_attention";
    int rc = check_cache(cache, who);
    if (rc) return rc;
    if ((uint64_t)seq_pos + token_count > cache->max_seq_len)
        return imh::fail(IMH_ERANGE, std::string(who) + ": seq_pos + token_count exceeds max_seq_len");
    rc = imh_encode_kv_scatter(stream, cache, k_proj, token_count, seq_pos, nullptr, 1);
    if (rc) return rc;
    rc = imh_encode_kv_scatter(stream, cache, v_proj, token_count, seq_pos, nullptr, 0);
    if (rc) return rc;
    return imh_encode_fp16_attention(stream, cache, q, num_heads, token_count, seq_pos + token_count, nullptr,
                                     attn_scale, out, 0);
}

}  // extern "C"

namespace imh {

// One token per sequence at device positions, without the ring wrap of
// imh_encode_kv_scatter: a position at or past max_seq_len writes nothing
// (the decoder's step past a full cache).
int encode_kv_scatter_bounded(imh_stream *stream, const imh_fp16_kv_cache *cache, const uint16_t *proj,
                              const int32_t *positions, int is_k) {
    const char *who = "encode_kv_scatter_bounded";
    if (!stream || !proj || !positions) return fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_cache(cache, who);
    if (rc) return rc;
    if (reinterpret_cast<uintptr_t>(proj) & 15)
        return fail(IMH_EINVAL, std::string(who) + ": projection must be 16-byte aligned");
    rc = use_device(stream->dev);
    if (rc) return rc;
    dim3 grid(cache->num_kv_heads, 1, cache->batch);
    hipLaunchKernelGGL(fp16_kv_scatter_kernel, grid, dim3(kD / 8), 0, stream->stream,
                       reinterpret_cast<const __half *>(proj), 1, (int)cache->num_kv_heads,
                       (int)cache->max_seq_len, 0, positions,
                       reinterpret_cast<__half *>(is_k ? cache->k : cache->v), 0);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

}  // namespace imh
