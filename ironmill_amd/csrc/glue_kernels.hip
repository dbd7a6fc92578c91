// glue_kernels.hip -- the per-token glue of the decode step around the INT4
// projections and the KV-cache attention: embedding lookup + first RMSNorm,
// RMSNorm, residual add (+ RMSNorm), per-head QK RMSNorm + rotary position
// embedding, and the host-side RoPE table.
//
// Semantics follow the reference kernels named at each entry point; every
// kernel is one pass over its rows with f32 arithmetic and f16 storage.
// These are latency kernels (a decode step moves a few KB through each), so
// the design goal is one launch per op with no LDS round trips beyond the
// block reduction: one workgroup per row, 16-byte loads where the row allows.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cmath>
#include <cstring>
#include <string>

#include "dpp_reduce.h"
#include "qk_norm_rope.h"
#include "imh_internal.h"

namespace {

constexpr int kRowThreads = 256;

// sum over a wave: DPP row sums, then the four rows
__device__ __forceinline__ float wave_sum(float v) {
    v = imh_dpp::row16_sum(v);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// sum over a workgroup of kRowThreads threads; every thread gets the total
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kRowThreads / 64; w++) t += red[w];
    return t;
}

__device__ __forceinline__ float h2f(const __half *p, size_t i) { return __half2float(p[i]); }

// 8 consecutive halves as floats
__device__ __forceinline__ void load8(const __half *p, float *v) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p);
    const __half2 *h = reinterpret_cast<const __half2 *>(&u);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float2 f = __half22float2(h[i]);
        v[2 * i] = f.x;
        v[2 * i + 1] = f.y;
    }
}

__device__ __forceinline__ void store8(__half *p, const float *v) {
    uint4 u;
    __half2 *h = reinterpret_cast<__half2 *>(&u);
#pragma unroll
    for (int i = 0; i < 4; i++) h[i] = __floats2half2_rn(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<uint4 *>(p) = u;
}

// Row kernels.  MODE 0: rms_norm (x = in)          -> out = f16(x * rms_inv * w)
//               MODE 1: fused residual + rms_norm  (x = a + b) -> res = f16(x), out = f16(x * rms_inv * w)
//               MODE 2: fused embedding + rms_norm (x = table[id] * embed_scale, 0 for an id >= vocab)
//                                                   -> res = f16(x), out = f16(x * rms_inv * w)
// grid (rows), block kRowThreads.  VEC: hidden % 8 == 0 and 16-byte aligned rows.
template <int MODE, bool VEC>
__global__ void __launch_bounds__(kRowThreads) row_norm_kernel(const __half *__restrict__ a,
                                                               const __half *__restrict__ b,
                                                               const uint32_t *__restrict__ ids, int vocab,
                                                               float embed_scale, const __half *__restrict__ w,
                                                               __half *__restrict__ out, __half *__restrict__ res,
                                                               int hidden, float eps) {
    __shared__ float red[kRowThreads / 64];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const __half *pa = a;
    bool valid = true;
    if (MODE == 2) {
        const uint32_t id = ids[row];
        valid = id < (uint32_t)vocab;
        pa = a + (size_t)(valid ? id : 0) * hidden;
    } else {
        pa = a + (size_t)row * hidden;
    }
    const __half *pb = MODE == 1 ? b + (size_t)row * hidden : nullptr;
    const size_t ob = (size_t)row * hidden;

    auto value = [&](float av, float bv) {
        if (MODE == 1) return av + bv;
        if (MODE == 2) return valid ? av * embed_scale : 0.0f;
        return av;
    };

    float ss = 0.0f;
    if (VEC) {
        for (int c = tid; c * 8 < hidden; c += kRowThreads) {
            float va[8], vb[8] = {0, 0, 0, 0, 0, 0, 0, 0}, x[8];
            load8(pa + c * 8, va);
            if (MODE == 1) load8(pb + c * 8, vb);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                x[i] = value(va[i], vb[i]);
                ss += x[i] * x[i];
            }
            if (MODE != 0) store8(res + ob + c * 8, x);
        }
    } else {
        for (int i = tid; i < hidden; i += kRowThreads) {
            const float x = value(h2f(pa, i), MODE == 1 ? h2f(pb, i) : 0.0f);
            ss += x * x;
            if (MODE != 0) res[ob + i] = __float2half(x);
        }
    }
    const float total = block_sum(ss, red);
    const float rms_inv = 1.0f / sqrtf(total / (float)hidden + eps);
    if (VEC) {
        for (int c = tid; c * 8 < hidden; c += kRowThreads) {
            float va[8], vb[8] = {0, 0, 0, 0, 0, 0, 0, 0}, wv[8], y[8];
            load8(pa + c * 8, va);
            if (MODE == 1) load8(pb + c * 8, vb);
            load8(w + c * 8, wv);
#pragma unroll
            for (int i = 0; i < 8; i++) y[i] = value(va[i], vb[i]) * rms_inv * wv[i];
            store8(out + ob + c * 8, y);
        }
    } else {
        for (int i = tid; i < hidden; i += kRowThreads) {
            const float x = value(h2f(pa, i), MODE == 1 ? h2f(pb, i) : 0.0f);
            out[ob + i] = __float2half(x * rms_inv * h2f(w, i));
        }
    }
}

// out = f16(f32(a) + f32(b)), grid-stride
__global__ void __launch_bounds__(256) residual_add_kernel(const __half *__restrict__ a, const __half *__restrict__ b,
                                                           __half *__restrict__ out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        out[i] = __float2half(__half2float(a[i]) + __half2float(b[i]));
}

// Per-head RMSNorm + RoPE in place.  grid (nh + nkv, batch * token_count),
// block 64 (one wave).  With norm weights: fused_qk_norm_rope semantics,
// pairs (d, d + rotary/2) inside the first rotary_dim dims, the rest only
// normalised.  Without: rope semantics, pairs (d, d + head_dim/2), the table
// supplying identity beyond rotary/2.  Tables are [max_pos][head_dim/2].
__global__ void __launch_bounds__(64) qk_norm_rope_kernel(__half *__restrict__ q, __half *__restrict__ k,
                                                          const __half *__restrict__ q_norm,
                                                          const __half *__restrict__ k_norm,
                                                          const __half *__restrict__ cos_t,
                                                          const __half *__restrict__ sin_t, int nh, int nkv, int hd,
                                                          int rotary, int max_pos, int seq_offset,
                                                          const int32_t *__restrict__ positions, int tokens,
                                                          float eps) {
    __shared__ float xs[256];
    const int slot = blockIdx.x;
    const int row = blockIdx.y;  // b * tokens + t
    const int tid = threadIdx.x;
    const bool is_q = slot < nh;
    const int heads = is_q ? nh : nkv;
    const int head = is_q ? slot : slot - nh;
    __half *p = (is_q ? q : k) + ((size_t)row * heads + head) * hd;
    const __half *nw = is_q ? q_norm : k_norm;
    const int b = row / tokens, t = row % tokens;
    long pos = (long)(positions ? positions[b] : seq_offset) + t;
    pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
    const int half_dim = hd / 2;
    const __half *cs = cos_t + (size_t)pos * half_dim;
    const __half *sn = sin_t + (size_t)pos * half_dim;
    if (nw && hd == imh_qk::kHd && rotary == imh_qk::kHd) {   // one head in registers (qk_norm_rope.h)
        float x0 = h2f(p, tid), x1 = h2f(p, tid + 64);
        imh_qk::norm_rope_128(x0, x1, tid, nw, cs, sn, eps);
        p[tid] = __float2half(x0);
        p[tid + 64] = __float2half(x1);
        return;
    }

    float ss = 0.0f;
    for (int d = tid; d < hd; d += 64) {
        const float v = h2f(p, d);
        xs[d] = v;
        ss += v * v;
    }
    __syncthreads();
    if (nw) {
        const float rms_inv = 1.0f / sqrtf(wave_sum(ss) / (float)hd + eps);
        const int hr = rotary / 2;
        for (int d = tid; d < hr; d += 64) {
            const float lo = xs[d] * rms_inv * h2f(nw, d);
            const float hi = xs[d + hr] * rms_inv * h2f(nw, d + hr);
            const float c = h2f(cs, d), s = h2f(sn, d);
            p[d] = __float2half(lo * c - hi * s);
            p[d + hr] = __float2half(lo * s + hi * c);
        }
        for (int d = rotary + tid; d < hd; d += 64) p[d] = __float2half(xs[d] * rms_inv * h2f(nw, d));
    } else {
        for (int d = tid; d < half_dim; d += 64) {
            const float lo = xs[d], hi = xs[d + half_dim];
            const float c = h2f(cs, d), s = h2f(sn, d);
            p[d] = __float2half(lo * c - hi * s);
            p[d + half_dim] = __float2half(lo * s + hi * c);
        }
    }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int MODE>
int launch_row_norm(imh_stream *s, const __half *a, const __half *b, const uint32_t *ids, int vocab, float scale,
                    const __half *w, __half *out, __half *res, uint32_t hidden, uint32_t rows, float eps) {
    const bool vec = hidden % 8 == 0 && aligned16(a) && (!b || aligned16(b)) && aligned16(w) && aligned16(out) &&
                     (!res || aligned16(res));
    if (vec)
        hipLaunchKernelGGL((row_norm_kernel<MODE, true>), dim3(rows), dim3(kRowThreads), 0, s->stream, a, b, ids,
                           vocab, scale, w, out, res, (int)hidden, eps);
    else
        hipLaunchKernelGGL((row_norm_kernel<MODE, false>), dim3(rows), dim3(kRowThreads), 0, s->stream, a, b, ids,
                           vocab, scale, w, out, res, (int)hidden, eps);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

// f64 -> f16 bits, round to nearest even, directly from the double (one rounding)
uint16_t f64_to_f16_rne(double x) {
    uint64_t u;
    std::memcpy(&u, &x, 8);
    const uint16_t sign = (uint16_t)((u >> 48) & 0x8000);
    const double ax = std::fabs(x);
    if (std::isnan(x)) return sign | 0x7E00;
    if (ax >= 65520.0) return sign | 0x7C00;  // rounds to infinity
    if (ax < std::ldexp(1.0, -14)) {
        // subnormal: units of 2^-24, nearest even
        const double q = ax * std::ldexp(1.0, 24);
        double r = std::nearbyint(q);  // default rounding mode: to nearest even
        return sign | (uint16_t)r;
    }
    int e;
    const double m = std::frexp(ax, &e);  // ax = m * 2^e, m in [0.5, 1)
    // 11 significant bits: scale to [1024, 2048)
    double q = std::nearbyint(std::ldexp(m, 11));
    if (q == 2048.0) {
        q = 1024.0;
        e += 1;
    }
    const int exp_field = e - 1 + 15;
    if (exp_field >= 31) return sign | 0x7C00;
    return sign | (uint16_t)(exp_field << 10) | (uint16_t)((uint32_t)q - 1024);
}

}  // namespace

extern "C" {

int imh_encode_rms_norm(imh_stream *stream, const uint16_t *input, const uint16_t *weight, uint16_t *output,
                        uint32_t hidden_size, uint32_t token_count, float eps) {
    if (!stream || !input || !weight || !output) return imh::fail(IMH_EINVAL, "imh_encode_rms_norm: NULL argument");
    if (hidden_size == 0) return imh::fail(IMH_EINVAL, "imh_encode_rms_norm: hidden_size 0");
    if (token_count == 0) return IMH_OK;
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    return launch_row_norm<0>(stream, reinterpret_cast<const __half *>(input), nullptr, nullptr, 0, 1.0f,
                              reinterpret_cast<const __half *>(weight), reinterpret_cast<__half *>(output), nullptr,
                              hidden_size, token_count, eps);
}

int imh_encode_fused_residual_rms_norm(imh_stream *stream, const uint16_t *a, const uint16_t *b,
                                       const uint16_t *weight, uint16_t *normed_output, uint16_t *residual_output,
                                       uint32_t hidden_size, uint32_t token_count, float eps) {
    if (!stream || !a || !b || !weight || !normed_output || !residual_output)
        return imh::fail(IMH_EINVAL, "imh_encode_fused_residual_rms_norm: NULL argument");
    if (hidden_size == 0) return imh::fail(IMH_EINVAL, "imh_encode_fused_residual_rms_norm: hidden_size 0");
    if (token_count == 0) return IMH_OK;
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    return launch_row_norm<1>(stream, reinterpret_cast<const __half *>(a), reinterpret_cast<const __half *>(b),
                              nullptr, 0, 1.0f, reinterpret_cast<const __half *>(weight),
                              reinterpret_cast<__half *>(normed_output), reinterpret_cast<__half *>(residual_output),
                              hidden_size, token_count, eps);
}

int imh_encode_residual_add(imh_stream *stream, const uint16_t *a, const uint16_t *b, uint16_t *out, size_t n) {
    if (!stream || !a || !b || !out) return imh::fail(IMH_EINVAL, "imh_encode_residual_add: NULL argument");
    if (n == 0) return IMH_OK;
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)blocks), dim3(256), 0, stream->stream,
                       reinterpret_cast<const __half *>(a), reinterpret_cast<const __half *>(b),
                       reinterpret_cast<__half *>(out), n);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

int imh_encode_fused_embedding_norm(imh_stream *stream, const uint32_t *token_ids, const uint16_t *embedding,
                                    const uint16_t *norm_weight, uint16_t *normed_output, uint16_t *raw_output,
                                    uint32_t hidden_size, uint32_t token_count, uint32_t vocab_size, float eps,
                                    float embed_scale) {
    if (!stream || !token_ids || !embedding || !norm_weight || !normed_output || !raw_output)
        return imh::fail(IMH_EINVAL, "imh_encode_fused_embedding_norm: NULL argument");
    if (hidden_size == 0 || vocab_size == 0)
        return imh::fail(IMH_EINVAL, "imh_encode_fused_embedding_norm: empty table");
    if (token_count == 0) return IMH_OK;
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    return launch_row_norm<2>(stream, reinterpret_cast<const __half *>(embedding), nullptr, token_ids,
                              (int)vocab_size, embed_scale, reinterpret_cast<const __half *>(norm_weight),
                              reinterpret_cast<__half *>(normed_output), reinterpret_cast<__half *>(raw_output),
                              hidden_size, token_count, eps);
}

int imh_rope_cache_fill(uint32_t head_dim, uint32_t max_pos, double theta, uint32_t rotary_dim, uint16_t *cos_out,
                        uint16_t *sin_out) {
    if (!cos_out || !sin_out) return imh::fail(IMH_EINVAL, "imh_rope_cache_fill: NULL argument");
    if (head_dim == 0 || head_dim % 2) return imh::fail(IMH_EINVAL, "imh_rope_cache_fill: head_dim must be even");
    const uint32_t rd = rotary_dim ? rotary_dim : head_dim;
    if (rd > head_dim || rd % 2) return imh::fail(IMH_EINVAL, "imh_rope_cache_fill: bad rotary_dim");
    const uint32_t half_dim = head_dim / 2, rh = rd / 2;
    for (uint32_t pos = 0; pos < max_pos; pos++)
        for (uint32_t i = 0; i < half_dim; i++) {
            const size_t o = (size_t)pos * half_dim + i;
            if (i < rh) {
                const double freq = 1.0 / std::pow(theta, 2.0 * (double)i / (double)rd);
                const double angle = (double)pos * freq;
                cos_out[o] = f64_to_f16_rne(std::cos(angle));
                sin_out[o] = f64_to_f16_rne(std::sin(angle));
            } else {
                cos_out[o] = 0x3C00;  // 1.0
                sin_out[o] = 0x0000;
            }
        }
    return IMH_OK;
}

int imh_encode_qk_norm_rope(imh_stream *stream, const imh_qk_norm_rope_params *p) {
    const char *who = "imh_encode_qk_norm_rope";
    if (!stream || !p || !p->q || !p->k || !p->cos_cache || !p->sin_cache)
        return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    if (!p->q_norm != !p->k_norm) return imh::fail(IMH_EINVAL, std::string(who) + ": give both norm weights or none");
    const uint32_t hd = p->head_dim;
    const uint32_t rd = p->rotary_dim ? p->rotary_dim : hd;
    if (hd == 0 || hd % 2 || hd > 256) return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": head_dim must be even, <= 256");
    if (rd > hd || rd % 2) return imh::fail(IMH_EINVAL, std::string(who) + ": bad rotary_dim");
    if (p->max_pos == 0) return imh::fail(IMH_EINVAL, std::string(who) + ": empty RoPE table");
    if (!p->positions && (uint64_t)p->seq_offset + p->token_count > p->max_pos)
        return imh::fail(IMH_ERANGE, std::string(who) + ": seq_offset + token_count beyond the RoPE table");
    const uint64_t rows = (uint64_t)p->batch * p->token_count;
    if (rows == 0 || p->num_heads + p->num_kv_heads == 0) return IMH_OK;
    if (rows > 65535) return imh::fail(IMH_EINVAL, std::string(who) + ": batch * token_count above 65535");
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(p->num_heads + p->num_kv_heads, (unsigned)rows), dim3(64), 0,
                       stream->stream, reinterpret_cast<__half *>(p->q), reinterpret_cast<__half *>(p->k),
                       reinterpret_cast<const __half *>(p->q_norm), reinterpret_cast<const __half *>(p->k_norm),
                       reinterpret_cast<const __half *>(p->cos_cache), reinterpret_cast<const __half *>(p->sin_cache),
                       (int)p->num_heads, (int)p->num_kv_heads, (int)hd, (int)rd, (int)p->max_pos,
                       (int)p->seq_offset, p->positions, (int)p->token_count, p->eps);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

}  // extern "C"
