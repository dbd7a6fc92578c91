// decoder.hip -- one decode step of a standard pre-norm transformer over the
// library's ops: the per-layer schedule of run_pipeline_inner
// (metal/pipeline.rs:228-1313, layer loop :533-1135) for INT4-affine weights
// and a TurboQuant INT8 or FP16 KV cache, for `batch` sequences at once.
//
// All per-step state lives in device memory: positions[b] (the cache row the
// step writes) and seq_lens[b] = positions[b] + 1 are read by the kernels and
// advanced by the step's last kernel.  A step therefore has no host-side
// arguments that change between tokens, so a caller can capture one step into
// a HIP graph and replay it once per token (the graph replaces the
// reference's per-token command-buffer encode).
//
// Schedule per layer l (B rows = one token per sequence):
//   [l == 0] embedding + input RMSNorm          -> hidden, norm_out
//   Q | K | V projections of norm_out as the row segments of one launch
//     (for l > 0 fused into the previous layer's end, see below)
//   TurboQuant: cache write of K, V at positions[b] and attention over
//     [0, seq_lens[b]) in one launch, the QK RMSNorm + RoPE of K and Q inside
//     it; FP16 cache: QK RMSNorm + RoPE, K / V scatter, attention -> attn_out
//   O projection                                -> ffn_down
//   residual + post-attention RMSNorm + gate/up + SiLU/GELU (one launch)
//                                               -> residual, act
//   down projection                             -> ffn_down
//     (at 1-2 rows: reads the operand image the gate/up launch wrote)
//   [l < L-1] residual + next input RMSNorm + next Q | K | V (one launch)
//   [l = L-1] residual add                      -> hidden
// final RMSNorm, LM head -> logits; positions += 1.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "imh_internal.h"

struct imh_decoder {
    imh_device *dev;
    imh_decoder_config cfg;
    std::vector<imh_decoder_layer_weights> layers;
    std::vector<bool> layer_set;
    const uint16_t *embedding = nullptr;
    const uint16_t *final_norm = nullptr;
    imh_affine_int4_weight lm_head{};
    bool model_set = false;

    void *arena = nullptr;  // activations, positions, RoPE tables
    uint16_t *hidden, *residual, *norm_out, *q, *k, *v, *attn_out, *ffn_down, *act;
    int32_t *positions, *seq_lens;
    int32_t *status;        // set by a step past the cache's end, cleared by reset
    uint16_t *rope_cos, *rope_sin;

    void *kv_arena = nullptr;
    imh_tq_tables *own_tq = nullptr;   // created from cfg.tq_seed
    imh_tq_tables *tq = nullptr;       // in use: own_tq or the caller's (imh_decoder_set_tq_tables)
    std::vector<imh_tq_kv_cache> tq_caches;
    std::vector<imh_fp16_kv_cache> fp16_caches;
    void *prefill_arena = nullptr;   // activation rows of imh_decoder_prefill
    size_t prefill_bytes = 0;
    // per layer: sliding-window size (0 = full attention); a windowed layer's
    // cache is a ring of that many positions
    std::vector<uint32_t> windows;

    // mirror of positions for range checks: advanced by eager steps (not by
    // capture), refreshed from the device by imh_decoder_sync_positions
    std::vector<int32_t> host_positions;
};

namespace {

// The step's last kernel: positions[b] is the row the step wrote.  When the
// cache is full (the next position is max_seq) seq_lens[b] becomes 0, so a
// further step -- a graph replayed once too often -- writes no cache row
// (the TurboQuant writer skips an empty sequence, the FP16 scatter runs
// without wrap) and attends over nothing; that step then raises the status
// flag, which imh_decoder_sync_positions reports as IMH_ERANGE (the
// reference refuses such a step, metal/pipeline.rs:271-279).
__global__ void decoder_advance_kernel(int32_t *positions, int32_t *seq_lens, int32_t *status, int batch,
                                       int max_seq, int T) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= batch) return;
    const int p = positions[b];
    if (p + T > max_seq) {
        seq_lens[b] = 0;
        __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    positions[b] = p + T;
    seq_lens[b] = p + T >= max_seq ? 0 : p + T + 1;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int check_weight(const imh_affine_int4_weight &w, uint32_t n, uint32_t k, const char *name) {
    if (!w.data || !w.scales || !w.zeros)
        return imh::fail(IMH_EINVAL, std::string("imh_decoder: ") + name + ": NULL weight array");
    if (w.n != n || w.k != k)
        return imh::fail(IMH_EINVAL, std::string("imh_decoder: ") + name + " is " + std::to_string(w.n) + "x" +
                                         std::to_string(w.k) + ", expected " + std::to_string(n) + "x" +
                                         std::to_string(k));
    return IMH_OK;
}

// The activation buffers of one schedule run (decode: the arena's B rows;
// prefill: B x T rows), T tokens per sequence, the attention lengths.
struct Rows {
    uint16_t *hidden, *residual, *norm_out, *q, *k, *v, *attn_out, *ffn_down, *act;
    uint32_t T;
    const int32_t *attn_lens;
};

int check_ready(const imh_decoder *d, const imh_stream *s, const uint32_t *token_ids, const uint16_t *logits,
                uint32_t token_count, const char *who) {
    if (!d || !s || !token_ids || !logits) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    if (token_count == 0) return imh::fail(IMH_EINVAL, std::string(who) + ": token_count 0");
    if (!d->model_set) return imh::fail(IMH_EINVAL, std::string(who) + ": model weights not set");
    for (uint32_t l = 0; l < d->cfg.num_layers; l++)
        if (!d->layer_set[l])
            return imh::fail(IMH_EINVAL, std::string(who) + ": layer " + std::to_string(l) + " weights not set");
    // the step guard of pipeline.rs:270-279 (and cache.rs:494-504)
    for (int32_t p : d->host_positions)
        if ((uint64_t)(uint32_t)p + token_count > d->cfg.max_seq_len)
            return imh::fail(IMH_ERANGE, std::string(who) + ": sequence position " + std::to_string(p) + " + " +
                                             std::to_string(token_count) + " token(s) beyond max_seq_len " +
                                             std::to_string(d->cfg.max_seq_len));
    return IMH_OK;
}

__global__ void prefill_lens_kernel(const int32_t *positions, int32_t *lens, int batch, int T) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < batch) lens[b] = positions[b] + T;
}

// out[b] = rows[b * T + T - 1] (H halfs each)
__global__ void gather_last_rows_kernel(const uint16_t *rows, uint16_t *out, int T, int H) {
    const int b = blockIdx.x;
    const uint16_t *src = rows + ((size_t)b * T + T - 1) * H;
    for (int i = threadIdx.x; i < H; i += blockDim.x) out[(size_t)b * H + i] = src[i];
}

// The per-layer schedule for T tokens per sequence (rows b * T + t) over the
// activation rows in r, attention lengths from r.attn_lens; logits of each
// sequence's last token.  T = 1 is the decode step.
int run_schedule(imh_decoder *d, imh_stream *s, const uint32_t *token_ids, const Rows &r, uint16_t *logits) {
    const imh_decoder_config &c = d->cfg;
    const uint32_t T = r.T, R = c.batch * r.T, H = c.hidden_size;
#define IMH_TRY(call)            \
    do {                         \
        int rc_ = (call);        \
        if (rc_) return rc_;     \
    } while (0)

    IMH_TRY(imh_encode_fused_embedding_norm(s, token_ids, d->embedding, d->layers[0].input_norm, r.norm_out,
                                            r.hidden, H, R, c.vocab_size, c.rms_eps, c.embed_scale));
    // Q, K and V read the same activation: when they share the AWQ scales
    // (or have none) they run as the row segments of one launch, which at a
    // layer's end also does the residual add and the input norm
    auto shared_awq = [](const imh_decoder_layer_weights &w) {
        return w.q_proj.awq_scales == w.k_proj.awq_scales && w.k_proj.awq_scales == w.v_proj.awq_scales;
    };
    uint16_t *qkv_out[3] = {r.q, r.k, r.v};
    bool q_done = false, kv_done = false;
    for (uint32_t l = 0; l < c.num_layers; l++) {
        const imh_decoder_layer_weights &w = d->layers[l];
        const imh_affine_int4_weight *qkv[3] = {&w.q_proj, &w.k_proj, &w.v_proj};
        if (!q_done && shared_awq(w)) {
            IMH_TRY(imh::encode_segmented_matvec_int4(s, r.norm_out, nullptr, R, 3, qkv, qkv_out));
            kv_done = true;
        } else if (!q_done) {
            IMH_TRY(imh_encode_affine_projection_int4(s, r.norm_out, R, &w.q_proj, r.q));
        }
        if (!kv_done) {
            if (w.k_proj.awq_scales == w.v_proj.awq_scales)
                IMH_TRY(imh::encode_segmented_matvec_int4(s, r.norm_out, nullptr, R, 2, qkv + 1, qkv_out + 1));
            else {
                IMH_TRY(imh_encode_affine_projection_int4(s, r.norm_out, R, &w.k_proj, r.k));
                IMH_TRY(imh_encode_affine_projection_int4(s, r.norm_out, R, &w.v_proj, r.v));
            }
        }
        imh_qk_norm_rope_params qp{};
        qp.q = r.q;
        qp.k = r.k;
        qp.q_norm = w.q_norm;
        qp.k_norm = w.k_norm;
        qp.cos_cache = d->rope_cos;
        qp.sin_cache = d->rope_sin;
        qp.num_heads = c.num_heads;
        qp.num_kv_heads = c.num_kv_heads;
        qp.head_dim = c.head_dim;
        qp.rotary_dim = c.rotary_dim;
        qp.max_pos = c.max_seq_len;
        qp.positions = d->positions;
        qp.batch = c.batch;
        qp.token_count = T;
        qp.eps = c.rms_eps;
        // TurboQuant: the token's cache write runs inside the attention launch;
        // with QK-norms at head_dim = rotary_dim = 128 so do the norm and
        // rotation of K (in the writing workgroup) and Q (in the prologue)
        const uint32_t win = d->windows[l];
        const bool fold = c.kv_cache == IMH_KV_TURBOQUANT && w.q_norm && w.k_norm && c.head_dim == 128 &&
                          (c.rotary_dim == 0 || c.rotary_dim == 128) && win == 0 && T == 1;
        if (win || T > 1) {
            // separate cache write and attention: a sliding-window layer
            // (attention.rs:141-163; its cache is a ring of `win` positions,
            // written at position % win, the attention bound being the ring's
            // size) or several tokens per sequence (token t at positions[b] + t
            // attends causally to [0, positions[b] + t + 1)).  RoPE uses the
            // absolute position.
            IMH_TRY(imh_encode_qk_norm_rope(s, &qp));
            if (c.kv_cache == IMH_KV_TURBOQUANT) {
                IMH_TRY(imh_encode_turboquant_cache_write_kv(s, d->tq, &d->tq_caches[l], r.k, r.v, T, 0,
                                                             d->positions));
                if (T == 1)
                    IMH_TRY(imh_encode_turboquant_attention(s, d->tq, &d->tq_caches[l], r.q, c.num_heads, 0,
                                                            r.attn_lens, c.attn_scale, r.attn_out, 0));
                else
                    IMH_TRY(imh_encode_turboquant_attention_tokens(s, d->tq, &d->tq_caches[l], r.q, c.num_heads, T,
                                                                   0, r.attn_lens, c.attn_scale, r.attn_out, 0));
            } else {
                const imh_fp16_kv_cache *kc = &d->fp16_caches[l];
                IMH_TRY(imh_encode_kv_scatter(s, kc, r.k, T, 0, d->positions, 1));
                IMH_TRY(imh_encode_kv_scatter(s, kc, r.v, T, 0, d->positions, 0));
                IMH_TRY(imh_encode_fp16_attention(s, kc, r.q, c.num_heads, T, 0, r.attn_lens, c.attn_scale,
                                                  r.attn_out, 0));
            }
        } else if (c.kv_cache == IMH_KV_TURBOQUANT) {
            if (!fold) IMH_TRY(imh_encode_qk_norm_rope(s, &qp));
            IMH_TRY(imh::encode_tq_write_attend(s, d->tq, &d->tq_caches[l], r.q, r.k, r.v, c.num_heads,
                                                r.attn_lens, c.attn_scale, r.attn_out, fold ? &qp : nullptr));
        } else {
            IMH_TRY(imh_encode_qk_norm_rope(s, &qp));
            const imh_fp16_kv_cache *kc = &d->fp16_caches[l];
            // no ring wrap: a step past the cache's end writes nothing
            IMH_TRY(imh::encode_kv_scatter_bounded(s, kc, r.k, d->positions, 1));
            IMH_TRY(imh::encode_kv_scatter_bounded(s, kc, r.v, d->positions, 0));
            IMH_TRY(imh_encode_fp16_attention(s, kc, r.q, c.num_heads, 1, 0, r.attn_lens, c.attn_scale,
                                              r.attn_out, 0));
        }
        IMH_TRY(imh_encode_affine_projection_int4(s, r.attn_out, R, &w.o_proj, r.ffn_down));
        {   // post-attention residual + norm, then gate + up + activation (one
            // launch), then down (at 1-2 rows from the operand image gate/up wrote)
            imh_fused_residual_norm_params rp{};
            rp.a = r.hidden;
            rp.b = r.ffn_down;
            rp.norm_weight = w.post_attn_norm;
            rp.residual_output = r.residual;
            rp.normed_output = r.norm_out;
            rp.token_count = R;
            rp.eps = c.rms_eps;
            IMH_TRY(imh::encode_resnorm_ffn_block_int4(s, &rp, R, &w.gate_proj, &w.up_proj, &w.down_proj, r.act,
                                                       r.ffn_down, c.use_gelu));
        }
        if (l + 1 < c.num_layers) {
            const imh_decoder_layer_weights &nw = d->layers[l + 1];
            imh_fused_residual_norm_params fp{};
            fp.a = r.residual;
            fp.b = r.ffn_down;
            fp.norm_weight = nw.input_norm;
            fp.residual_output = r.hidden;
            fp.weight = &nw.q_proj;
            fp.output = r.q;
            fp.normed_output = r.norm_out;
            fp.token_count = R;
            fp.eps = c.rms_eps;
            kv_done = shared_awq(nw);
            if (kv_done) {
                const imh_affine_int4_weight *nqkv[3] = {&nw.q_proj, &nw.k_proj, &nw.v_proj};
                IMH_TRY(imh::encode_segmented_matvec_int4(s, nullptr, &fp, R, 3, nqkv, qkv_out));
            } else {
                IMH_TRY(imh_encode_fused_residual_norm_affine_matvec_int4(s, &fp));
            }
            q_done = true;
        } else {
            IMH_TRY(imh_encode_residual_add(s, r.residual, r.ffn_down, r.hidden, (size_t)R * H));
        }
    }
    const uint16_t *last = r.hidden;
    if (T > 1) {   // each sequence's last token
        hipLaunchKernelGGL(gather_last_rows_kernel, dim3(c.batch), dim3(256), 0, s->stream, r.hidden, d->hidden,
                           (int)T, (int)H);
        IMH_HIP(hipGetLastError());
        last = d->hidden;
    }
    IMH_TRY(imh_encode_rms_norm(s, last, d->final_norm, d->norm_out, H, c.batch, c.rms_eps));
    IMH_TRY(imh_encode_affine_projection_int4(s, d->norm_out, c.batch, &d->lm_head, logits));
#undef IMH_TRY
    return IMH_OK;
}

}  // namespace

extern "C" {

int imh_decoder_create(imh_device *dev, const imh_decoder_config *cfg, imh_decoder **out) {
    const char *who = "imh_decoder_create";
    if (!dev || !cfg || !out) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    *out = nullptr;
    const imh_decoder_config &c = *cfg;
    if (!c.hidden_size || !c.intermediate_size || !c.num_layers || !c.num_heads || !c.num_kv_heads ||
        !c.head_dim || !c.vocab_size || !c.max_seq_len || !c.batch)
        return imh::fail(IMH_EINVAL, std::string(who) + ": zero dimension in the config");
    if (c.num_heads % c.num_kv_heads)
        return imh::fail(IMH_EINVAL, std::string(who) + ": num_heads must be a multiple of num_kv_heads");
    if (c.kv_cache != IMH_KV_TURBOQUANT && c.kv_cache != IMH_KV_FP16)
        return imh::fail(IMH_EINVAL, std::string(who) + ": unknown kv_cache kind");
    if (c.batch > 65535) return imh::fail(IMH_EINVAL, std::string(who) + ": batch above 65535");
    if (c.window_sizes)
        for (uint32_t l = 0; l < c.num_layers; l++)
            if (c.window_sizes[l] > c.max_seq_len)
                return imh::fail(IMH_EINVAL, std::string(who) + ": layer " + std::to_string(l) +
                                                 " window_size above max_seq_len");
    int rc = imh::use_device(dev);
    if (rc) return rc;

    imh_decoder *d = new imh_decoder();
    d->windows.assign(c.num_layers, 0);
    if (c.window_sizes) d->windows.assign(c.window_sizes, c.window_sizes + c.num_layers);
    d->cfg.window_sizes = nullptr;   // the decoder keeps its own copy
    d->dev = dev;
    d->cfg = c;
    if (d->cfg.attn_scale == 0.0f) d->cfg.attn_scale = 1.0f / std::sqrt((float)c.head_dim);
    if (d->cfg.embed_scale == 0.0f) d->cfg.embed_scale = 1.0f;
    d->layers.resize(c.num_layers);
    d->layer_set.assign(c.num_layers, false);
    d->host_positions.assign(c.batch, 0);

    const size_t B = c.batch, H = c.hidden_size, F = c.intermediate_size;
    const size_t qd = (size_t)c.num_heads * c.head_dim, kvd = (size_t)c.num_kv_heads * c.head_dim;
    const size_t half_dim = c.head_dim / 2;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    const size_t o_hidden = take(B * H * 2), o_res = take(B * H * 2), o_norm = take(B * H * 2);
    const size_t o_q = take(B * qd * 2), o_k = take(B * kvd * 2), o_v = take(B * kvd * 2);
    const size_t o_attn = take(B * qd * 2), o_down = take(B * H * 2), o_act = take(B * F * 2);
    const size_t o_pos = take(B * 4), o_sl = take(B * 4), o_st = take(4);
    const size_t o_cos = take((size_t)c.max_seq_len * half_dim * 2), o_sin = take((size_t)c.max_seq_len * half_dim * 2);
    hipError_t e = hipMalloc(&d->arena, off);
    if (e != hipSuccess) {
        delete d;
        return imh::fail(IMH_ENOMEM, std::string(who) + ": activation arena of " + std::to_string(off) + " bytes");
    }
    char *base = static_cast<char *>(d->arena);
    d->hidden = reinterpret_cast<uint16_t *>(base + o_hidden);
    d->residual = reinterpret_cast<uint16_t *>(base + o_res);
    d->norm_out = reinterpret_cast<uint16_t *>(base + o_norm);
    d->q = reinterpret_cast<uint16_t *>(base + o_q);
    d->k = reinterpret_cast<uint16_t *>(base + o_k);
    d->v = reinterpret_cast<uint16_t *>(base + o_v);
    d->attn_out = reinterpret_cast<uint16_t *>(base + o_attn);
    d->ffn_down = reinterpret_cast<uint16_t *>(base + o_down);
    d->act = reinterpret_cast<uint16_t *>(base + o_act);
    d->positions = reinterpret_cast<int32_t *>(base + o_pos);
    d->seq_lens = reinterpret_cast<int32_t *>(base + o_sl);
    d->status = reinterpret_cast<int32_t *>(base + o_st);
    d->rope_cos = reinterpret_cast<uint16_t *>(base + o_cos);
    d->rope_sin = reinterpret_cast<uint16_t *>(base + o_sin);

    auto cleanup = [&](int code) {
        imh_decoder_free(d);
        return code;
    };
    // RoPE tables (rope.rs:22-50), built on the host once
    {
        std::vector<uint16_t> cs((size_t)c.max_seq_len * half_dim), sn(cs.size());
        rc = imh_rope_cache_fill(c.head_dim, c.max_seq_len, c.rope_theta, c.rotary_dim, cs.data(), sn.data());
        if (rc) return cleanup(rc);
        e = hipMemcpy(d->rope_cos, cs.data(), cs.size() * 2, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(d->rope_sin, sn.data(), sn.size() * 2, hipMemcpyHostToDevice);
        if (e != hipSuccess) return cleanup(imh::hip_fail(e, "imh_decoder_create: RoPE upload"));
    }
    e = hipMemset(d->arena, 0, o_cos);
    if (e != hipSuccess) return cleanup(imh::hip_fail(e, "imh_decoder_create: clear"));
    {
        std::vector<int32_t> sl(B, 1);
        e = hipMemcpy(d->seq_lens, sl.data(), B * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) return cleanup(imh::hip_fail(e, "imh_decoder_create: seq_lens"));
    }

    // KV caches: one allocation for every layer, zeroed; a layer's positions:
    // max_seq_len, or its window (the buffer stride of a sliding-window layer,
    // effective_max_seq_len, turboquant/cache.rs:394-400)
    if (c.kv_cache == IMH_KV_TURBOQUANT) {
        rc = imh_tq_tables_create(dev, c.head_dim, 8, c.tq_seed, &d->own_tq);
        if (rc) return cleanup(rc);
        d->tq = d->own_tq;
    }
    auto stride_of = [&](uint32_t l) { return d->windows[l] ? d->windows[l] : c.max_seq_len; };
    auto layer_bytes = [&](uint32_t l) {
        const size_t rows = B * c.num_kv_heads * (size_t)stride_of(l);
        return c.kv_cache == IMH_KV_TURBOQUANT ? 2 * align256(rows * c.head_dim) + 3 * align256(rows * 4)
                                               : 2 * align256(rows * c.head_dim * 2);
    };
    size_t kv_bytes = 0;
    for (uint32_t l = 0; l < c.num_layers; l++) kv_bytes += layer_bytes(l);
    e = hipMalloc(&d->kv_arena, kv_bytes);
    if (e != hipSuccess)
        return cleanup(imh::fail(IMH_ENOMEM, std::string(who) + ": KV cache of " + std::to_string(kv_bytes) + " bytes"));
    e = hipMemset(d->kv_arena, 0, kv_bytes);
    if (e != hipSuccess) return cleanup(imh::hip_fail(e, "imh_decoder_create: KV clear"));
    char *kv = static_cast<char *>(d->kv_arena);
    for (uint32_t l = 0; l < c.num_layers; l++) {
        char *p = kv;
        kv += layer_bytes(l);
        const size_t rows = B * c.num_kv_heads * (size_t)stride_of(l);
        if (c.kv_cache == IMH_KV_TURBOQUANT) {
            imh_tq_kv_cache t{};
            t.k_codes = reinterpret_cast<uint8_t *>(p);
            p += align256(rows * c.head_dim);
            t.v_codes = reinterpret_cast<uint8_t *>(p);
            p += align256(rows * c.head_dim);
            t.k_scales = reinterpret_cast<float *>(p);
            p += align256(rows * 4);
            t.v_scales = reinterpret_cast<float *>(p);
            p += align256(rows * 4);
            t.k_r_norms = reinterpret_cast<float *>(p);
            t.batch = c.batch;
            t.num_kv_heads = c.num_kv_heads;
            t.head_dim = c.head_dim;
            t.max_seq_len = stride_of(l);
            d->tq_caches.push_back(t);
        } else {
            imh_fp16_kv_cache f{};
            f.k = reinterpret_cast<uint16_t *>(p);
            f.v = reinterpret_cast<uint16_t *>(p + align256(rows * c.head_dim * 2));
            f.batch = c.batch;
            f.num_kv_heads = c.num_kv_heads;
            f.head_dim = c.head_dim;
            f.max_seq_len = stride_of(l);
            d->fp16_caches.push_back(f);
        }
    }
    *out = d;
    return IMH_OK;
}

void imh_decoder_free(imh_decoder *d) {
    if (!d) return;
    imh::use_device(d->dev);
    if (d->arena) (void)hipFree(d->arena);
    if (d->kv_arena) (void)hipFree(d->kv_arena);
    if (d->prefill_arena) (void)hipFree(d->prefill_arena);
    if (d->own_tq) imh_tq_tables_free(d->own_tq);
    delete d;
}

int imh_decoder_set_layer(imh_decoder *d, uint32_t layer, const imh_decoder_layer_weights *w) {
    if (!d || !w) return imh::fail(IMH_EINVAL, "imh_decoder_set_layer: NULL argument");
    const imh_decoder_config &c = d->cfg;
    if (layer >= c.num_layers) return imh::fail(IMH_EINVAL, "imh_decoder_set_layer: layer out of range");
    if (!w->input_norm || !w->post_attn_norm)
        return imh::fail(IMH_EINVAL, "imh_decoder_set_layer: NULL norm weight");
    if (!w->q_norm != !w->k_norm)
        return imh::fail(IMH_EINVAL, "imh_decoder_set_layer: give both QK-norm weights or none");
    const uint32_t H = c.hidden_size, F = c.intermediate_size;
    const uint32_t qd = c.num_heads * c.head_dim, kvd = c.num_kv_heads * c.head_dim;
    int rc = check_weight(w->q_proj, qd, H, "q_proj");
    if (!rc) rc = check_weight(w->k_proj, kvd, H, "k_proj");
    if (!rc) rc = check_weight(w->v_proj, kvd, H, "v_proj");
    if (!rc) rc = check_weight(w->o_proj, H, qd, "o_proj");
    if (!rc) rc = check_weight(w->gate_proj, F, H, "gate_proj");
    if (!rc) rc = check_weight(w->up_proj, F, H, "up_proj");
    if (!rc) rc = check_weight(w->down_proj, H, F, "down_proj");
    if (rc) return rc;
    d->layers[layer] = *w;
    d->layer_set[layer] = true;
    return IMH_OK;
}

int imh_decoder_set_model(imh_decoder *d, const uint16_t *embedding, const uint16_t *final_norm,
                          const imh_affine_int4_weight *lm_head) {
    if (!d || !embedding || !final_norm || !lm_head) return imh::fail(IMH_EINVAL, "imh_decoder_set_model: NULL argument");
    int rc = check_weight(*lm_head, d->cfg.vocab_size, d->cfg.hidden_size, "lm_head");
    if (rc) return rc;
    d->embedding = embedding;
    d->final_norm = final_norm;
    d->lm_head = *lm_head;
    d->model_set = true;
    return IMH_OK;
}

int imh_decoder_reset(imh_decoder *d, imh_stream *stream, const int32_t *positions) {
    if (!d || !stream) return imh::fail(IMH_EINVAL, "imh_decoder_reset: NULL argument");
    if (stream->capturing) return imh::fail(IMH_EINVAL, "imh_decoder_reset: not allowed while capturing");
    const uint32_t B = d->cfg.batch;
    std::vector<int32_t> pos(B, 0), sl(B);
    for (uint32_t b = 0; b < B; b++) {
        if (positions) pos[b] = positions[b];
        if (pos[b] < 0 || (uint32_t)pos[b] >= d->cfg.max_seq_len)
            return imh::fail(IMH_ERANGE, "imh_decoder_reset: position " + std::to_string(pos[b]) +
                                             " outside the cache of " + std::to_string(d->cfg.max_seq_len));
        sl[b] = pos[b] + 1;
    }
    int rc = imh::use_device(d->dev);
    if (rc) return rc;
    const int32_t zero = 0;
    IMH_HIP(hipMemcpyAsync(d->positions, pos.data(), B * 4, hipMemcpyHostToDevice, stream->stream));
    IMH_HIP(hipMemcpyAsync(d->seq_lens, sl.data(), B * 4, hipMemcpyHostToDevice, stream->stream));
    IMH_HIP(hipMemcpyAsync(d->status, &zero, 4, hipMemcpyHostToDevice, stream->stream));
    IMH_HIP(hipStreamSynchronize(stream->stream));
    d->host_positions = pos;
    return IMH_OK;
}

int imh_decoder_step(imh_decoder *d, imh_stream *s, const uint32_t *token_ids, uint16_t *logits) {
    const char *who = "imh_decoder_step";
    int rc = check_ready(d, s, token_ids, logits, 1, who);
    if (rc) return rc;
    rc = imh::use_device(d->dev);
    if (rc) return rc;
    const imh_decoder_config &c = d->cfg;
    const uint32_t B = c.batch;
    Rows r{d->hidden, d->residual, d->norm_out, d->q, d->k, d->v, d->attn_out, d->ffn_down, d->act, 1, d->seq_lens};
    rc = run_schedule(d, s, token_ids, r, logits);
    if (rc) return rc;
    hipLaunchKernelGGL(decoder_advance_kernel, dim3((B + 63) / 64), dim3(64), 0, s->stream, d->positions, d->seq_lens,
                       d->status, (int)B, (int)c.max_seq_len, 1);
    IMH_HIP(hipGetLastError());
    // a captured step runs only when replayed: the mirror follows eager steps
    if (!s->capturing)
        for (auto &p : d->host_positions) p++;
    return IMH_OK;
}

int imh_decoder_prefill(imh_decoder *d, imh_stream *s, const uint32_t *token_ids, uint32_t token_count,
                        uint16_t *logits) {
    const char *who = "imh_decoder_prefill";
    int rc = check_ready(d, s, token_ids, logits, token_count, who);
    if (rc) return rc;
    if (token_count == 1) return imh_decoder_step(d, s, token_ids, logits);
    const imh_decoder_config &c = d->cfg;
    for (uint32_t l = 0; l < c.num_layers; l++)
        if (d->windows[l] && token_count > d->windows[l])
            return imh::fail(IMH_EINVAL, std::string(who) + ": token_count above layer " + std::to_string(l) +
                                             "'s window (" + std::to_string(d->windows[l]) + ")");
    const uint32_t B = c.batch, T = token_count, R = B * T;
    if (R > 65535) return imh::fail(IMH_EINVAL, std::string(who) + ": batch x token_count above 65535");
    rc = imh::use_device(d->dev);
    if (rc) return rc;
    // activation rows for R tokens, grown on demand (not while capturing)
    const size_t H = c.hidden_size, F = c.intermediate_size;
    const size_t qd = (size_t)c.num_heads * c.head_dim, kvd = (size_t)c.num_kv_heads * c.head_dim;
    const size_t need = align256(R * H * 2) * 4 + align256(R * qd * 2) * 2 + align256(R * kvd * 2) * 2 +
                        align256(R * F * 2) + align256(B * 4);
    if (need > d->prefill_bytes) {
        if (s->capturing)
            return imh::fail(IMH_EINVAL, std::string(who) + ": needs " + std::to_string(need) +
                                             " bytes of activation rows; run a prefill of this size before capturing");
        if (d->prefill_arena) {
            // earlier work on any stream may still read the old rows
            IMH_HIP(hipDeviceSynchronize());
            (void)hipFree(d->prefill_arena);
            d->prefill_arena = nullptr;
            d->prefill_bytes = 0;
        }
        hipError_t e = hipMalloc(&d->prefill_arena, need);
        if (e != hipSuccess)
            return imh::fail(IMH_ENOMEM, std::string(who) + ": activation rows of " + std::to_string(need) + " bytes");
        d->prefill_bytes = need;
    }
    char *p = static_cast<char *>(d->prefill_arena);
    auto take = [&](size_t bytes) {
        char *o = p;
        p += align256(bytes);
        return o;
    };
    Rows r{};
    r.hidden = reinterpret_cast<uint16_t *>(take(R * H * 2));
    r.residual = reinterpret_cast<uint16_t *>(take(R * H * 2));
    r.norm_out = reinterpret_cast<uint16_t *>(take(R * H * 2));
    r.q = reinterpret_cast<uint16_t *>(take(R * qd * 2));
    r.k = reinterpret_cast<uint16_t *>(take(R * kvd * 2));
    r.v = reinterpret_cast<uint16_t *>(take(R * kvd * 2));
    r.attn_out = reinterpret_cast<uint16_t *>(take(R * qd * 2));
    r.ffn_down = reinterpret_cast<uint16_t *>(take(R * H * 2));
    r.act = reinterpret_cast<uint16_t *>(take(R * F * 2));
    r.T = T;
    int32_t *lens = reinterpret_cast<int32_t *>(take(B * 4));
    r.attn_lens = lens;
    // the chunk's attention length: positions[b] + T
    hipLaunchKernelGGL(prefill_lens_kernel, dim3((B + 63) / 64), dim3(64), 0, s->stream, d->positions, lens, (int)B,
                       (int)T);
    IMH_HIP(hipGetLastError());
    rc = run_schedule(d, s, token_ids, r, logits);
    if (rc) return rc;
    hipLaunchKernelGGL(decoder_advance_kernel, dim3((B + 63) / 64), dim3(64), 0, s->stream, d->positions, d->seq_lens,
                       d->status, (int)B, (int)c.max_seq_len, (int)T);
    IMH_HIP(hipGetLastError());
    if (!s->capturing)
        for (auto &q : d->host_positions) q += (int32_t)T;
    return IMH_OK;
}

int imh_decoder_write_kv(imh_decoder *d, imh_stream *s, uint32_t layer, const uint16_t *k_proj,
                         const uint16_t *v_proj, uint32_t token_count, uint32_t base_pos) {
    if (!d || !s || !k_proj || !v_proj) return imh::fail(IMH_EINVAL, "imh_decoder_write_kv: NULL argument");
    if (layer >= d->cfg.num_layers) return imh::fail(IMH_EINVAL, "imh_decoder_write_kv: layer out of range");
    if ((uint64_t)base_pos + token_count > d->cfg.max_seq_len)
        return imh::fail(IMH_ERANGE, "imh_decoder_write_kv: base_pos + token_count beyond max_seq_len");
    // a windowed layer's ring takes positions modulo its window (the cache
    // write wraps at the cache's max_seq_len); more tokens than the ring holds
    // would overwrite each other within one write
    if (d->windows[layer] && token_count > d->windows[layer])
        return imh::fail(IMH_EINVAL, "imh_decoder_write_kv: token_count above the layer's window");
    if (d->cfg.kv_cache == IMH_KV_TURBOQUANT) {
        return imh_encode_turboquant_cache_write_kv(s, d->tq, &d->tq_caches[layer], k_proj, v_proj, token_count,
                                                    base_pos, nullptr);
    }
    int rc = imh_encode_kv_scatter(s, &d->fp16_caches[layer], k_proj, token_count, base_pos, nullptr, 1);
    if (rc) return rc;
    return imh_encode_kv_scatter(s, &d->fp16_caches[layer], v_proj, token_count, base_pos, nullptr, 0);
}

int imh_decoder_positions(const imh_decoder *d, int32_t *out) {
    if (!d || !out) return imh::fail(IMH_EINVAL, "imh_decoder_positions: NULL argument");
    std::memcpy(out, d->host_positions.data(), d->host_positions.size() * 4);
    return IMH_OK;
}

int imh_decoder_sync_positions(imh_decoder *d, imh_stream *stream, int32_t *out) {
    const char *who = "imh_decoder_sync_positions";
    if (!d || !stream) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    if (stream->capturing) return imh::fail(IMH_EINVAL, std::string(who) + ": not allowed while capturing");
    int rc = imh::use_device(d->dev);
    if (rc) return rc;
    const uint32_t B = d->cfg.batch;
    std::vector<int32_t> pos(B);
    int32_t st = 0;
    IMH_HIP(hipMemcpyAsync(pos.data(), d->positions, B * 4, hipMemcpyDeviceToHost, stream->stream));
    IMH_HIP(hipMemcpyAsync(&st, d->status, 4, hipMemcpyDeviceToHost, stream->stream));
    IMH_HIP(hipStreamSynchronize(stream->stream));
    d->host_positions = pos;
    if (out) std::memcpy(out, pos.data(), B * 4);
    if (st)
        return imh::fail(IMH_ERANGE, std::string(who) + ": a step ran with a sequence at max_seq_len " +
                                         std::to_string(d->cfg.max_seq_len) +
                                         " (its logits are invalid; reset the decoder)");
    return IMH_OK;
}

int imh_decoder_kv_cache(const imh_decoder *d, uint32_t layer, imh_tq_kv_cache *tq_out, imh_fp16_kv_cache *fp16_out) {
    if (!d) return imh::fail(IMH_EINVAL, "imh_decoder_kv_cache: NULL decoder");
    if (layer >= d->cfg.num_layers) return imh::fail(IMH_EINVAL, "imh_decoder_kv_cache: layer out of range");
    if (d->cfg.kv_cache == IMH_KV_TURBOQUANT) {
        if (!tq_out) return imh::fail(IMH_EINVAL, "imh_decoder_kv_cache: TurboQuant cache needs tq_out");
        *tq_out = d->tq_caches[layer];
    } else {
        if (!fp16_out) return imh::fail(IMH_EINVAL, "imh_decoder_kv_cache: FP16 cache needs fp16_out");
        *fp16_out = d->fp16_caches[layer];
    }
    return IMH_OK;
}

int imh_decoder_set_tq_tables(imh_decoder *d, imh_tq_tables *t) {
    const char *who = "imh_decoder_set_tq_tables";
    if (!d || !t) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    if (d->cfg.kv_cache != IMH_KV_TURBOQUANT)
        return imh::fail(IMH_EINVAL, std::string(who) + ": the decoder has an FP16 KV cache");
    if (t->dev->ordinal != d->dev->ordinal)
        return imh::fail(IMH_EINVAL, std::string(who) + ": tables live on another device");
    if (t->head_dim != d->cfg.head_dim || t->n_bits != 8)
        return imh::fail(IMH_EINVAL, std::string(who) + ": tables are for head_dim " + std::to_string(t->head_dim) +
                                         ", " + std::to_string(t->n_bits) + " bits; the cache needs head_dim " +
                                         std::to_string(d->cfg.head_dim) + ", 8 bits");
    d->tq = t;
    return IMH_OK;
}

int imh_decoder_tq_tables(const imh_decoder *d, imh_tq_tables **out) {
    if (!d || !out) return imh::fail(IMH_EINVAL, "imh_decoder_tq_tables: NULL argument");
    *out = d->tq;
    return IMH_OK;
}

}  // extern "C"
