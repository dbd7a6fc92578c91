// imh_internal.h -- shared host-side definitions of libironmill_hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/ironmill_hip.h"

namespace imh {

// Thread-local last-error text (ironmill-compile-ffi/src/lib.rs:69-79 pattern).
int fail(int code, const std::string &msg);
int hip_fail(hipError_t e, const char *what);
void clear_error();

#define IMH_HIP(call)                                  \
    do {                                               \
        hipError_t e_ = (call);                        \
        if (e_ != hipSuccess) return imh::hip_fail(e_, #call); \
    } while (0)

// One token per sequence scattered into an FP16 cache at device positions
// without the ring wrap (positions at or past max_seq_len write nothing).
int encode_kv_scatter_bounded(imh_stream *stream, const imh_fp16_kv_cache *cache, const uint16_t *proj,
                              const int32_t *positions, int is_k);

}  // namespace imh

struct imh_device {
    int ordinal;
    hipDeviceProp_t props;
};

struct imh_buffer {
    imh_device *dev;
    void *ptr;
    size_t length;
};

// Per-stream scratch memory, grown on demand by the host code of an op.
// Slot 0: INT4 activation operand images, the query operand planes of the
// TurboQuant prefill attention; slot 1: attention split partials,
// the gate output of a prefill gate/up op; slot 2: GEMM and INT4 matvec split-K partials.
// A graph captured on the stream records the slots' addresses, so a slot that
// grows later keeps its old block alive (`retired`) until the stream is freed:
// a replay never touches freed memory.
constexpr int kScratchSlots = 3;
struct imh_stream {
    imh_device *dev;
    hipStream_t stream;
    void *scratch[kScratchSlots];
    size_t scratch_bytes[kScratchSlots];
    bool capturing;
    std::vector<void *> retired;
};

// A captured graph replays on the stream it was captured on only: its kernels
// use that stream's scratch slots (partials, arrival counters), which another
// stream's work could use at the same time.
struct imh_graph {
    imh_device *dev;
    hipGraph_t graph;
    hipGraphExec_t exec;
    imh_stream *stream;
};

struct imh_event {
    imh_device *dev;
    hipEvent_t ev;
};

struct imh_tq_tables {
    imh_device *dev;
    uint32_t head_dim;
    uint32_t n_bits;
    // one device allocation holding all tables, f32:
    //   signs[d] | k_cb[2^(b-1)] | k_bd[2^(b-1)-1] | v_cb[2^b] | v_bd[2^b-1] | qjl[d*d] | qjl_t[d*d]
    float *base;
    float *signs, *k_codebook, *k_bounds, *v_codebook, *v_bounds, *qjl, *qjl_t;
    size_t total_floats;
    // Exact fast form of the reference's index rule idx = 1 + max{j : u >= bd[j]}
    // (0 if none), for any boundary order: the boundaries sorted by value (NaN
    // dropped) with the running maximum of j + 1; idx = prefix max at
    // upper_bound(u), 0 at position 0.  One device allocation:
    //   k_sorted[k_search] f32 | k_prefmax[k_search] i32 | v_sorted | v_prefmax
    void *search_base;
    const float *k_sorted, *v_sorted;
    const int32_t *k_prefmax, *v_prefmax;
    int k_search, v_search;
};

namespace imh {

// Ensure scratch slot `slot` of the stream holds at least `bytes`.  A smaller
// block is replaced, not freed: graphs captured earlier may still address it.
int stream_scratch(imh_stream *s, int slot, size_t bytes, void **out);

// Make the stream's device current for the calling thread.
int use_device(const imh_device *dev);

// Look up, once per device, the address of the fixed scratch array that
// imh_encode_turboquant_attention_noalloc uses (called when a device opens).
int noalloc_scratch_init(int ordinal);

// Projections of one activation by up to three INT4 weights that share k and
// the AWQ scales (a layer's Q, K and V), as the row segments of one matvec
// launch: out[i] = act . w[i]^T.  The activation is x, or, when rn is given,
// the fused residual + RMSNorm of rn->a + rn->b (whose residual and normed
// rows are written as by imh_encode_fused_residual_norm_affine_matvec_int4;
// rn->weight and rn->output are not read): w[0] projects it as that op does,
// the other weights project the f16 normed rows.  Every segment but the last
// has a multiple of 16 rows.  Prefill-sized batches run one op per weight.
int encode_segmented_matvec_int4(imh_stream *s, const uint16_t *x, const imh_fused_residual_norm_params *rn,
                                 uint32_t B, int nseg, const imh_affine_int4_weight *const *w,
                                 uint16_t *const *out);

// The fused residual + RMSNorm of rn->a + rn->b (residual and normed rows
// written as by imh_encode_fused_residual_norm_affine_matvec_int4; rn->weight
// and rn->output are not read) feeding the fused gate + up + SiLU/GELU of
// imh_encode_fused_ffn_gate_up_act_int4 with the f16 normed rows as its
// input (as after a separate norm), in one launch below 32 tokens.
int encode_resnorm_gate_up_act_int4(imh_stream *s, const imh_fused_residual_norm_params *rn, uint32_t B,
                                    const imh_affine_int4_weight *gate, const imh_affine_int4_weight *up,
                                    uint16_t *out, int use_gelu);
// The residual + norm, gate/up + activation and down projection of a decoder
// layer's FFN: at 1-2 rows on the row-band kernel the gate/up launch hands
// down its operand image; otherwise the two ops.
int encode_resnorm_ffn_block_int4(imh_stream *s, const imh_fused_residual_norm_params *rn, uint32_t B,
                                  const imh_affine_int4_weight *gate, const imh_affine_int4_weight *up,
                                  const imh_affine_int4_weight *down, uint16_t *act, uint16_t *y, int use_gelu);

// The step's token written to the TurboQuant cache at row seq_lens[b] - 1
// and attended over [0, seq_lens[b]) in one launch (the write runs in one
// extra workgroup per (kv head, sequence) beside the attention splits).  With
// qk (head_dim = rotary_dim = 128, both norms, positions[b] = seq_lens[b] - 1)
// Q and K go through the QK-norm + RoPE inside the launch.
int encode_tq_write_attend(imh_stream *stream, const imh_tq_tables *t, const imh_tq_kv_cache *cache,
                           const uint16_t *q, const uint16_t *k_proj, const uint16_t *v_proj, uint32_t num_heads,
                           const int32_t *seq_lens, float attn_scale, uint16_t *out,
                           const imh_qk_norm_rope_params *qk);

// One token per sequence scattered into an FP16 cache at device positions
// without the ring wrap (positions at or past max_seq_len write nothing).
int encode_kv_scatter_bounded(imh_stream *stream, const imh_fp16_kv_cache *cache, const uint16_t *proj,
                              const int32_t *positions, int is_k);

}  // namespace imh
