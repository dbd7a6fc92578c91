/*
 * ironmill_hip.h -- C ABI of the MI355X (gfx950) quantized-decode backend.
 *
 * Two tiers, mirroring jafreck/ironmill's Metal backend boundary
 * (paths below are under the reference's crates/):
 *
 *  1. Runtime tier -- the counterpart of ironmill-metal-sys
 *     (ironmill-metal-sys/src/{device,buffer,command}.rs): device, buffers
 *     with bounds-checked read/write, in-order streams (command queues) and
 *     timing events.
 *  2. Op tier -- the counterpart of the Metal op encoders in
 *     ironmill-inference/src/metal/{projection.rs, ops/quantized.rs,
 *     ops/fused.rs, attention.rs}: every entry point enqueues work on a
 *     stream and returns immediately.
 *
 * Conventions (from ironmill-compile-ffi/src/lib.rs:13-31,69-79,446):
 *  - int status: IMH_OK (0) or a negative IMH_E* code; the thread-local
 *    message of the last failure is returned by imh_last_error().
 *  - every allocating call has a matching *_free; no C++ exception crosses
 *    the ABI.
 *  - op arguments are plain device pointers (any allocation on the stream's
 *    device: imh_buffer_device_ptr(), hipMalloc, a torch tensor's data_ptr)
 *    plus sizes.  f16 data is IEEE binary16 passed as uint16_t.
 *  - a stream must not be used from two threads at once (the analogue of a
 *    Metal ComputeEncoder being Send but not Sync, command.rs:339); handles
 *    may move between threads.
 *  - the library allocates per-stream scratch memory lazily (first op that
 *    needs it, or growth); the kernels themselves never allocate.
 */
#ifndef IRONMILL_HIP_H
#define IRONMILL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IMH_OK 0
#define IMH_EINVAL (-1)       /* bad argument (MetalSysError::InvalidArgument, error.rs:4-41) */
#define IMH_EUNSUPPORTED (-2) /* valid but not implemented here (e.g. group_size != 128) */
#define IMH_EDEVICE (-3)      /* HIP runtime failure */
#define IMH_ENOMEM (-4)       /* device allocation failed */
#define IMH_ERANGE (-5)       /* sequence position beyond the cache (cache.rs:494-504) */

typedef struct imh_device imh_device;
typedef struct imh_buffer imh_buffer;
typedef struct imh_stream imh_stream;
typedef struct imh_event imh_event;
typedef struct imh_tq_tables imh_tq_tables;

/* Thread-local message of the last failed call on this thread
 * (ironmill-compile-ffi/src/lib.rs:69-79 mil_last_error). Never NULL. */
const char *imh_last_error(void);

/* ===================== runtime tier (ironmill-metal-sys) ===================== */

typedef struct {
    int ordinal;
    int compute_units;
    int wavefront_size;
    int clock_khz;
    size_t total_global_mem;
    size_t lds_per_block;
    char arch[64]; /* e.g. "gfx950:sramecc+:xnack-" */
} imh_device_info;

/* MetalDevice::system_default (device.rs:74-96) generalised to an ordinal. */
int imh_device_count(int *count);
int imh_device_open(int ordinal, imh_device **out);
void imh_device_free(imh_device *dev);
/* recommended_max_working_set / device queries (device.rs:380-395) */
int imh_device_get_info(const imh_device *dev, imh_device_info *out);

/* MetalDevice::create_buffer / create_buffer_with_data (device.rs:105-160) */
int imh_buffer_alloc(imh_device *dev, size_t length, imh_buffer **out);
int imh_buffer_alloc_with_data(imh_device *dev, const void *data, size_t length,
                               imh_buffer **out);
void imh_buffer_free(imh_buffer *buf);
/* MetalBuffer::length / contents (buffer.rs:60-93); the pointer is a device address */
size_t imh_buffer_length(const imh_buffer *buf);
void *imh_buffer_device_ptr(const imh_buffer *buf);
/* MetalBuffer::write_bytes / read_bytes (buffer.rs:95-158): synchronous,
 * IMH_EINVAL when offset+length exceeds the buffer. */
int imh_buffer_write(imh_buffer *buf, size_t offset, const void *src, size_t length);
int imh_buffer_read(const imh_buffer *buf, size_t offset, void *dst, size_t length);
/* Synchronous copy of device memory the library handed out by pointer (a
 * decoder's KV cache) to the host (MetalBuffer::read_bytes, buffer.rs:130-158,
 * for memory without a buffer handle). */
int imh_copy_to_host(imh_device *dev, void *dst, const void *src, size_t length);

/* CommandQueue / CommandBuffer (command.rs:16-130): one in-order HIP stream
 * at default priority.  imh_stream_sync = commit + wait_until_completed. */
int imh_stream_create(imh_device *dev, imh_stream **out);
void imh_stream_free(imh_stream *stream);
int imh_stream_sync(imh_stream *stream);
void *imh_stream_native(imh_stream *stream); /* the hipStream_t */
/* Zero `length` bytes at a device pointer with a fill kernel (capturable). */
int imh_fill_zero(imh_stream *stream, void *dst, size_t length);

/* Recorded command sequence: ops encoded on a stream between begin and end
 * capture are recorded (not run) into a HIP graph, which can then be replayed
 * with one launch -- the counterpart of encoding a whole decode step into one
 * Metal command buffer and committing it (pipeline.rs:336-343,1205-1213).
 * Scratch memory an op needs must already exist (run it once before capture);
 * capture fails with IMH_EINVAL otherwise.  A graph replays only on the stream
 * it was captured on (IMH_EINVAL otherwise: its kernels use that stream's
 * scratch memory), and must be freed before that stream.  Scratch that grows
 * after a capture keeps its old blocks until imh_stream_free, so a replay
 * never addresses freed memory. */
typedef struct imh_graph imh_graph;
int imh_stream_begin_capture(imh_stream *stream);
int imh_stream_end_capture(imh_stream *stream, imh_graph **out);
int imh_graph_launch(imh_graph *graph, imh_stream *stream);
void imh_graph_free(imh_graph *graph);

/* gpu_start_time / gpu_end_time (command.rs:470-489) as stream events. */
int imh_event_create(imh_device *dev, imh_event **out);
void imh_event_free(imh_event *ev);
int imh_event_record(imh_event *ev, imh_stream *stream);
int imh_event_elapsed_ms(imh_event *start, imh_event *end, float *ms);

/* ========================= op tier: INT4 affine weights ========================= */

/* AffineQuantizedWeight (ironmill-inference/src/metal/weights.rs:129-147) in
 * the separate-array upload layout of metal/weights.rs:1064-1103:
 *   data   [n][k/2] bytes, element k of a row in the low nibble when k is even
 *          (int4_pack.rs:20-34, quantized.rs:441-447);
 *   scales [n][k/group_size] f16; zeros [n][k/group_size] f16 raw zero-points
 *          (dequant: w = (q - z) * s, core/dequant.rs:130-140);
 *   awq_scales [k] f16 or NULL: the activation is divided by it
 *          (affine_batched.metal:70-79).
 * group_size must be 128 and k a multiple of 128 (IMH_EUNSUPPORTED otherwise). */
typedef struct {
    const uint8_t *data;
    const uint16_t *scales;
    const uint16_t *zeros;
    const uint16_t *awq_scales;
    uint32_t n;
    uint32_t k;
    uint32_t group_size;
} imh_affine_int4_weight;

/* encode_projection -> encode_affine_projection (projection.rs:35-56,227-312),
 * with the dequantize-then-compute semantics of core/dequant.rs:85-180:
 *   y[t][r] = f16( sum_k (x[t][k] / awq[k]) * (q[r][k] - z) * s ),  f32 accumulate.
 * x: [token_count][k] f16, y: [token_count][n] f16. */
int imh_encode_affine_projection_int4(imh_stream *stream, const uint16_t *x,
                                      uint32_t token_count, const imh_affine_int4_weight *w,
                                      uint16_t *y);

/* encode_batched_affine_matvec_int4 (ops/quantized.rs:198-232): gate and up in
 * one launch; gate's awq_scales divide the activation for both
 * (ops/quantized.rs:218-224).  gate->n must equal up->n. */
int imh_encode_batched_affine_matvec_int4(imh_stream *stream, const uint16_t *x,
                                          uint32_t token_count,
                                          const imh_affine_int4_weight *gate, uint16_t *gate_out,
                                          const imh_affine_int4_weight *up, uint16_t *up_out);

/* encode_fused_ffn_gate_up_act_int4 (ops/quantized.rs:238-270,
 * affine_fused.metal:89-107): out = f16(act(gate) * up) with gate, up in f32;
 * act = SiLU g/(1+e^-g), or tanh-GELU with the inner term clamped to +-10. */
int imh_encode_fused_ffn_gate_up_act_int4(imh_stream *stream, const uint16_t *x,
                                          uint32_t token_count,
                                          const imh_affine_int4_weight *gate,
                                          const imh_affine_int4_weight *up, uint16_t *out,
                                          int use_gelu);

/* encode_ffn_block (metal/ffn.rs:13-144) for INT4 gate/up/down: act_out =
 * f16(act(x.Wg) * (x.Wu)) as imh_encode_fused_ffn_gate_up_act_int4 writes it
 * (act_out [token_count][gate->n]), then y = act_out . Wd^T with down's
 * awq_scales (y [token_count][down->n]), with the two ops' results (matvec
 * below 32 tokens, GEMM from 32; at 1-2 tokens the gate/up launch also hands
 * the down launch its operand image through the stream's scratch).  down->k
 * must equal gate->n. */
int imh_encode_ffn_block_int4(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                              const imh_affine_int4_weight *gate, const imh_affine_int4_weight *up,
                              const imh_affine_int4_weight *down, uint16_t *act_out, uint16_t *y,
                              int use_gelu);

/* Prefill GEMM at a chosen matrix-core precision (superblock_matmul_int4,
 * affine_matmul.metal:10-152, at the precisions of the prefill workload):
 *   y[m][n] = sum_k a[m][k] * (q[n][k] - z) * s,  f32 accumulate, a = x / awq.
 * IMH_GEMM_F16: x and y f16 -- the projection op above (matvec below 32
 *   tokens, the f16 GEMM from 32);
 * IMH_GEMM_BF16: x and y bf16, a rounded once to bf16, bf16 matrix cores;
 * IMH_GEMM_FP8_E4M3: x and y bf16, a rounded once to OCP e4m3 (saturating at
 *   +-448), fp8 matrix cores.
 * The weights are not rounded at any precision (exact codes, zero-point and
 * scale applied in f32).  x [M][K], y [M][N]; M <= 65535. */
#define IMH_GEMM_F16 0
#define IMH_GEMM_BF16 1
#define IMH_GEMM_FP8_E4M3 2
int imh_affine_gemm_int4(imh_stream *stream, const void *x, uint32_t M, const imh_affine_int4_weight *w,
                         void *y, int precision);

/* INT8 "sensitive-layer" weight (quantize_tensor_int8, quantized.rs:852-901;
 * uploaded like the INT4 weight, metal/weights.rs:1036-1114): data [n][k] code
 * bytes 0..255, scales / zeros [n][k/128] f16 (raw zero-points), awq [k] f16
 * or NULL.  group_size must be 128. */
typedef struct {
    const uint8_t *data;
    const uint16_t *scales;
    const uint16_t *zeros;
    const uint16_t *awq_scales;
    uint32_t n;
    uint32_t k;
    uint32_t group_size;
} imh_affine_int8_weight;

/* superblock_matvec_int8 (affine_matvec.metal:123-189) for token_count rows:
 * y[t][r] = f16( sum_k (x[t][k] / awq[k]) * (q[r][k] - z) * s ), f32 accumulate.
 * x [token_count][k] f16, y [token_count][n] f16. */
int imh_encode_affine_projection_int8(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                      const imh_affine_int8_weight *w, uint16_t *y);

/* quantize_input_q8 (quantize.metal:21-52), per 128-element group of each row:
 * scale = absmax / 127, q = clamp(rint(x * (127 / absmax)), -127, 127) (0 for
 * an all-zero group).  x [token_count][k] f16 -> q8 [token_count][k] int8,
 * q8_scales [token_count][k/128] f32.  (The reference reduces the absmax per
 * 32-lane simdgroup while storing one scale per group; this is the per-group
 * rule it states.) */
int imh_encode_quantize_input_q8(imh_stream *stream, const uint16_t *x, uint32_t token_count, uint32_t k,
                                 int8_t *q8, float *q8_scales);

/* superblock_affine_matvec_int4xq8 (affine_fused.metal:115-176), the decode
 * variant on Q8 activations (pipeline.rs:639-664, projection.rs:123-143):
 * y[t][r] = f16( sum_g ws * as[t][g] * sum_{k in g} q8[t][k] * (q[r][k] - rint(z)) ),
 * on the integer matrix cores (each group's sum exact in int32).  The Q8
 * group is the weight group (128); w->awq_scales must be NULL (the reference
 * takes this path only without AWQ). */
int imh_encode_affine_matvec_int4xq8(imh_stream *stream, const int8_t *q8, const float *q8_scales,
                                     uint32_t token_count, const imh_affine_int4_weight *w, uint16_t *y);

/* The decode projection on Q8 activations from the f16 row (pipeline.rs:639-664
 * then projection.rs:123-143: encode_quantize_input_q8 followed by
 * encode_affine_matvec_int4xq8) in one launch at 1-8 rows: each workgroup
 * quantizes the row groups it stages with quantize_input_q8's arithmetic, so y
 * equals imh_encode_quantize_input_q8 + imh_encode_affine_matvec_int4xq8 bit for
 * bit.  q8_out [token_count][k] / q8_scales_out [token_count][k/128] (both or
 * neither; 16-byte aligned) receive the codes and scales for reuse by the
 * layer's other projections, as the reference reuses them.  Above 8 rows, or
 * for shapes outside the one-launch kernel, the two launches run (codes in
 * q8_out, or in the stream's scratch memory).  w->awq_scales must be NULL. */
int imh_encode_affine_projection_int4_q8(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                         const imh_affine_int4_weight *w, uint16_t *y, int8_t *q8_out,
                                         float *q8_scales_out);

/* FusedResidualNormAffineInt4Params (ops/fused.rs:45-66) with a token count. */
typedef struct {
    const uint16_t *a;           /* [token_count][k] */
    const uint16_t *b;           /* [token_count][k] */
    const uint16_t *norm_weight; /* [k] */
    uint16_t *residual_output;   /* [token_count][k]: f16(a + b) */
    const imh_affine_int4_weight *weight;
    uint16_t *output;            /* [token_count][n] */
    uint16_t *normed_output;     /* [token_count][k]: f16((a+b) * rms_inv * gamma) */
    uint32_t token_count;
    float eps;
} imh_fused_residual_norm_params;

/* encode_fused_residual_norm_affine_matvec_int4 (ops/fused.rs:102-129,
 * superblock_fused_norm.metal:37-124): r = a + b, rms_inv = 1/sqrt(mean(r^2)+eps),
 * output = f16(rms_inv * sum_k r_k*gamma_k(/awq_k) * W[n][k]). */
int imh_encode_fused_residual_norm_affine_matvec_int4(imh_stream *stream,
                                                      const imh_fused_residual_norm_params *p);

/* ====================== op tier: TurboQuant INT8 KV cache ====================== */

/* MetalTurboQuantModel (metal/turboquant/mod.rs:51-79,221-287): rotation signs
 * (seed), K codebook of 2^(n_bits-1) Lloyd-Max levels + boundaries, V codebook of
 * 2^n_bits levels + boundaries, QJL matrix [head_dim][head_dim] (seed + 1).
 * head_dim must be a power of two (IMH_EINVAL otherwise, mod.rs:222-226); the
 * kernels are built for head_dim 128 and n_bits 8 (IMH_EUNSUPPORTED otherwise). */
int imh_tq_tables_create(imh_device *dev, uint32_t head_dim, uint32_t n_bits,
                         uint64_t rotation_seed, imh_tq_tables **out);
/* Same from caller-provided host tables (f32): signs[head_dim],
 * k_codebook[2^(n_bits-1)], k_bounds[2^(n_bits-1)-1], v_codebook[2^n_bits],
 * v_bounds[2^n_bits-1], qjl[head_dim*head_dim] row-major. */
int imh_tq_tables_create_from_host(imh_device *dev, uint32_t head_dim, uint32_t n_bits,
                                   const float *signs, const float *k_codebook,
                                   const float *k_bounds, const float *v_codebook,
                                   const float *v_bounds, const float *qjl,
                                   imh_tq_tables **out);
void imh_tq_tables_free(imh_tq_tables *t);
#define IMH_TQ_SIGNS 0
#define IMH_TQ_K_CODEBOOK 1
#define IMH_TQ_K_BOUNDS 2
#define IMH_TQ_V_CODEBOOK 3
#define IMH_TQ_V_BOUNDS 4
#define IMH_TQ_QJL 5
/* Copy one table back to the host; *count receives its length in floats. */
int imh_tq_tables_read(const imh_tq_tables *t, int which, float *dst, size_t capacity,
                       size_t *count);

/* One layer of MetalKvCache (metal/turboquant/cache.rs:45-96) for `batch`
 * sequences, TurboQuantCacheLayout (turboquant/cache_layout.rs:83-142) per sequence:
 *   k_codes, v_codes: [batch][num_kv_heads][max_seq_len][head_dim] bytes
 *     (K byte = 7-bit codebook index | QJL sign in bit 7; V byte = 8-bit index);
 *   k_scales, v_scales, k_r_norms: [batch][num_kv_heads][max_seq_len] f32. */
typedef struct {
    uint8_t *k_codes;
    uint8_t *v_codes;
    float *k_scales;
    float *v_scales;
    float *k_r_norms;
    uint32_t batch;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t max_seq_len;
} imh_tq_kv_cache;

/* Byte sizes of the five arrays above (cache_layout.rs:83-142). */
int imh_tq_cache_sizes(uint32_t batch, uint32_t num_kv_heads, uint32_t head_dim,
                       uint32_t max_seq_len, size_t *codes_bytes, size_t *scale_bytes);

/* turboquant_cache_write (turboquant.metal:52-170) as encoded at
 * attention.rs:344-391, for K (is_k = 1) or V (is_k = 0):
 * kv_proj [batch][token_count][num_kv_heads][head_dim] f16; token t of sequence b
 * goes to position ((positions ? positions[b] : base_pos) + t) % max_seq_len.
 * positions is a device int32 array [batch] or NULL. */
int imh_encode_turboquant_cache_write(imh_stream *stream, const imh_tq_tables *t,
                                      const imh_tq_kv_cache *cache, const uint16_t *kv_proj,
                                      uint32_t token_count, uint32_t base_pos,
                                      const int32_t *positions, int is_k);

/* Both writes of encode_kv_cache_and_attention (attention.rs:344-391) in one
 * launch: K from k_proj, V from v_proj, same layout and positions as above. */
int imh_encode_turboquant_cache_write_kv(imh_stream *stream, const imh_tq_tables *t,
                                         const imh_tq_kv_cache *cache, const uint16_t *k_proj,
                                         const uint16_t *v_proj, uint32_t token_count,
                                         uint32_t base_pos, const int32_t *positions);

/* Decode attention over the cache (turboquant_attention, turboquant.metal:202-462,
 * + the split/LSE combine of fused_sdpa_reduce, flash_decode.metal:163-215):
 * q [batch][num_heads][head_dim] f16, GQA head h reads kv head h/(num_heads/num_kv_heads),
 * sequence b attends to positions [0, seq_lens ? min(seq_lens[b], bound) : seq_len)
 * where, with seq_lens (a device int32 array [batch]), seq_len is the bound
 * (0 = max_seq_len) the KV splits span; out [batch][num_heads][head_dim] f16.
 * num_splits = 0 picks the KV split count from the shape; seq_len > max_seq_len
 * is IMH_ERANGE. */
int imh_encode_turboquant_attention(imh_stream *stream, const imh_tq_tables *t,
                                    const imh_tq_kv_cache *cache, const uint16_t *q,
                                    uint32_t num_heads, uint32_t seq_len,
                                    const int32_t *seq_lens, float attn_scale, uint16_t *out,
                                    uint32_t num_splits);

/* No counterpart in the reference: imh_encode_turboquant_attention for callers
 * that cannot allocate device memory (code under HIP graph capture on a stream
 * whose scratch has not grown yet, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results; the split partials live
 * in a fixed per-GPU device array (4 MiB -- batch x num_heads x splits x
 * 520 B) instead of the stream's scratch, so the call allocates nothing.  A
 * shape that needs more returns IMH_EINVAL (pass fewer num_splits or a
 * smaller batch).  Every call on one GPU shares that array: calls that
 * overlap on one GPU (two streams at once) race; calls in one stream are
 * ordered.  Each call writes every partial it reads, so nothing is cleared. */
int imh_encode_turboquant_attention_noalloc(imh_stream *stream, const imh_tq_tables *t,
                                            const imh_tq_kv_cache *cache, const uint16_t *q,
                                            uint32_t num_heads, uint32_t seq_len,
                                            const int32_t *seq_lens, float attn_scale, uint16_t *out,
                                            uint32_t num_splits);

/* Causal attention of token_count query tokens per sequence (the prefill form
 * of turboquant_attention, turboquant.metal:202-462 with token_idx = tgid.y,
 * seq_len = base + token_idx + 1): q and out [batch][token_count][num_heads]
 * [head_dim] f16; token t of sequence b attends to positions
 * [0, L_b - token_count + t + 1) with L_b as in imh_encode_turboquant_attention
 * (the length including the new tokens, whose K / V the cache already holds).
 * One workgroup serves 16 / GQA consecutive tokens x the GQA group's heads
 * (each KV chunk is read and decoded once for all of them), after a query
 * prep launch; num_splits as in imh_encode_turboquant_attention (0: automatic,
 * over the longest causal range), with a combine launch when there are
 * several.  Uses the stream's scratch (batch x token_count x num_heads KB of
 * query operands, plus the split partials).  batch x ceil(token_count x GQA /
 * 16) <= 65535. */
int imh_encode_turboquant_attention_tokens(imh_stream *stream, const imh_tq_tables *t,
                                           const imh_tq_kv_cache *cache, const uint16_t *q,
                                           uint32_t num_heads, uint32_t token_count, uint32_t seq_len,
                                           const int32_t *seq_lens, float attn_scale, uint16_t *out,
                                           uint32_t num_splits);

/* encode_kv_cache_and_attention (attention.rs:117-610), decode step (one token
 * per sequence): write K and V at position seq_pos and attend over
 * [0, seq_pos + 1), in one launch (the codes written equal
 * imh_encode_turboquant_cache_write_kv's bit for bit). */
int imh_encode_kv_cache_and_attention(imh_stream *stream, const imh_tq_tables *t,
                                      const imh_tq_kv_cache *cache, const uint16_t *k_proj,
                                      const uint16_t *v_proj, const uint16_t *q,
                                      uint32_t num_heads, uint32_t seq_pos, float attn_scale,
                                      uint16_t *out);

/* ========================= op tier: decode-step glue ========================= */

/* rms_norm (normalization.metal:19-57, encode_rms_norm): per row of
 * hidden_size, out = f16(x * rms_inv * w), rms_inv = 1/sqrt(mean(x^2) + eps),
 * f32 arithmetic.  input/output [token_count][hidden_size] f16, weight [hidden_size]. */
int imh_encode_rms_norm(imh_stream *stream, const uint16_t *input, const uint16_t *weight,
                        uint16_t *output, uint32_t hidden_size, uint32_t token_count, float eps);

/* fused_residual_rms_norm (fused_residual_norm.metal:33-75,
 * encode_fused_residual_rms_norm): x = f32(a) + f32(b); residual_output = f16(x);
 * normed_output = f16(x * rms_inv * w) with x unrounded. */
int imh_encode_fused_residual_rms_norm(imh_stream *stream, const uint16_t *a, const uint16_t *b,
                                       const uint16_t *weight, uint16_t *normed_output,
                                       uint16_t *residual_output, uint32_t hidden_size,
                                       uint32_t token_count, float eps);

/* residual_add (encode_residual_add, attention.rs:693-700): out = f16(f32(a) + f32(b))
 * over n elements. */
int imh_encode_residual_add(imh_stream *stream, const uint16_t *a, const uint16_t *b, uint16_t *out,
                            size_t n);

/* fused_embedding_norm (fused_embedding_norm.metal:29-73, pipeline.rs:476-489):
 * x = embedding[id] * embed_scale (0 for id >= vocab_size); raw_output = f16(x);
 * normed_output = f16(x * rms_inv * norm_weight).  token_ids is a device uint32
 * array [token_count]; embedding [vocab_size][hidden_size] f16. */
int imh_encode_fused_embedding_norm(imh_stream *stream, const uint32_t *token_ids,
                                    const uint16_t *embedding, const uint16_t *norm_weight,
                                    uint16_t *normed_output, uint16_t *raw_output,
                                    uint32_t hidden_size, uint32_t token_count, uint32_t vocab_size,
                                    float eps, float embed_scale);

/* precompute_rope_cache (ironmill-core/src/rope.rs:22-50), on the host: cos/sin
 * [max_pos][head_dim/2] f16, angle = pos / theta^(2i/rotary_dim) in f64, rounded
 * once to f16; entries i >= rotary_dim/2 are (1, 0).  rotary_dim 0 = head_dim. */
int imh_rope_cache_fill(uint32_t head_dim, uint32_t max_pos, double theta, uint32_t rotary_dim,
                        uint16_t *cos_out, uint16_t *sin_out);

/* QK RMSNorm + RoPE in place (encode_qk_norm_and_rope, attention.rs:26-92).
 * With q_norm and k_norm: fused_qk_norm_rope (fused_qk_norm_rope.metal:43-124),
 * RMSNorm over each head then rotation of pairs (d, d + rotary_dim/2),
 * d < rotary_dim/2.  Without (both NULL): rope (rope.metal), pairs
 * (d, d + head_dim/2).  q [batch][token_count][num_heads][head_dim],
 * k [batch][token_count][num_kv_heads][head_dim] f16; token t of sequence b sits
 * at position (positions ? positions[b] : seq_offset) + t, clamped to the table
 * (positions: device int32 [batch] or NULL). */
typedef struct {
    uint16_t *q;
    uint16_t *k;
    const uint16_t *q_norm;    /* [head_dim] or NULL */
    const uint16_t *k_norm;    /* [head_dim] or NULL */
    const uint16_t *cos_cache; /* [max_pos][head_dim/2] */
    const uint16_t *sin_cache;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t rotary_dim;       /* 0 = head_dim */
    uint32_t max_pos;
    uint32_t seq_offset;
    const int32_t *positions;
    uint32_t batch;
    uint32_t token_count;
    float eps;
} imh_qk_norm_rope_params;
int imh_encode_qk_norm_rope(imh_stream *stream, const imh_qk_norm_rope_params *p);

/* One layer of the FP16 KV cache (fp16_kv_cache.layer_caches, attention.rs:492-496)
 * for `batch` sequences: k, v [batch][num_kv_heads][max_seq_len][head_dim] f16,
 * 16-byte aligned.  The kernels are built for head_dim 128 (IMH_EUNSUPPORTED
 * otherwise). */
typedef struct {
    uint16_t *k;
    uint16_t *v;
    uint32_t batch;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t max_seq_len;
} imh_fp16_kv_cache;

/* Cache positions of one step of token_count tokens from seq_pos on, for a
 * layer with the given sliding window (0 = full attention): the arithmetic of
 * KvCacheAndAttentionParams (attention.rs:141-163) and the cache's ring_pos /
 * effective_max_seq_len (turboquant/cache.rs:382-400):
 *   stride    = window_size ? window_size : max_seq_len  (the layer cache's max_seq_len)
 *   write_pos = window_size ? seq_pos % window_size : seq_pos  (base_pos of the cache writes)
 *   attn_base = window_size ? min(min(seq_pos + T, W) - T, W - T), saturating at 0 : seq_pos
 *   attn_len  = attn_base + token_count  (seq_len of the attention ops; token t
 *               attends to slots [0, attn_base + t + 1))
 * IMH_ERANGE when seq_pos + token_count exceeds max_seq_len (the step guard of
 * pipeline.rs:270-279), IMH_EINVAL for token_count 0 or above the stride. */
typedef struct {
    uint32_t stride;
    uint32_t write_pos;
    uint32_t attn_base;
    uint32_t attn_len;
} imh_kv_positions;
int imh_kv_positions_for(uint32_t seq_pos, uint32_t token_count, uint32_t window_size, uint32_t max_seq_len,
                         imh_kv_positions *out);

/* encode_kv_scatter (ops/kv.rs:35-58, kv_scatter.metal:20-45) for the K
 * (is_k = 1) or V (is_k = 0) array: proj [batch][token_count][num_kv_heads][head_dim]
 * f16; token t of sequence b goes to position
 * ((positions ? positions[b] : base_pos) + t) % max_seq_len (the ring-buffer
 * wrap of kv_scatter.metal:36-39).  positions is a device int32 array [batch]
 * or NULL. */
int imh_encode_kv_scatter(imh_stream *stream, const imh_fp16_kv_cache *cache, const uint16_t *proj,
                          uint32_t token_count, uint32_t base_pos, const int32_t *positions,
                          int is_k);

/* FP16-KV attention: fused_sdpa (fused_sdpa.metal:52-251, encode_fused_sdpa,
 * attention_ops.rs:274-306) and its FlashDecoding split + reduce
 * (flash_decode.metal:25-215, encode_flash_decode, attention_ops.rs:346-417).
 * q [batch][token_count][num_heads][head_dim] f16; GQA head h reads kv head
 * h/(num_heads/num_kv_heads); token t of sequence b attends to positions
 * [0, L_b - token_count + t + 1) with L_b = seq_lens ? min(seq_lens[b], bound) :
 * seq_len (the causal limit of fused_sdpa.metal:166-173), the bound being
 * seq_len, 0 = max_seq_len, when seq_lens is given; out has q's layout.  A row
 * with no position gives 0.  num_splits = 0 picks the KV split count from the
 * shape.  seq_len > max_seq_len is IMH_ERANGE; token_count > seq_len (without
 * seq_lens) is IMH_EINVAL.  The kernel is built for decode (token_count 1);
 * larger token counts are computed correctly, without prefill tiling. */
int imh_encode_fp16_attention(imh_stream *stream, const imh_fp16_kv_cache *cache, const uint16_t *q,
                              uint32_t num_heads, uint32_t token_count, uint32_t seq_len,
                              const int32_t *seq_lens, float attn_scale, uint16_t *out,
                              uint32_t num_splits);

/* The FP16 branch of encode_kv_cache_and_attention (attention.rs:491-607):
 * scatter K and V at seq_pos, then attend over [0, seq_pos + token_count)
 * causally. */
int imh_encode_fp16_kv_cache_and_attention(imh_stream *stream, const imh_fp16_kv_cache *cache,
                                           const uint16_t *k_proj, const uint16_t *v_proj,
                                           const uint16_t *q, uint32_t num_heads,
                                           uint32_t token_count, uint32_t seq_pos,
                                           float attn_scale, uint16_t *out);

/* ===================== decode step (InferenceEngine::decode_step) ===================== */

/* One decode step of a standard pre-norm transformer (MetalInference::decode_step,
 * metal/engine.rs:178-180 -> run_pipeline_inner, metal/pipeline.rs:228-1313) with
 * INT4-affine projections (LM head included), QK RMSNorm + RoPE, and a TurboQuant
 * INT8 or FP16 KV cache, for `batch` sequences of one token each.  The decoder
 * owns the activations, the RoPE tables (rope_theta, rotary_dim; 0 = head_dim),
 * the KV caches of every layer and the per-sequence positions, all in device
 * memory; weights stay caller-owned.  A step reads token_ids (device uint32
 * [batch]), writes logits (device f16 [batch][vocab_size]) and advances every
 * position by one on the device, so a captured step replays as the next token.
 * A replay with a sequence already at max_seq_len writes no cache row and is
 * reported by imh_decoder_sync_positions.  attn_scale 0 = 1/sqrt(head_dim);
 * embed_scale 0 = 1. */
#define IMH_KV_TURBOQUANT 0
#define IMH_KV_FP16 1
typedef struct imh_decoder imh_decoder;
typedef struct {
    uint32_t hidden_size;
    uint32_t intermediate_size;
    uint32_t num_layers;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t vocab_size;
    uint32_t max_seq_len;
    uint32_t batch;
    uint32_t rotary_dim;
    float rms_eps;
    float attn_scale;
    float embed_scale;
    int use_gelu;
    int kv_cache;       /* IMH_KV_TURBOQUANT or IMH_KV_FP16 */
    double rope_theta;
    uint64_t tq_seed;   /* TurboQuant rotation seed (QJL uses seed + 1) */
    /* per-layer sliding-window sizes, 0 = full attention, or NULL for none
     * (TurboQuantMetalConfig::window_sizes, turboquant/cache.rs:92-135): a
     * windowed layer's cache is a ring of window_size positions, written at
     * position % window_size, and attends over min(position + 1, window_size)
     * slots (attention.rs:141-163).  Copied at creation. */
    const uint32_t *window_sizes;
} imh_decoder_config;

/* The weights of one layer (LayerWeights of metal/weights.rs) as the schedule
 * reads them; q_norm/k_norm both NULL selects plain RoPE. */
typedef struct {
    const uint16_t *input_norm;      /* [hidden] */
    const uint16_t *post_attn_norm;  /* [hidden] */
    const uint16_t *q_norm;          /* [head_dim] or NULL */
    const uint16_t *k_norm;          /* [head_dim] or NULL */
    imh_affine_int4_weight q_proj;   /* [num_heads*head_dim][hidden] */
    imh_affine_int4_weight k_proj;   /* [num_kv_heads*head_dim][hidden] */
    imh_affine_int4_weight v_proj;
    imh_affine_int4_weight o_proj;   /* [hidden][num_heads*head_dim] */
    imh_affine_int4_weight gate_proj;/* [intermediate][hidden] */
    imh_affine_int4_weight up_proj;
    imh_affine_int4_weight down_proj;/* [hidden][intermediate] */
} imh_decoder_layer_weights;

int imh_decoder_create(imh_device *dev, const imh_decoder_config *cfg, imh_decoder **out);
void imh_decoder_free(imh_decoder *d);
int imh_decoder_set_layer(imh_decoder *d, uint32_t layer, const imh_decoder_layer_weights *w);
/* embedding [vocab][hidden] f16, final_norm [hidden], lm_head [vocab][hidden] INT4 */
int imh_decoder_set_model(imh_decoder *d, const uint16_t *embedding, const uint16_t *final_norm,
                          const imh_affine_int4_weight *lm_head);
/* Set every sequence's next write position (host int32 [batch], NULL = 0); synchronises. */
int imh_decoder_reset(imh_decoder *d, imh_stream *stream, const int32_t *positions);
/* Encode one step (pipeline.rs:424-1172 for token_count 1).  IMH_ERANGE when a
 * position has reached max_seq_len (cache.rs:494-504). */
int imh_decoder_step(imh_decoder *d, imh_stream *stream, const uint32_t *token_ids, uint16_t *logits);

/* Prefill of token_count tokens per sequence (run_pipeline_inner with
 * token_count > 1, metal/pipeline.rs:228-1313, as the chunked prefill of
 * metal/engine.rs:182-228 runs it): token_ids [batch][token_count]; token t of
 * sequence b goes to position positions[b] + t and attends causally to
 * [0, positions[b] + t + 1).  A sliding-window layer (token_count <=
 * window_size W) writes its ring at (p + t) % W and token t attends to slots
 * [0, min(p + T, W) - T + t + 1) (attention.rs:141-163): the last W positions
 * while p + T <= W; past that the reference's clamp, under which a chunk's
 * early tokens see slots its later tokens rewrote.  logits [batch][vocab] f16 of each
 * sequence's last token; the positions advance by token_count.  The
 * projections of batch x token_count >= 32 rows run on the GEMM ops.
 * Activation rows for batch x token_count tokens are allocated on the first
 * call of a size (IMH_EINVAL while capturing before that); token_count 1 is
 * imh_decoder_step.  IMH_ERANGE when a sequence would pass max_seq_len. */
int imh_decoder_prefill(imh_decoder *d, imh_stream *stream, const uint32_t *token_ids, uint32_t token_count,
                        uint16_t *logits);
/* Write token_count K/V projections ([batch][token_count][num_kv_heads][head_dim]
 * f16) of one layer into its cache at positions base_pos.. (the cache-write half
 * of encode_kv_cache_and_attention, attention.rs:344-391 / :497-525, as a
 * prefill would run it). */
int imh_decoder_write_kv(imh_decoder *d, imh_stream *stream, uint32_t layer, const uint16_t *k_proj,
                         const uint16_t *v_proj, uint32_t token_count, uint32_t base_pos);
/* Host mirror of the positions after the eager steps (host int32 [batch]).
 * Steps encoded during capture and graph replays do not move it; see
 * imh_decoder_sync_positions. */
int imh_decoder_positions(const imh_decoder *d, int32_t *out);
/* Synchronise the stream, read the device positions into the host mirror (and
 * into out, host int32 [batch], when not NULL).  IMH_ERANGE when a step ran
 * with a sequence already at max_seq_len -- a graph replayed past the cache
 * (pipeline.rs:271-279 refuses that step): such a step writes no cache row,
 * its logits are invalid, and the condition holds until imh_decoder_reset. */
int imh_decoder_sync_positions(imh_decoder *d, imh_stream *stream, int32_t *out);
/* The KV cache of one layer (a view; the decoder owns the memory). */
int imh_decoder_kv_cache(const imh_decoder *d, uint32_t layer, imh_tq_kv_cache *tq_out,
                         imh_fp16_kv_cache *fp16_out);
/* The TurboQuant tables the decoder uses (NULL for an FP16 cache). */
int imh_decoder_tq_tables(const imh_decoder *d, imh_tq_tables **out);
/* Use caller-built tables instead of the ones created from tq_seed -- the
 * counterpart of MetalTurboQuantModel::new (metal/turboquant/mod.rs:221-287)
 * handing its signs, codebooks and QJL matrix to the backend: build them with
 * imh_tq_tables_create_from_host from the reference's own generators
 * (turboquant/rotation.rs:13-49, codebook.rs:20-52) so the cache codes follow
 * the reference's tables exactly.  The tables stay caller-owned and must
 * outlive the decoder; set them before the first step (rows already in the
 * cache were written under the previous tables). */
int imh_decoder_set_tq_tables(imh_decoder *d, imh_tq_tables *t);

#ifdef __cplusplus
}
#endif
#endif /* IRONMILL_HIP_H */
