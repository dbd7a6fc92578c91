/*
 * oracle.h -- CPU restatement of ironmill's quantized-decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library (ironmill_amd/)
 * links, loads or calls this code.  It is used by tests/, by the smoke check
 * in __graft_entry__.py and by the cpu_baseline leg of bench.py, always as
 * the checker, never as the thing measured for the GPU numbers.
 *
 * Every function cites the reference file:line it restates (paths are under
 * jafreck/ironmill's crates/).  Pinning status of each function (what
 * independent check pins it) is listed beside it; "parity unpinned" marks
 * the functions for which no reference vector or closed form exists.
 *
 * Conventions: f16 values travel as uint16_t bit patterns (IEEE binary16),
 * all f32 arithmetic is compiled with -ffp-contract=off so that a*b+c is two
 * roundings unless fmaf() is written explicitly.
 */
#ifndef IRONMILL_ORACLE_H
#define IRONMILL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- binary16 conversion (half 2.7.1 f16::from_f32 / to_f32: IEEE RNE) ----
 * Used by ironmill-core/src/dequant.rs:138,326.  Pinned against numpy's
 * float16 conversion over every f16 pattern and a large random f32 sample. */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_array(const float *src, uint16_t *dst, size_t n);
void orc_f16_to_f32_array(const uint16_t *src, float *dst, size_t n);

/* ---- INT4 affine quantization (mil-rs/src/ir/passes/affine_quantize.rs:256-298)
 * Pinned by the reference's known-answer tests (affine_quantize.rs:552-629,
 * 723-762, 892-911) and brute-force checks on tiny groups. */
void orc_quantize_affine(const float *values, size_t n, float qmax,
                         uint8_t *q_out, float *scale_out, float *zp_out);

/* ---- nibble packing (mil-rs/src/ir/passes/int4_pack.rs:20-73) ----
 * Pinned by int4_pack.rs:109-170 known bytes/words. */
void orc_pack_int4(const uint8_t *values, size_t n, uint8_t *out);      /* out: ceil(n/2) */
void orc_unpack_int4(const uint8_t *packed, size_t count, uint8_t *out);
void orc_pack_int4_u32(const uint8_t *values, size_t n, uint32_t *out); /* out: ceil(n/8) */

/* ---- per-group INT4 tensor quantization
 * (ironmill-compile/src/weights/quantized.rs:408-465).  rows x k, groups of
 * gs along k (last group may be partial); packed = ceil(rows*k/2) bytes,
 * scales/zeros = rows*ceil(k/gs) f32.  Pinned through A1/A2 + the partial
 * last group case (affine_quantize.rs:765-796). */
void orc_quantize_tensor_int4(const float *w, size_t rows, size_t k, size_t gs,
                              uint8_t *packed, float *scales, float *zeros);

/* ---- f32 params -> f16 (ironmill-core/src/dequant.rs:305-345) ---- */
void orc_quantize_tensor_int8(const float *w, size_t rows, size_t k, size_t gs,
                              uint8_t *codes, float *scales, float *zeros);
void orc_dequant_affine_int8(const uint8_t *codes, const float *scales, const float *zeros,
                             size_t n, size_t k, size_t gs, uint16_t *w_out);
void orc_quantize_input_q8(const uint16_t *x, size_t rows, size_t k, size_t gs, int8_t *q8,
                           float *scales);
void orc_matvec_int4xq8(const int8_t *q8, const float *q8_scales, const uint8_t *packed,
                        const uint16_t *scales, const uint16_t *zeros, size_t batch, size_t n,
                        size_t k, size_t gs, double *y);
void orc_convert_params_to_f16(const float *params, size_t n, uint16_t *out);

/* ---- CPU dequant to dense f16 (ironmill-core/src/dequant.rs:85-180, group
 * branch :122-142): W[n,k] = f16((q - z) * s), s,z as f32.
 * Pinned by dequant.rs:404-463 vectors and the closed form. */
void orc_dequant_affine_int4(const uint8_t *packed, const float *scales,
                             const float *zeros, size_t n, size_t k, size_t gs,
                             uint16_t *w_out);
/* Same but the scale/zero arrays are the f16 GPU-upload copies
 * (metal/weights.rs:1064-1092); used to bound how far the fp16 params move y. */
void orc_dequant_affine_int4_f16params(const uint8_t *packed, const uint16_t *scales,
                                       const uint16_t *zeros, size_t n, size_t k,
                                       size_t gs, uint16_t *w_out);

/* ---- dequantize-then-compute matvec (the CPU reference path:
 * weight_loading.rs:554-599 -> dense f16 W, then the f32-accumulate dot of
 * ironmill-bench/tests/kernel_correctness.rs:42-48).  AWQ per D3 of the
 * reference divergence list: x_k / awq_k in f32 (affine_batched.metal:70-79).
 * y[b*n_rows + r] = sum_k xe[b,k] * W[r,k], f32 sequential accumulate.
 * nthreads > 1 splits rows over OpenMP threads (each row's order unchanged). */
void orc_matvec_f16w(const uint16_t *w, const uint16_t *x, const uint16_t *awq,
                     size_t batch, size_t n_rows, size_t k, float *y, int nthreads);

/* activation epilogues (affine_fused.metal:89-107, activation.metal:15-31) */
float orc_silu(float g);
float orc_gelu_tanh(float g);

/* fused residual + RMSNorm + INT4 projection
 * (norm/superblock_fused_norm.metal:37-124): r = a + b (f32);
 * rms_inv = 1/sqrt(sum r^2 / K + eps); y[n] = f16(rms_inv * sum_k r_k*g_k(/awq_k) * W[n,k]);
 * residual_out = f16(r); normed_out = f16(r * rms_inv * g).  Batched over rows
 * of a/b (the reference kernel is M=1; each row is independent). */
void orc_fused_residual_norm_matvec(const uint16_t *a, const uint16_t *b,
                                    const uint16_t *gamma, const uint16_t *awq,
                                    float eps, const uint16_t *w, size_t batch,
                                    size_t n_rows, size_t k, float *y,
                                    uint16_t *residual_out, uint16_t *normed_out);

/* ================= TurboQuant (INT8 KV cache) ================= */

/* Lloyd-Max codebook for N(0, 1/sqrt(dim)) (turboquant/codebook.rs:20-200,
 * incl. its Beasley-Springer-Moro quantile :114-184 and A&S erf :187-200).
 * levels: 2^bits, bounds: 2^bits - 1.  Pinned by Max (1960) centroids at
 * sigma=1 (dim=1) and the reference's invariants (codebook.rs:206-255). */
void orc_lloyd_max_gaussian(int dim, int bits, float *levels, float *bounds);
double orc_normal_quantile(double p);
double orc_erf(double x);

/* rand 0.10 StdRng restated: ChaCha12 (64-bit block counter in words 12-13,
 * stream words 14-15 zero) keyed by rand_core's PCG32 seed_from_u64
 * expansion.  Pinned: the block function at 8, 12 and 20 rounds and the
 * counter step (the all-zero-key vectors of draft-strombergson-chacha-test-
 * vectors and RFC 8439's block), the keyed stream's word order (a zero key
 * gives those blocks' words, low word first in each u64), and the PCG32
 * advance and XSH-RR output (the pcg32 demo sequence).  Unpinned: how
 * seed_from_u64 composes them (advance first, fixed increment; read from
 * rand_core's published source -- rand/chacha20 are not vendored in the
 * reference). */
void orc_chacha_block(const uint32_t in[16], int rounds, uint32_t out[16]);
typedef struct {
    uint32_t key[8];
    uint64_t counter;
    uint32_t buf[64];
    int idx;
} orc_stdrng;
uint64_t orc_pcg32_advance(uint64_t state, uint64_t inc);
uint32_t orc_pcg32_xsh_rr(uint64_t state);
void orc_stdrng_from_key(orc_stdrng *r, const uint32_t key[8]);
void orc_stdrng_seed_from_u64(orc_stdrng *r, uint64_t seed);
uint64_t orc_stdrng_next_u64(orc_stdrng *r);
/* n u64 draws of the stream keyed by key, or by seed_from_u64(seed) if key is NULL */
void orc_stdrng_stream(const uint32_t *key, uint64_t seed, int n, uint64_t *out);
/* turboquant/rotation.rs:13-25 (random_bool(0.5) per sign) and :31-49
 * (Box-Muller over random::<f64>()) -- parity unpinned, see above. */
void orc_rotation_signs(int dim, uint64_t seed, float *signs);
void orc_qjl_matrix(int dim, uint64_t seed, float *s);

/* randomized Hadamard R = D.H.D/sqrt(d) in place, butterfly order of
 * turboquant_helpers.metal:128-157.  Pinned by R.R = I and norm preservation. */
void orc_hadamard_rotate(float *x, const float *signs, int d);

/* Cache write (turboquant.metal:52-170) for one vector: fixed f32 order
 * (tree reductions over 128 lanes with halving stride, fmaf QJL projection
 * in increasing k).  Returns the code bytes, the L2 scale and (K only) the
 * residual norm.  Bit-exact target for the GPU write kernel. */
void orc_tq_quantize_vector(const uint16_t *x_f16, int d, int is_k,
                            const float *signs, const float *codebook,
                            const float *bounds, int n_levels,
                            const float *qjl, uint8_t *codes, float *scale,
                            float *r_norm);

/* Batched cache write over [batch][tokens][nkv][d] inputs into caches laid
 * out [batch][nkv][max_seq][d] (codes) and [batch][nkv][max_seq] (f32);
 * position = (positions ? positions[b] : base_pos) + t, modulo max_seq. */
void orc_tq_cache_write(const uint16_t *kv, int batch, int tokens, int nkv, int d,
                        int max_seq, int base_pos, const int32_t *positions,
                        int is_k, const float *signs, const float *codebook,
                        const float *bounds, int n_levels, const float *qjl,
                        uint8_t *cache, float *scales, float *r_norms);

/* Decode attention over the TQ cache (turboquant.metal:202-462 semantics,
 * dequantize-then-compute in f64): for each (b, h), kv = h / (nh/nkv),
 * q_rot = R q, s_q = S q_rot, score_p = attn_scale * ks_p * (q_rot . kcb[c&127]
 * + r_norm_p * sqrt(2/pi)/d * sum_d s_q[d]*sign(c)), softmax over
 * p < seq_len(b), o = R (sum_p w_p vs_p vcb[cv]).  out is f32 [batch][nh][d]. */
void orc_tq_attention(const uint16_t *q, int batch, int nh, int nkv, int d,
                      int max_seq, int seq_len, const int32_t *seq_lens,
                      float attn_scale, const float *signs, const float *k_codebook,
                      const float *v_codebook, const float *qjl,
                      const uint8_t *k_cache, const uint8_t *v_cache,
                      const float *k_scales, const float *v_scales,
                      const float *k_r_norms, float *out, int nthreads);

/* FP16-KV attention (metal/inference.rs:222-280 cpu_attention, the semantics
 * of fused_sdpa.metal:52-251 and flash_decode.metal:25-215) in f64: q
 * [batch][T][nh][d]; token t of sequence b attends to p < seq_len(b) - T + t + 1;
 * softmax(attn_scale * q . k) . v; caches [batch][nkv][max_seq][d] f16; out f32
 * [batch][T][nh][d].  Pinned by closed forms (one position -> its V; identical
 * keys -> mean of V; a dominant score selects its V; the causal rows of a
 * prefill equal decode steps at growing lengths) and equality with a float64
 * numpy softmax on small cases. */
void orc_fp16_attention(const uint16_t *q, int batch, int token_count, int nh, int nkv, int d,
                        int max_seq, int seq_len, const int32_t *seq_lens, float attn_scale,
                        const uint16_t *k_cache, const uint16_t *v_cache, float *out, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
