/*
 * oracle.c -- INT4 affine part of the CPU oracle (test infrastructure only;
 * see oracle.h).  Compiled with -ffp-contract=off: every a*b+c below is two
 * IEEE roundings, as in the reference's Rust code (rustc never contracts).
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* binary16 <-> binary32 (IEEE 754 round-to-nearest-even)              */
/* ------------------------------------------------------------------ */

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                 /* inf / nan */
        if (ax == 0x7F800000u) return sign | 0x7C00u;
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    if (ax >= 0x477FF000u) return sign | 0x7C00u;   /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                 /* result is a normal f16 */
        uint32_t mant = ax & 0x7FFFFFu;
        uint32_t e = (ax >> 23) - 127u + 15u;
        uint32_t h = (e << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return sign;       /* below 2^-25: rounds to zero */
    {                                         /* subnormal f16 */
        uint32_t e = ax >> 23;
        uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;           /* value in units of 2^-24 */
        uint32_t h = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {                              /* subnormal: m * 2^-24 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void orc_f32_to_f16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_f16(src[i]);
}

void orc_f16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(src[i]);
}

/* 64K-entry decode table used by the hot loops of the matvec oracle. */
static float g_f16_lut[65536];
static int g_f16_lut_ready = 0;

static void ensure_lut(void) {
    if (g_f16_lut_ready) return;
    for (uint32_t i = 0; i < 65536u; i++) g_f16_lut[i] = orc_f16_to_f32((uint16_t)i);
    g_f16_lut_ready = 1;
}

/* ------------------------------------------------------------------ */
/* quantize_affine  (affine_quantize.rs:256-298)                       */
/* ------------------------------------------------------------------ */

void orc_quantize_affine(const float *values, size_t n, float qmax, uint8_t *q_out,
                         float *scale_out, float *zp_out) {
    if (n == 0) {                             /* :257-259 */
        *scale_out = 1.0f;
        *zp_out = 0.0f;
        return;
    }
    float mn = INFINITY, mx = -INFINITY;      /* :261-273, finite values only */
    for (size_t i = 0; i < n; i++) {
        float v = values[i];
        if (isfinite(v)) {
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
    }
    if (!isfinite(mn) || !isfinite(mx)) {     /* :275-278 */
        memset(q_out, 0, n);
        *scale_out = 1.0f;
        *zp_out = 0.0f;
        return;
    }
    float scale, zp;
    if (fabsf(mx - mn) < FLT_EPSILON) {       /* :280-284 degenerate */
        scale = 1.0f;
        zp = roundf(-mn);
    } else {                                  /* :285-288 */
        scale = (mx - mn) / qmax;
        zp = roundf(-mn / scale);
    }
    for (size_t i = 0; i < n; i++) {          /* :291-297 */
        float t = roundf(values[i] / scale + zp);
        /* f32::clamp keeps NaN; `as u8` then maps NaN to 0 */
        if (isnan(t)) {
            q_out[i] = 0;
            continue;
        }
        if (t < 0.0f) t = 0.0f;
        if (t > qmax) t = qmax;
        q_out[i] = (uint8_t)t;
    }
    *scale_out = scale;
    *zp_out = zp;
}

/* ------------------------------------------------------------------ */
/* nibble packing  (int4_pack.rs:20-73)                                */
/* ------------------------------------------------------------------ */

void orc_pack_int4(const uint8_t *values, size_t n, uint8_t *out) {
    for (size_t i = 0, o = 0; i < n; i += 2, o++) {
        uint8_t lo = values[i] & 0x0F;
        uint8_t hi = (i + 1 < n) ? (values[i + 1] & 0x0F) : 0;
        out[o] = (uint8_t)((hi << 4) | lo);
    }
}

void orc_unpack_int4(const uint8_t *packed, size_t count, uint8_t *out) {
    for (size_t i = 0; i < count; i++) {
        uint8_t b = packed[i / 2];
        out[i] = (i % 2 == 0) ? (b & 0x0F) : ((b >> 4) & 0x0F);
    }
}

void orc_pack_int4_u32(const uint8_t *values, size_t n, uint32_t *out) {
    size_t words = (n + 7) / 8;
    for (size_t w = 0; w < words; w++) {
        uint32_t word = 0;
        for (size_t j = 0; j < 8 && w * 8 + j < n; j++)
            word |= (uint32_t)(values[w * 8 + j] & 0x0F) << (4 * j);
        out[w] = word;
    }
}

/* ------------------------------------------------------------------ */
/* quantize_tensor_int4  (ironmill-compile/src/weights/quantized.rs:408-465) */
/* ------------------------------------------------------------------ */

void orc_quantize_tensor_int4(const float *w, size_t rows, size_t k, size_t gs,
                              uint8_t *packed, float *scales, float *zeros) {
    size_t ngroups = (k + gs - 1) / gs;
    size_t total = rows * k;
    /* codes are produced row by row, group by group, then packed as one flat
     * stream (:441-447), so a row of odd length shares a byte with the next */
    uint8_t *codes = (uint8_t *)malloc(total ? total : 1);
    size_t pi = 0;
    for (size_t r = 0; r < rows; r++) {
        size_t row_start = r * k;
        for (size_t g = 0; g < ngroups; g++) {
            size_t g_start = row_start + g * gs;
            size_t g_end = g_start + gs;
            if (g_end > row_start + k) g_end = row_start + k;
            orc_quantize_affine(w + g_start, g_end - g_start, 15.0f, codes + g_start,
                                &scales[pi], &zeros[pi]);
            pi++;
        }
    }
    orc_pack_int4(codes, total, packed);
    free(codes);
}

static inline float read_q4(const uint8_t *packed, size_t i);

/* quantize_tensor_int8 (ironmill-compile/src/weights/quantized.rs:852-901):
 * the INT4 walk with qmax 255 and one code byte per element (no packing). */
void orc_quantize_tensor_int8(const float *w, size_t rows, size_t k, size_t gs,
                              uint8_t *codes, float *scales, float *zeros) {
    size_t ngroups = (k + gs - 1) / gs;
    size_t pi = 0;
    for (size_t r = 0; r < rows; r++) {
        size_t row_start = r * k;
        for (size_t g = 0; g < ngroups; g++) {
            size_t g_start = row_start + g * gs;
            size_t g_end = g_start + gs;
            if (g_end > row_start + k) g_end = row_start + k;
            orc_quantize_affine(w + g_start, g_end - g_start, 255.0f, codes + g_start,
                                &scales[pi], &zeros[pi]);
            pi++;
        }
    }
}

/* dequant_affine for 8-bit codes (ironmill-core/src/dequant.rs:122-142 with
 * bit_width 8: one byte per element): f16((q - z) * s), f32 arithmetic. */
void orc_dequant_affine_int8(const uint8_t *codes, const float *scales, const float *zeros,
                             size_t n, size_t k, size_t gs, uint16_t *w_out) {
    size_t ng = (k + gs - 1) / gs;
    for (size_t r = 0; r < n; r++)
        for (size_t c = 0; c < k; c++) {
            size_t pi = r * ng + c / gs;
            w_out[r * k + c] = orc_f32_to_f16(((float)codes[r * k + c] - zeros[pi]) * scales[pi]);
        }
}

/* quantize_input_q8 (quantize.metal:21-52) per group of gs elements of each
 * row: scale = absmax / 127, inv = absmax > 0 ? 127 / absmax : 0,
 * q = clamp(rint(x * inv), -127, 127), f32 arithmetic.  The group's absmax is
 * taken over the whole group (the kernel's stated rule; its simdgroup-scope
 * reduction is not reproduced). */
void orc_quantize_input_q8(const uint16_t *x, size_t rows, size_t k, size_t gs, int8_t *q8,
                           float *scales) {
    size_t ng = k / gs;
    for (size_t r = 0; r < rows; r++)
        for (size_t g = 0; g < ng; g++) {
            const uint16_t *xg = x + r * k + g * gs;
            float m = 0.0f;
            for (size_t i = 0; i < gs; i++) {
                float a = fabsf(orc_f16_to_f32(xg[i]));
                if (a > m) m = a;
            }
            scales[r * ng + g] = m / 127.0f;
            float inv = m > 0.0f ? 127.0f / m : 0.0f;
            for (size_t i = 0; i < gs; i++) {
                float v = rintf(orc_f16_to_f32(xg[i]) * inv);
                if (v < -127.0f) v = -127.0f;
                if (v > 127.0f) v = 127.0f;
                q8[r * k + g * gs + i] = (int8_t)v;
            }
        }
}

/* superblock_affine_matvec_int4xq8 (affine_fused.metal:115-176) with the Q8
 * group equal to the weight group: y = sum_g ws * as * sum q8 (q - rint(z)),
 * f64 accumulation (the reference's per-term f32 products differ from this
 * by f32 rounding only).  Scales and zero-points as uploaded (f16). */
void orc_matvec_int4xq8(const int8_t *q8, const float *q8_scales, const uint8_t *packed,
                        const uint16_t *scales, const uint16_t *zeros, size_t batch, size_t n,
                        size_t k, size_t gs, double *y) {
    size_t ng = k / gs;
    for (size_t b = 0; b < batch; b++)
        for (size_t r = 0; r < n; r++) {
            double acc = 0.0;
            for (size_t g = 0; g < ng; g++) {
                double ws = orc_f16_to_f32(scales[r * ng + g]);
                double iz = rintf(orc_f16_to_f32(zeros[r * ng + g]));
                long long s = 0;
                for (size_t i = 0; i < gs; i++) {
                    size_t c = g * gs + i;
                    long long q = (long long)read_q4(packed, r * k + c);
                    s += (long long)q8[b * k + c] * (q - (long long)iz);
                }
                acc += ws * (double)q8_scales[b * ng + g] * (double)s;
            }
            y[b * n + r] = acc;
        }
}

void orc_convert_params_to_f16(const float *params, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(params[i]);
}

/* ------------------------------------------------------------------ */
/* dequant_affine, group branch  (ironmill-core/src/dequant.rs:122-142) */
/* ------------------------------------------------------------------ */

static inline float read_q4(const uint8_t *packed, size_t i) {
    uint8_t b = packed[i / 2];
    return (float)((i % 2 == 0) ? (b & 0x0F) : ((b >> 4) & 0x0F));
}

void orc_dequant_affine_int4(const uint8_t *packed, const float *scales,
                             const float *zeros, size_t n, size_t k, size_t gs,
                             uint16_t *w_out) {
    size_t ng = (k + gs - 1) / gs;
    for (size_t r = 0; r < n; r++)
        for (size_t c = 0; c < k; c++) {
            size_t pi = r * ng + c / gs;
            float q = read_q4(packed, r * k + c);
            w_out[r * k + c] = orc_f32_to_f16((q - zeros[pi]) * scales[pi]);
        }
}

void orc_dequant_affine_int4_f16params(const uint8_t *packed, const uint16_t *scales,
                                       const uint16_t *zeros, size_t n, size_t k,
                                       size_t gs, uint16_t *w_out) {
    size_t ng = (k + gs - 1) / gs;
    for (size_t r = 0; r < n; r++)
        for (size_t c = 0; c < k; c++) {
            size_t pi = r * ng + c / gs;
            float q = read_q4(packed, r * k + c);
            float s = orc_f16_to_f32(scales[pi]);
            float z = orc_f16_to_f32(zeros[pi]);
            w_out[r * k + c] = orc_f32_to_f16((q - z) * s);
        }
}

/* ------------------------------------------------------------------ */
/* dequantize-then-compute matvec                                      */
/* ------------------------------------------------------------------ */

void orc_matvec_f16w(const uint16_t *w, const uint16_t *x, const uint16_t *awq,
                     size_t batch, size_t n_rows, size_t k, float *y, int nthreads) {
    ensure_lut();
    float *xe = (float *)malloc(sizeof(float) * ((batch * k) > 0 ? (batch * k) : 1));
    for (size_t b = 0; b < batch; b++)
        for (size_t c = 0; c < k; c++) {
            float v = g_f16_lut[x[b * k + c]];
            if (awq) v = v / g_f16_lut[awq[c]];
            xe[b * k + c] = v;
        }
    long nr = (long)n_rows;
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : 1;
#pragma omp parallel for num_threads(nt) schedule(static)
#endif
    for (long r = 0; r < nr; r++) {
        const uint16_t *wr = w + (size_t)r * k;
        for (size_t b = 0; b < batch; b++) {
            const float *xb = xe + b * k;
            float acc = 0.0f;
            for (size_t c = 0; c < k; c++) acc += xb[c] * g_f16_lut[wr[c]];
            y[b * n_rows + (size_t)r] = acc;
        }
    }
    (void)nthreads;
    free(xe);
}

float orc_silu(float g) { return g / (1.0f + expf(-g)); }

float orc_gelu_tanh(float g) {
    const float k = 0.7978845608f;
    float inner = k * (g + 0.044715f * g * g * g);
    if (inner < -10.0f) inner = -10.0f;
    if (inner > 10.0f) inner = 10.0f;
    return 0.5f * g * (1.0f + tanhf(inner));
}

void orc_fused_residual_norm_matvec(const uint16_t *a, const uint16_t *b,
                                    const uint16_t *gamma, const uint16_t *awq,
                                    float eps, const uint16_t *w, size_t batch,
                                    size_t n_rows, size_t k, float *y,
                                    uint16_t *residual_out, uint16_t *normed_out) {
    ensure_lut();
    float *r = (float *)malloc(sizeof(float) * (k ? k : 1));
    float *xe = (float *)malloc(sizeof(float) * (k ? k : 1));
    for (size_t m = 0; m < batch; m++) {
        const uint16_t *am = a + m * k, *bm = b + m * k;
        float sq = 0.0f;
        for (size_t c = 0; c < k; c++) {
            r[c] = g_f16_lut[am[c]] + g_f16_lut[bm[c]];
            sq += r[c] * r[c];
        }
        float rms_inv = 1.0f / sqrtf(sq / (float)k + eps);
        for (size_t c = 0; c < k; c++) {
            float v = r[c] * g_f16_lut[gamma[c]];
            if (awq) v = v / g_f16_lut[awq[c]];
            xe[c] = v;
            residual_out[m * k + c] = orc_f32_to_f16(r[c]);
            normed_out[m * k + c] = orc_f32_to_f16(r[c] * rms_inv * g_f16_lut[gamma[c]]);
        }
        for (size_t n = 0; n < n_rows; n++) {
            const uint16_t *wr = w + n * k;
            float acc = 0.0f;
            for (size_t c = 0; c < k; c++) acc += xe[c] * g_f16_lut[wr[c]];
            y[m * n_rows + n] = acc * rms_inv;
        }
    }
    free(r);
    free(xe);
}
