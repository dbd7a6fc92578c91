/*
 * oracle_tq.c -- TurboQuant (INT8 KV cache) part of the CPU oracle.
 * Test infrastructure only; see oracle.h.  Compiled with -ffp-contract=off.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* Lloyd-Max codebook  (turboquant/codebook.rs:20-200)                 */
/* The initial-level quantile and the erf approximation are kept with  */
/* the reference's coefficients: with at most 200 iterations the 7/8-bit */
/* tables have not fully converged, so the starting point shows in the */
/* final f32 values.                                                    */
/* ------------------------------------------------------------------ */

double orc_erf(double x) {                     /* codebook.rs:187-200 */
    const double a1 = 0.254829592, a2 = -0.284496736, a3 = 1.421413741;
    const double a4 = -1.453152027, a5 = 1.061405429, p = 0.3275911;
    double sign = x < 0.0 ? -1.0 : 1.0;
    double ax = fabs(x);
    double t = 1.0 / (1.0 + p * ax);
    double y = 1.0 - (((((a5 * t + a4) * t) + a3) * t + a2) * t + a1) * t * exp(-ax * ax);
    return sign * y;
}

static double normal_cdf(double x) { return 0.5 * (1.0 + orc_erf(x * 0.70710678118654752440)); }

static double normal_pdf(double x) {
    return exp(-0.5 * x * x) / sqrt(2.0 * 3.14159265358979323846);
}

double orc_normal_quantile(double p) {         /* codebook.rs:114-184 */
    if (p <= 0.0) return -INFINITY;
    if (p >= 1.0) return INFINITY;
    double t = p - 0.5;
    if (fabs(t) <= 0.42) {
        double r = t * t;
        double num = t * (((2.5066282746310002 * r + 18.6150006252966) * r + 41.39119773534996) * r +
                          25.44106049637689);
        double den = (((14.382029373388 * r + 63.690613) * r + 84.681) * r + 40.304) * r + 1.0;
        return num / den;
    }
    double r = t < 0.0 ? p : 1.0 - p;
    double s = sqrt(-log(r));
    double res;
    if (s <= 5.0) {
        double ss = s - 1.6;
        double num = ((((((0.000124818987 * ss + 0.0227061845) * ss + 0.2728688) * ss + 1.3058437) * ss +
                         2.7580128) * ss + 2.2311569) * ss + 0.6462025) * ss + 0.001612;
        double den = ((((((0.000038746 * ss + 0.00745102) * ss + 0.09234118) * ss + 0.4710441) * ss +
                         1.0507501) * ss + 1.0) * ss + 0.2127601) * ss + 1.0;
        res = num / den;
    } else {
        double ss = s - 5.0;
        res = (((((((0.0000000271 * ss + 0.00000342556) * ss + 0.000170717) * ss + 0.004531901) * ss +
                   0.06871337) * ss + 0.56419917) * ss + 1.9715909) * ss + 2.1538256) /
              (((((((0.0000000393 * ss + 0.00000489649) * ss + 0.000230147) * ss + 0.005492439) * ss +
                   0.06353648) * ss + 0.3445453) * ss + 0.73741429) * ss + 1.0);
    }
    return t < 0.0 ? -res : res;
}

static double cond_mean(double sigma, double lo, double hi) {   /* codebook.rs:86-104 */
    double lo_z = lo / sigma, hi_z = hi / sigma;
    double prob = normal_cdf(hi_z) - normal_cdf(lo_z);
    if (prob < 1e-30) {
        if (isinf(lo)) return hi;
        if (isinf(hi)) return lo;
        return (lo + hi) / 2.0;
    }
    return sigma * (normal_pdf(lo_z) - normal_pdf(hi_z)) / prob;
}

void orc_lloyd_max_gaussian(int dim, int bits, float *levels_out, float *bounds_out) {
    int n = 1 << bits;
    double sigma = 1.0 / sqrt((double)dim);
    double *lv = (double *)malloc(sizeof(double) * n);
    double *nl = (double *)malloc(sizeof(double) * n);
    double *bd = (double *)malloc(sizeof(double) * (n > 1 ? n - 1 : 1));
    for (int i = 0; i < n; i++) lv[i] = sigma * orc_normal_quantile(((double)i + 0.5) / (double)n);
    for (int it = 0; it < 200; it++) {
        for (int i = 0; i + 1 < n; i++) bd[i] = (lv[i] + lv[i + 1]) / 2.0;
        double max_delta = 0.0;
        for (int i = 0; i < n; i++) {
            double lo = (i == 0) ? -INFINITY : bd[i - 1];
            double hi = (i == n - 1) ? INFINITY : bd[i];
            nl[i] = cond_mean(sigma, lo, hi);
        }
        for (int i = 0; i < n; i++) {
            double d = fabs(lv[i] - nl[i]);
            if (d > max_delta) max_delta = d;
            lv[i] = nl[i];
        }
        if (max_delta < 1e-10) break;
    }
    for (int i = 0; i + 1 < n; i++) bd[i] = (lv[i] + lv[i + 1]) / 2.0;
    for (int i = 0; i < n; i++) levels_out[i] = (float)lv[i];
    for (int i = 0; i + 1 < n; i++) bounds_out[i] = (float)bd[i];
    free(lv);
    free(nl);
    free(bd);
}

/* ------------------------------------------------------------------ */
/* ChaCha12 StdRng (rand 0.10 / chacha20 0.10, restated from the       */
/* published ChaCha definition and rand_core's seed_from_u64)          */
/* ------------------------------------------------------------------ */

static inline uint32_t rotl32(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }

#define QR(a, b, c, d)                 \
    a += b; d ^= a; d = rotl32(d, 16); \
    c += d; b ^= c; b = rotl32(b, 12); \
    a += b; d ^= a; d = rotl32(d, 8);  \
    c += d; b ^= c; b = rotl32(b, 7);

void orc_chacha_block(const uint32_t in[16], int rounds, uint32_t out[16]) {
    uint32_t x[16];
    memcpy(x, in, sizeof(x));
    for (int i = 0; i < rounds; i += 2) {
        QR(x[0], x[4], x[8], x[12]);
        QR(x[1], x[5], x[9], x[13]);
        QR(x[2], x[6], x[10], x[14]);
        QR(x[3], x[7], x[11], x[15]);
        QR(x[0], x[5], x[10], x[15]);
        QR(x[1], x[6], x[11], x[12]);
        QR(x[2], x[7], x[8], x[13]);
        QR(x[3], x[4], x[9], x[14]);
    }
    for (int i = 0; i < 16; i++) out[i] = x[i] + in[i];
}

/* PCG32 (O'Neill 2014): the LCG step and the XSH-RR output of a state */
uint64_t orc_pcg32_advance(uint64_t state, uint64_t inc) { return state * 6364136223846793005ULL + inc; }

uint32_t orc_pcg32_xsh_rr(uint64_t state) {
    uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
    uint32_t rot = (uint32_t)(state >> 59);
    return (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
}

void orc_stdrng_from_key(orc_stdrng *r, const uint32_t key[8]) {
    for (int i = 0; i < 8; i++) r->key[i] = key[i];
    r->counter = 0;
    r->idx = 64;
}

void orc_stdrng_seed_from_u64(orc_stdrng *r, uint64_t state) {
    /* rand_core SeedableRng::seed_from_u64: the state advances first (fixed
     * increment), then its XSH-RR output is the next seed word */
    uint32_t key[8];
    for (int i = 0; i < 8; i++) {
        state = orc_pcg32_advance(state, 11634580027462260723ULL);
        key[i] = orc_pcg32_xsh_rr(state);
    }
    orc_stdrng_from_key(r, key);
}

void orc_stdrng_stream(const uint32_t *key, uint64_t seed, int n, uint64_t *out) {
    orc_stdrng r;
    if (key)
        orc_stdrng_from_key(&r, key);
    else
        orc_stdrng_seed_from_u64(&r, seed);
    for (int i = 0; i < n; i++) out[i] = orc_stdrng_next_u64(&r);
}

static void stdrng_refill(orc_stdrng *r) {
    for (int blk = 0; blk < 4; blk++) {
        uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
        for (int i = 0; i < 8; i++) in[4 + i] = r->key[i];
        uint64_t c = r->counter + (uint64_t)blk;
        in[12] = (uint32_t)c;
        in[13] = (uint32_t)(c >> 32);
        in[14] = 0;
        in[15] = 0;
        orc_chacha_block(in, 12, r->buf + 16 * blk);
    }
    r->counter += 4;
    r->idx = 0;
}

uint64_t orc_stdrng_next_u64(orc_stdrng *r) {
    if (r->idx >= 63) stdrng_refill(r);   /* idx stays even: only u64 draws */
    uint64_t lo = r->buf[r->idx], hi = r->buf[r->idx + 1];
    r->idx += 2;
    return (hi << 32) | lo;
}

void orc_rotation_signs(int dim, uint64_t seed, float *signs) {   /* rotation.rs:13-25 */
    orc_stdrng r;
    orc_stdrng_seed_from_u64(&r, seed);
    for (int i = 0; i < dim; i++)
        signs[i] = (orc_stdrng_next_u64(&r) < (1ULL << 63)) ? 1.0f : -1.0f;
}

void orc_qjl_matrix(int dim, uint64_t seed, float *s) {           /* rotation.rs:31-49 */
    orc_stdrng r;
    orc_stdrng_seed_from_u64(&r, seed);
    size_t n = (size_t)dim * (size_t)dim, i = 0;
    const double two_pi = 2.0 * 3.14159265358979323846;
    while (i < n) {
        double u1 = (double)(orc_stdrng_next_u64(&r) >> 11) * (1.0 / 9007199254740992.0);
        double u2 = (double)(orc_stdrng_next_u64(&r) >> 11) * (1.0 / 9007199254740992.0);
        if (u1 < 1e-300) u1 = 1e-300;
        double rad = sqrt(-2.0 * log(u1));
        double th = two_pi * u2;
        s[i++] = (float)(rad * cos(th));
        if (i < n) s[i++] = (float)(rad * sin(th));
    }
}

/* ------------------------------------------------------------------ */
/* Hadamard rotation  (turboquant_helpers.metal:128-157)               */
/* ------------------------------------------------------------------ */

void orc_hadamard_rotate(float *x, const float *signs, int d) {
    for (int i = 0; i < d; i++) x[i] *= signs[i];
    for (int step = 1; step < d; step *= 2)
        for (int i = 0; i < d / 2; i++) {
            int j = (i / step) * (step * 2) + (i % step);
            float a = x[j], b = x[j + step];
            x[j] = a + b;
            x[j + step] = a - b;
        }
    float scale = 1.0f / sqrtf((float)d);
    for (int i = 0; i < d; i++) x[i] *= signs[i] * scale;
}

static void hadamard_rotate_f64(double *x, const float *signs, int d) {
    for (int i = 0; i < d; i++) x[i] *= signs[i];
    for (int step = 1; step < d; step *= 2)
        for (int i = 0; i < d / 2; i++) {
            int j = (i / step) * (step * 2) + (i % step);
            double a = x[j], b = x[j + step];
            x[j] = a + b;
            x[j + step] = a - b;
        }
    double scale = 1.0 / sqrt((double)d);
    for (int i = 0; i < d; i++) x[i] *= signs[i] * scale;
}

/* sum of v[0..d) by the halving-stride tree of turboquant.metal:101-110 */
static float tree_sum(float *v, int d) {
    for (int s = d / 2; s > 0; s >>= 1)
        for (int i = 0; i < s; i++) v[i] += v[i + s];
    return v[0];
}

/* ------------------------------------------------------------------ */
/* cache write  (turboquant.metal:52-170)                              */
/* ------------------------------------------------------------------ */

void orc_tq_quantize_vector(const uint16_t *x_f16, int d, int is_k, const float *signs,
                            const float *codebook, const float *bounds, int n_levels,
                            const float *qjl, uint8_t *codes, float *scale_out,
                            float *r_norm_out) {
    float x[1024], red[1024], res[1024];
    for (int i = 0; i < d; i++) x[i] = orc_f16_to_f32(x_f16[i]);
    orc_hadamard_rotate(x, signs, d);
    for (int i = 0; i < d; i++) red[i] = x[i] * x[i];
    float l2 = sqrtf(fmaxf(tree_sum(red, d), 1e-20f));
    *scale_out = l2;
    float inv = 1.0f / fmaxf(l2, 1e-10f);
    for (int i = 0; i < d; i++) {
        float u = x[i] * inv;
        int idx = 0;
        for (int b = 0; b < n_levels - 1; b++)
            if (u >= bounds[b]) idx = b + 1;
        codes[i] = (uint8_t)idx;
        res[i] = u - codebook[idx];
    }
    if (!is_k) {
        if (r_norm_out) *r_norm_out = 0.0f;
        return;
    }
    for (int i = 0; i < d; i++) red[i] = res[i] * res[i];
    float rn = sqrtf(fmaxf(tree_sum(red, d), 1e-20f));
    if (r_norm_out) *r_norm_out = rn;
    for (int i = 0; i < d; i++) {
        float acc = 0.0f;
        for (int k = 0; k < d; k++) acc = fmaf(qjl[(size_t)i * d + k], res[k], acc);
        if (acc >= 0.0f) codes[i] |= 0x80u;
    }
}

void orc_tq_cache_write(const uint16_t *kv, int batch, int tokens, int nkv, int d,
                        int max_seq, int base_pos, const int32_t *positions, int is_k,
                        const float *signs, const float *codebook, const float *bounds,
                        int n_levels, const float *qjl, uint8_t *cache, float *scales,
                        float *r_norms) {
    for (int b = 0; b < batch; b++)
        for (int t = 0; t < tokens; t++)
            for (int h = 0; h < nkv; h++) {
                int start = positions ? positions[b] : base_pos;
                int pos = (start + t) % max_seq;
                size_t slot = ((size_t)b * nkv + h) * (size_t)max_seq + (size_t)pos;
                const uint16_t *src = kv + (((size_t)b * tokens + t) * nkv + h) * (size_t)d;
                float rn = 0.0f;
                orc_tq_quantize_vector(src, d, is_k, signs, codebook, bounds, n_levels, qjl,
                                       cache + slot * (size_t)d, &scales[slot], &rn);
                if (is_k && r_norms) r_norms[slot] = rn;
            }
}

/* ------------------------------------------------------------------ */
/* decode attention, dequantize-then-compute in f64                    */
/* (turboquant.metal:202-462; fused_sdpa_reduce flash_decode.metal:163-215 */
/* is exactness-neutral: the split/LSE combine equals one softmax)      */
/* ------------------------------------------------------------------ */

void orc_tq_attention(const uint16_t *q, int batch, int nh, int nkv, int d, int max_seq,
                      int seq_len, const int32_t *seq_lens, float attn_scale,
                      const float *signs, const float *k_codebook, const float *v_codebook,
                      const float *qjl, const uint8_t *k_cache, const uint8_t *v_cache,
                      const float *k_scales, const float *v_scales, const float *k_r_norms,
                      float *out, int nthreads) {
    int group = nh / nkv;
    float qjl_factor_f = sqrtf(2.0f / 3.14159265f) / (float)d;   /* turboquant.metal:305 */
    double qjl_factor = (double)qjl_factor_f;
    long total = (long)batch * nh;
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : 1;
#pragma omp parallel for num_threads(nt) schedule(dynamic)
#endif
    for (long bh = 0; bh < total; bh++) {
        int b = (int)(bh / nh), h = (int)(bh % nh);
        int kvh = h / group;
        int L = seq_lens ? seq_lens[b] : seq_len;
        double qr[1024], sq[1024], o[1024];
        for (int i = 0; i < d; i++) qr[i] = orc_f16_to_f32(q[((size_t)b * nh + h) * d + i]);
        hadamard_rotate_f64(qr, signs, d);
        for (int i = 0; i < d; i++) {
            double acc = 0.0;
            for (int k = 0; k < d; k++) acc += (double)qjl[(size_t)i * d + k] * qr[k];
            sq[i] = acc;
        }
        for (int i = 0; i < d; i++) o[i] = 0.0;
        size_t base = ((size_t)b * nkv + kvh) * (size_t)max_seq;
        double *sc = (double *)malloc(sizeof(double) * (L > 0 ? L : 1));
        double mx = -INFINITY;
        for (int p = 0; p < L; p++) {
            const uint8_t *kc = k_cache + (base + p) * (size_t)d;
            double ks = k_scales[base + p];
            double w = k_r_norms[base + p] * qjl_factor * ks;
            double t1 = 0.0, t2 = 0.0;
            for (int i = 0; i < d; i++) {
                t1 += qr[i] * (double)k_codebook[kc[i] & 0x7F] * ks;
                t2 += sq[i] * ((kc[i] & 0x80) ? 1.0 : -1.0);
            }
            sc[p] = (double)attn_scale * (t1 + t2 * w);
            if (sc[p] > mx) mx = sc[p];
        }
        double den = 0.0;
        for (int p = 0; p < L; p++) {
            double wgt = exp(sc[p] - mx);
            den += wgt;
            const uint8_t *vc = v_cache + (base + p) * (size_t)d;
            double vs = v_scales[base + p];
            for (int i = 0; i < d; i++) o[i] += wgt * (double)v_codebook[vc[i]] * vs;
        }
        free(sc);
        if (den < 1e-10) den = 1e-10;
        for (int i = 0; i < d; i++) o[i] /= den;
        hadamard_rotate_f64(o, signs, d);
        for (int i = 0; i < d; i++) out[((size_t)b * nh + h) * d + i] = (float)o[i];
    }
    (void)nthreads;
}

/* FP16-KV attention (metal/inference.rs:222-280 cpu_attention, the semantics
 * of fused_sdpa.metal:52-251 / flash_decode.metal:25-215), in f64.  q is
 * [batch][T][nh][d] for T = token_count query tokens per sequence; token t of
 * sequence b attends causally to p < seq_len(b) - T + t + 1 (inference.rs:241,
 * fused_sdpa.metal:166-173); kv head = h / (nh/nkv); score_p = attn_scale *
 * q . k_p; o = sum_p w_p v_p / sum_p w_p.  Caches are [batch][nkv][max_seq][d]
 * f16; out is f32 [batch][T][nh][d]; a row with no position gives 0. */
void orc_fp16_attention(const uint16_t *q, int batch, int token_count, int nh, int nkv, int d,
                        int max_seq, int seq_len, const int32_t *seq_lens, float attn_scale,
                        const uint16_t *k_cache, const uint16_t *v_cache, float *out, int nthreads) {
    int group = nh / nkv;
    int T = token_count;
    long total = (long)batch * T * nh;
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : 1;
#pragma omp parallel for num_threads(nt) schedule(dynamic)
#endif
    for (long row = 0; row < total; row++) {
        int b = (int)(row / ((long)T * nh));
        int t = (int)((row / nh) % T);
        int h = (int)(row % nh);
        int kvh = h / group;
        int L = seq_lens ? seq_lens[b] : seq_len;
        if (L > max_seq) L = max_seq;
        L = L - T + t + 1;
        if (L < 0) L = 0;
        double qv[1024], o[1024];
        for (int i = 0; i < d; i++) {
            qv[i] = orc_f16_to_f32(q[(size_t)row * d + i]);
            o[i] = 0.0;
        }
        size_t base = ((size_t)b * nkv + kvh) * (size_t)max_seq;
        double *sc = (double *)malloc(sizeof(double) * (L > 0 ? L : 1));
        double mx = -INFINITY;
        for (int p = 0; p < L; p++) {
            const uint16_t *kp = k_cache + (base + p) * (size_t)d;
            double acc = 0.0;
            for (int i = 0; i < d; i++) acc += qv[i] * (double)orc_f16_to_f32(kp[i]);
            sc[p] = (double)attn_scale * acc;
            if (sc[p] > mx) mx = sc[p];
        }
        double den = 0.0;
        for (int p = 0; p < L; p++) {
            double wgt = exp(sc[p] - mx);
            den += wgt;
            const uint16_t *vp = v_cache + (base + p) * (size_t)d;
            for (int i = 0; i < d; i++) o[i] += wgt * (double)orc_f16_to_f32(vp[i]);
        }
        free(sc);
        for (int i = 0; i < d; i++) out[(size_t)row * d + i] = L > 0 ? (float)(o[i] / den) : 0.0f;
    }
    (void)nthreads;
}
