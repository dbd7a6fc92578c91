/*
 * san_check.c -- drives every oracle entry point once on small, ragged inputs
 * whose buffers are allocated to their exact sizes, for the AddressSanitizer /
 * UndefinedBehaviorSanitizer build (`make -C oracle sanitize`).  Test
 * infrastructure only: any out-of-bounds access, leak or undefined operation
 * aborts the run; the few value checks below only catch a driver that no
 * longer exercises the code it names.  Exit status 0 = clean.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define CHECK(c)                                                    \
    do {                                                            \
        if (!(c)) {                                                 \
            fprintf(stderr, "san_check: %s:%d %s\n", __FILE__, __LINE__, #c); \
            exit(2);                                                \
        }                                                           \
    } while (0)

static uint64_t lcg = 0x9E3779B97F4A7C15ULL;
static float frand(void) {   /* uniform in [-1, 1) */
    lcg = lcg * 6364136223846793005ULL + 1442695040888963407ULL;
    return (float)((lcg >> 40) * (1.0 / 8388608.0)) - 1.0f;
}

static void *xmalloc(size_t n) {
    void *p = malloc(n ? n : 1);
    CHECK(p != NULL);
    return p;
}

static uint16_t *f16_vec(size_t n, float scale) {
    uint16_t *v = xmalloc(n * sizeof(uint16_t));
    for (size_t i = 0; i < n; i++) v[i] = orc_f32_to_f16(frand() * scale);
    return v;
}

static void check_f16_and_packing(void) {
    float src[5] = {0.0f, -1.5f, 65504.0f, 1e-8f, NAN};
    uint16_t h[5];
    float back[5];
    orc_f32_to_f16_array(src, h, 5);
    orc_f16_to_f32_array(h, back, 5);
    CHECK(back[1] == -1.5f && isnan(back[4]));
    uint8_t vals[7] = {3, 12, 0, 15, 7, 1, 9}, packed[4], un[7];
    uint32_t words[1];
    orc_pack_int4(vals, 7, packed);   /* odd count: the last byte is half filled */
    orc_unpack_int4(packed, 7, un);
    CHECK(memcmp(vals, un, 7) == 0 && packed[0] == 0xC3);
    orc_pack_int4_u32(vals, 7, words);
    float v[5] = {-3, 0, 3, 6, 12}, s, z;
    uint8_t q[5];
    orc_quantize_affine(v, 5, 15.0f, q, &s, &z);
    CHECK(q[0] == 0 && q[4] == 15);
}

static void check_int4_int8(void) {
    const size_t rows = 3, k = 200, gs = 128, ng = 2, batch = 2;   /* ragged k: partial last group */
    float *w = xmalloc(rows * k * sizeof(float));
    for (size_t i = 0; i < rows * k; i++) w[i] = frand() * 0.05f;
    uint8_t *packed = xmalloc((rows * k + 1) / 2);
    float *sc = xmalloc(rows * ng * sizeof(float)), *zp = xmalloc(rows * ng * sizeof(float));
    orc_quantize_tensor_int4(w, rows, k, gs, packed, sc, zp);
    uint16_t *sc16 = xmalloc(rows * ng * 2), *zp16 = xmalloc(rows * ng * 2);
    orc_convert_params_to_f16(sc, rows * ng, sc16);
    orc_convert_params_to_f16(zp, rows * ng, zp16);
    uint16_t *dense = xmalloc(rows * k * 2), *dense2 = xmalloc(rows * k * 2);
    orc_dequant_affine_int4(packed, sc, zp, rows, k, gs, dense);
    orc_dequant_affine_int4_f16params(packed, sc16, zp16, rows, k, gs, dense2);
    uint16_t *x = f16_vec(batch * k, 1.0f), *awq = xmalloc(k * 2), *gamma = xmalloc(k * 2);
    for (size_t i = 0; i < k; i++) {
        awq[i] = orc_f32_to_f16(0.5f + 0.75f * (frand() + 1.0f));
        gamma[i] = orc_f32_to_f16(1.0f + 0.2f * frand());
    }
    float *y = xmalloc(batch * rows * sizeof(float));
    orc_matvec_f16w(dense, x, awq, batch, rows, k, y, 2);
    orc_matvec_f16w(dense, x, NULL, batch, rows, k, y, 1);
    CHECK(isfinite(y[0]) && isfinite(y[batch * rows - 1]));
    uint16_t *b = f16_vec(batch * k, 0.3f), *res = xmalloc(batch * k * 2), *nrm = xmalloc(batch * k * 2);
    orc_fused_residual_norm_matvec(x, b, gamma, awq, 1e-6f, dense, batch, rows, k, y, res, nrm);
    CHECK(isfinite(orc_silu(-90.0f)) && isfinite(orc_gelu_tanh(30.0f)));

    uint8_t *codes8 = xmalloc(rows * k);
    orc_quantize_tensor_int8(w, rows, k, gs, codes8, sc, zp);
    orc_dequant_affine_int8(codes8, sc, zp, rows, k, gs, dense);

    const size_t kq = 256, gq = 2;   /* Q8 needs whole groups */
    uint16_t *xq = f16_vec(batch * kq, 3.0f);
    memset(xq, 0, 128 * 2);          /* an all-zero group: scale 0 */
    int8_t *q8 = xmalloc(batch * kq);
    float *q8s = xmalloc(batch * gq * sizeof(float));
    orc_quantize_input_q8(xq, batch, kq, gs, q8, q8s);
    CHECK(q8s[0] == 0.0f);
    float *wq = xmalloc(rows * kq * sizeof(float));
    for (size_t i = 0; i < rows * kq; i++) wq[i] = frand() * 0.05f;
    uint8_t *pq = xmalloc(rows * kq / 2);
    float *sq = xmalloc(rows * gq * sizeof(float)), *zq = xmalloc(rows * gq * sizeof(float));
    orc_quantize_tensor_int4(wq, rows, kq, gs, pq, sq, zq);
    uint16_t *sq16 = xmalloc(rows * gq * 2), *zq16 = xmalloc(rows * gq * 2);
    orc_convert_params_to_f16(sq, rows * gq, sq16);
    orc_convert_params_to_f16(zq, rows * gq, zq16);
    double *yd = xmalloc(batch * rows * sizeof(double));
    orc_matvec_int4xq8(q8, q8s, pq, sq16, zq16, batch, rows, kq, gs, yd);
    CHECK(isfinite(yd[batch * rows - 1]));

    free(w); free(packed); free(sc); free(zp); free(sc16); free(zp16); free(dense); free(dense2);
    free(x); free(awq); free(gamma); free(y); free(b); free(res); free(nrm); free(codes8);
    free(xq); free(q8); free(q8s); free(wq); free(pq); free(sq); free(zq); free(sq16); free(zq16); free(yd);
}

static void check_turboquant(void) {
    enum { D = 128, B = 2, T = 3, NKV = 2, NH = 4, MAXSEQ = 5 };
    float levels[256], bounds[255], klev[128], kbd[127];
    orc_lloyd_max_gaussian(D, 8, levels, bounds);
    orc_lloyd_max_gaussian(D, 7, klev, kbd);
    CHECK(isfinite(orc_normal_quantile(0.3)) && isfinite(orc_erf(0.7)));
    uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u}, out[16];
    orc_chacha_block(in, 12, out);
    uint64_t draws[70];
    orc_stdrng_stream(NULL, 42, 70, draws);   /* crosses a 4-block refill */
    CHECK(orc_pcg32_xsh_rr(orc_pcg32_advance(1, 3)) == orc_pcg32_xsh_rr(6364136223846793008ULL));
    float signs[D], *qjl = xmalloc((size_t)D * D * sizeof(float));
    orc_rotation_signs(D, 42, signs);
    orc_qjl_matrix(D, 43, qjl);
    float xr[D];
    for (int i = 0; i < D; i++) xr[i] = frand();
    orc_hadamard_rotate(xr, signs, D);

    uint16_t *one = f16_vec(D, 2.0f);
    uint8_t codes[D];
    float scale, rn;
    orc_tq_quantize_vector(one, D, 1, signs, klev, kbd, 128, qjl, codes, &scale, &rn);
    orc_tq_quantize_vector(one, D, 0, signs, levels, bounds, 256, qjl, codes, &scale, &rn);

    const size_t cells = (size_t)B * NKV * MAXSEQ;
    uint16_t *kv = f16_vec((size_t)B * T * NKV * D, 1.0f);
    uint8_t *kc = xmalloc(cells * D), *vc = xmalloc(cells * D);
    float *ks = xmalloc(cells * 4), *vs = xmalloc(cells * 4), *kr = xmalloc(cells * 4);
    memset(kc, 0, cells * D); memset(vc, 0, cells * D);
    memset(ks, 0, cells * 4); memset(vs, 0, cells * 4); memset(kr, 0, cells * 4);
    int32_t pos[B] = {3, 0};   /* sequence 0 wraps the ring of 5 */
    orc_tq_cache_write(kv, B, T, NKV, D, MAXSEQ, 0, pos, 1, signs, klev, kbd, 128, qjl, kc, ks, kr);
    orc_tq_cache_write(kv, B, T, NKV, D, MAXSEQ, 1, NULL, 0, signs, levels, bounds, 256, qjl, vc, vs, NULL);
    uint16_t *q = f16_vec((size_t)B * NH * D, 1.0f);
    float *o = xmalloc((size_t)B * NH * D * sizeof(float));
    int32_t lens[B] = {MAXSEQ, 0};   /* a full and an empty sequence */
    orc_tq_attention(q, B, NH, NKV, D, MAXSEQ, 0, lens, 0.088f, signs, klev, levels, qjl, kc, vc, ks, vs, kr, o, 2);
    CHECK(o[(size_t)NH * D] == 0.0f);

    uint16_t *kf = f16_vec(cells * D, 1.0f), *vf = f16_vec(cells * D, 1.0f);
    uint16_t *qp = f16_vec((size_t)B * T * NH * D, 1.0f);
    float *op = xmalloc((size_t)B * T * NH * D * sizeof(float));
    int32_t lens2[B] = {MAXSEQ, 2};   /* 3 query tokens over 2 positions: the first sees none */
    orc_fp16_attention(qp, B, T, NH, NKV, D, MAXSEQ, 0, lens2, 0.088f, kf, vf, op, 2);
    CHECK(op[(size_t)T * NH * D] == 0.0f);

    free(qjl); free(one); free(kv); free(kc); free(vc); free(ks); free(vs); free(kr); free(q); free(o);
    free(kf); free(vf); free(qp); free(op);
}

int main(void) {
    check_f16_and_packing();
    check_int4_int8();
    check_turboquant();
    printf("san_check: every oracle entry point ran clean\n");
    return 0;
}
