// int4_matvec.hip -- INT4-affine (group 128) decode matvec ops for gfx950:
// the C entry points, the image prep kernels, and the host logic that picks a
// launch shape and an activation source for the matvec kernel
// (int4_matvec_kernel.h, which describes the design).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <string>

#include "imh_internal.h"
#include "int4_gemm.h"
#include "int4_matvec_kernel.h"

namespace {

using namespace imh_int4;

// ---------------------------------------------------------------------------
// prep: activation -> operand image in memory (IMAGE source)
// ---------------------------------------------------------------------------
// Stores one group's sums (16 consecutive lanes -- a DPP row -- all live or
// all not) from the group's first lane, prescaled by 2^-24.
__device__ __forceinline__ void store_group_sums(float sh, float sl, bool live, float *gs_row, int G,
                                                 int g) {
    sh = row16_sum(sh);
    sl = row16_sum(sl);
    if (live && (threadIdx.x & 15) == 0) {
        gs_row[g] = sh * kTwoM24;
        gs_row[G + g] = sl * kTwoM24;
    }
}

// Plain mode.  grid (ceil(K/8/256), B), block 256; thread = one 8-element
// chunk; the 16 chunks of a group are 16 consecutive lanes (K % 128 == 0).
__global__ void __launch_bounds__(256) int4_prep_plain(const __half *__restrict__ x,
                                                        const __half *__restrict__ awq,
                                                        _Float16 *__restrict__ xa_hi,
                                                        _Float16 *__restrict__ xa_lo,
                                                        float *__restrict__ gsum, int K) {
    const int m = blockIdx.y;
    const int c_raw = blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = c_raw * 8 < K;
    const int c = live ? c_raw : 0;
    const int G = K / kGS;
    const size_t base = (size_t)m * K + (size_t)c * 8;
    uint4 xv = *reinterpret_cast<const uint4 *>(x + base);
    const _Float16 *xh = reinterpret_cast<const _Float16 *>(&xv);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (float)xh[i];
    if (awq) {
        uint4 av = *reinterpret_cast<const uint4 *>(awq + (size_t)c * 8);
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&av);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = div_awq(v[i], (float)ah[i]);
    }
    half8_t hi, lo;
    float sh, sl;
    chunk_operands(v, hi, lo, sh, sl);
    if (live) {
        const size_t ib = (size_t)m * K + (size_t)img_chunk(c) * 8;
        *reinterpret_cast<half8_t *>(xa_hi + ib) = hi;
        *reinterpret_cast<half8_t *>(xa_lo + ib) = lo;
    }
    store_group_sums(sh, sl, live, gsum + (size_t)m * 2 * G, G, c / 16);
}

// Residual + RMSNorm mode.  grid (B), block 256: r = a + b, rms_inv, writes
// residual_out / normed_out and the operand image of r * gamma / awq (the
// matvec then scales by rms_inv); `rounded` 1: of normed_out / awq instead;
// 2: both, the rounded one as the second image (hi2 / lo2 / gsum2).
// Thread t takes chunks t, t + 256, ..: the first CPT of them (all of them
// for K <= 2048 CPT) are loaded before the reduction and stay in registers,
// so the row waits one memory latency; chunks past those (K > 16384 at CPT 8)
// are read again after it.
template <int CPT>
__global__ void __launch_bounds__(256) int4_prep_resnorm(
    const __half *__restrict__ a, const __half *__restrict__ b, const __half *__restrict__ gamma,
    const __half *__restrict__ awq, float eps, __half *__restrict__ residual_out,
    __half *__restrict__ normed_out, _Float16 *__restrict__ xa_hi, _Float16 *__restrict__ xa_lo,
    float *__restrict__ gsum, float *__restrict__ rms_out, int K, int rounded, _Float16 *__restrict__ xa_hi2,
    _Float16 *__restrict__ xa_lo2, float *__restrict__ gsum2) {
    const int m = blockIdx.x;
    const int G = K / kGS;
    const int nchunk = K / 8;
    const size_t row = (size_t)m * K;
    __shared__ float red[256];
    __shared__ float rms_s;
    uint4 av[CPT], bv[CPT], gv[CPT], wv[CPT];
#pragma unroll
    for (int it = 0; it < CPT; it++) {
        const int c_raw = it * 256 + (int)threadIdx.x;
        const int c = c_raw < nchunk ? c_raw : 0;
        av[it] = *reinterpret_cast<const uint4 *>(a + row + (size_t)c * 8);
        bv[it] = *reinterpret_cast<const uint4 *>(b + row + (size_t)c * 8);
        gv[it] = *reinterpret_cast<const uint4 *>(gamma + (size_t)c * 8);
        wv[it] = awq ? *reinterpret_cast<const uint4 *>(awq + (size_t)c * 8) : make_uint4(0, 0, 0, 0);
    }
    const int iters = (nchunk + 255) / 256;   // > CPT only at CPT 8, K > 16384
    float sq = 0.0f;
    auto add_sq = [&](const uint4 &x, const uint4 &y) __attribute__((always_inline)) {
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&x);
        const _Float16 *bh = reinterpret_cast<const _Float16 *>(&y);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float r = (float)ah[i] + (float)bh[i];
            sq = __builtin_fmaf(r, r, sq);
        }
    };
#pragma unroll
    for (int it = 0; it < CPT; it++)
        if (it * 256 + (int)threadIdx.x < nchunk) add_sq(av[it], bv[it]);
    for (int it = CPT; it < iters; it++) {
        const int c = it * 256 + (int)threadIdx.x;
        if (c < nchunk)
            add_sq(*reinterpret_cast<const uint4 *>(a + row + (size_t)c * 8),
                   *reinterpret_cast<const uint4 *>(b + row + (size_t)c * 8));
    }
    const float rms_inv = block_rms_inv(sq, red, &rms_s, K, eps);
    if (threadIdx.x == 0) rms_out[m] = rms_inv;
    // every thread runs the same iterations (K / 8 is a multiple of 16), so
    // the 16 lanes of a group always meet in store_group_sums
    auto emit = [&](int it, const uint4 &x, const uint4 &y, const uint4 &gw, const uint4 &ww)
                    __attribute__((always_inline)) {
        const int c_raw = it * 256 + (int)threadIdx.x;
        const bool live = c_raw < nchunk;
        const int c = live ? c_raw : 0;
        const size_t off = row + (size_t)c * 8;
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&x);
        const _Float16 *bh = reinterpret_cast<const _Float16 *>(&y);
        const _Float16 *gh = reinterpret_cast<const _Float16 *>(&gw);
        float v[8], v2[8];
        half8_t res, nrm;
        for (int i = 0; i < 8; i++) {
            float r = (float)ah[i] + (float)bh[i];
            res[i] = (_Float16)r;
            nrm[i] = (_Float16)(r * rms_inv * (float)gh[i]);
            v[i] = rounded == 1 ? (float)nrm[i] : r * (float)gh[i];
            v2[i] = (float)nrm[i];
        }
        if (awq) {
            const _Float16 *wh = reinterpret_cast<const _Float16 *>(&ww);
            for (int i = 0; i < 8; i++) {
                v[i] = div_awq(v[i], (float)wh[i]);
                v2[i] = div_awq(v2[i], (float)wh[i]);
            }
        }
        half8_t hi, lo;
        float sh, sl;
        chunk_operands(v, hi, lo, sh, sl);
        const size_t ioff = row + (size_t)img_chunk(c) * 8;
        if (live) {
            *reinterpret_cast<half8_t *>(residual_out + off) = res;
            *reinterpret_cast<half8_t *>(normed_out + off) = nrm;
            *reinterpret_cast<half8_t *>(xa_hi + ioff) = hi;
            *reinterpret_cast<half8_t *>(xa_lo + ioff) = lo;
        }
        store_group_sums(sh, sl, live, gsum + (size_t)m * 2 * G, G, c / 16);
        if (rounded == 2) {   // uniform: the second (rounded) image
            chunk_operands(v2, hi, lo, sh, sl);
            if (live) {
                *reinterpret_cast<half8_t *>(xa_hi2 + ioff) = hi;
                *reinterpret_cast<half8_t *>(xa_lo2 + ioff) = lo;
            }
            store_group_sums(sh, sl, live, gsum2 + (size_t)m * 2 * G, G, c / 16);
        }
    };
#pragma unroll
    for (int it = 0; it < CPT; it++) emit(it, av[it], bv[it], gv[it], wv[it]);
    for (int it = CPT; it < iters; it++) {
        const int c = min(it * 256 + (int)threadIdx.x, nchunk - 1);
        emit(it, *reinterpret_cast<const uint4 *>(a + row + (size_t)c * 8),
             *reinterpret_cast<const uint4 *>(b + row + (size_t)c * 8),
             *reinterpret_cast<const uint4 *>(gamma + (size_t)c * 8),
             awq ? *reinterpret_cast<const uint4 *>(awq + (size_t)c * 8) : make_uint4(0, 0, 0, 0));
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

int check_weight(const imh_affine_int4_weight *w, const char *who) {
    if (!w || !w->data || !w->scales || !w->zeros)
        return imh::fail(IMH_EINVAL, std::string(who) + ": weight or one of its arrays is NULL");
    if (w->group_size != kGS)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": group_size " +
                                               std::to_string(w->group_size) +
                                               " not supported (built for 128)");
    if (w->n == 0 || w->k == 0 || w->k % kGS != 0)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": k=" + std::to_string(w->k) +
                                               " must be a non-zero multiple of 128, n=" +
                                               std::to_string(w->n) + " non-zero");
    if ((reinterpret_cast<uintptr_t>(w->data) & 15) != 0)
        return imh::fail(IMH_EINVAL, std::string(who) + ": weight data must be 16-byte aligned");
    return IMH_OK;
}

bool misaligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

// image layout in stream scratch: hi [B][K] f16, lo [B][K] f16, group sums
// [B][2][K/128] f32, row scales [B] f32
size_t image_bytes(uint32_t B, uint32_t K) {
    return (size_t)B * K * 4 + (size_t)B * 2 * (K / kGS) * 4 + (size_t)B * 4 + 256;
}

void image_layout(void *storage, uint32_t B, uint32_t K, ActIn &in, float **rms) {
    _Float16 *hi = static_cast<_Float16 *>(storage);
    _Float16 *lo = hi + (size_t)B * K;
    float *gs = reinterpret_cast<float *>(lo + (size_t)B * K);
    *rms = gs + (size_t)B * 2 * (K / kGS);
    in.hi = hi;
    in.lo = lo;
    in.gsum = gs;
    in.row_scale = nullptr;
}

// Waves per tile.  Each wave holds at most kMaxGroups groups per stage, and
// the whole grid should be resident at once -- one round of workgroups, so
// every weight load is in flight together.  The kernels run 6 waves per SIMD
// (24 per CU); within that, ~6 waves per SIMD in total is enough to cover
// HBM latency.
int pick_parts(int tiles, int nmat, int G, int cus) {
    const int need = (G + kMaxGroups - 1) / kMaxGroups;
    const int per_cu = (tiles + cus - 1) / cus;              // workgroups each CU must hold
    const int resident = 24 / per_cu / nmat;
    const int total = 6 * 4 * cus / std::max(1, tiles * nmat);
    const int cap = std::min(kMaxWaves / nmat, G);
    return std::max(1, std::min(cap, std::max(need, std::min(resident, total))));
}

// The launch shape of one op.  raw: the workgroups build the image
// themselves (when all of K fits one stage at two 8-element chunks per thread).
struct Plan {
    Launch L;
    bool raw;
};

int plan_launch(imh_stream *s, int nmat, bool rn, int N, int K, int B, const char *who, Plan &p) {
    const int G = K / kGS;
    const int rows = std::min(B, 16);
    const int MT = rows > 8 ? 2 : 1;
    const int tiles = (N + 15) / 16;
    const int btiles = (B + 15) / 16;
    // the residual-norm source at one row (the decoder's Q|K|V, 384 tiles):
    // eight waves per tile, not the twelve the residency rule gives --
    // decode step B=1 1.613 -> 1.565 ms (4 waves 1.564, 5 1.573, 6 1.585,
    // 10 1.604, 16 1.725 ms; A/B on one box, two rounds)
    const int parts = (rn && nmat == 1 && B == 1)
                          ? std::max((G + kMaxGroups - 1) / kMaxGroups, std::min(8, G))
                          : pick_parts(tiles * btiles, nmat, G, s->dev->props.multiProcessorCount);
    const int waves = nmat * parts;
    const int nthr = 64 * waves;
    const size_t red_bytes = (size_t)MT * waves * 64 * sizeof(float4_t);
    const size_t per_group = (size_t)2 * rows * kGS * sizeof(_Float16);
    const size_t pad = (size_t)2 * rows * 8 * sizeof(_Float16);
    // RAW when the workgroup's share of building the operand is small: all of
    // K in one stage at two chunks per thread, or (plain source, any number
    // of stages) up to 96 row-groups -- ~12K elements, measured the break-even
    // against the prep launch at batch 2-8 (K 2560-9728).  Else IMAGE.
    size_t fixed = 0;
    int SG = 0;
    for (int raw = 1; raw >= 0; raw--) {
        p.raw = raw && MT == 1 && (rows * G * 16 <= 2 * nthr || (!rn && rows * G <= 96));
        if (raw && !p.raw) continue;
        // LDS: scales/zeros, group sums (+ RN sums and rms), then
        // max(activation planes, partial sums)
        fixed = (size_t)nmat * G * 16 * 4 + (size_t)G * MT * 16 * 4 + (rn && p.raw ? (size_t)G * 16 * 4 + 64 : 0);
        if (fixed + pad + per_group > (size_t)kLdsBudget || fixed + red_bytes > (size_t)kLdsBudget)
            return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": k=" + std::to_string(K) +
                                                   " too large for the LDS staging of this kernel");
        SG = (int)((kLdsBudget - fixed - pad) / per_group);
        SG = std::min(std::min(SG, parts * kMaxGroups), G);
        // several RAW stages only under the row-group rule (RAW_RN needs the
        // whole row in one stage)
        if (!p.raw || SG == G || (!rn && rows * G <= 96)) break;
    }
    Launch &L = p.L;
    L.grid = dim3(tiles, btiles);
    L.block = dim3(nthr);
    L.lds = fixed + std::max(pad + (size_t)SG * per_group, red_bytes);
    L.st = s->stream;
    L.N = N, L.K = K, L.B = B, L.parts = parts, L.SG = SG;
    L.ng = (SG + parts - 1) / parts;
    L.xc = rows * SG * 16 <= nthr ? 1 : 2;
    L.mt = MT;
    return IMH_OK;
}

int launch_image(int nmat, int epi, const Launch &L, const MatPtrs &mp, const ActIn &in) {
    if (L.mt == 2) {
        launch_image_mt2(nmat, epi, L, mp, in);
    } else if (nmat == 1) {
        launch_ng<1, EPI_STORE, 1, SRC_IMAGE>(L, mp, in);
    } else if (epi == EPI_SILU) {
        launch_ng<2, EPI_SILU, 1, SRC_IMAGE>(L, mp, in);
    } else if (epi == EPI_GELU) {
        launch_ng<2, EPI_GELU, 1, SRC_IMAGE>(L, mp, in);
    } else {
        launch_ng<2, EPI_STORE, 1, SRC_IMAGE>(L, mp, in);
    }
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

// Prefill-sized token counts: the residual-norm rows first when asked, then
// the GEMM (one matrix, or a gate/up pair with its epilogue).  Scratch slot 2
// holds the GEMM's split-K partials.
int run_gemm(imh_stream *s, const ActIn &in, int M, const imh_affine_int4_weight *w0,
             const imh_affine_int4_weight *w1, int epi, uint16_t *out0, uint16_t *out1) {
    const int N = (int)w0->n, K = (int)w0->k;
    const int nmat = w1 ? 2 : 1;
    const int cus = s->dev->props.multiProcessorCount;
    void *ws = nullptr;
    const size_t ws_bytes = gemm_workspace_bytes(M, N, K, nmat, cus);
    int rc = IMH_OK;
    if (ws_bytes) {
        rc = imh::stream_scratch(s, 2, ws_bytes, &ws);
        if (rc) return rc;
    }
    const __half *x = in.a;
    if (in.b) {   // residual + RMSNorm rows, then the projection of the normed rows
        rc = encode_resnorm_rows(s, in.a, in.b, in.gamma, in.eps, in.residual_out, in.normed_out, M, K);
        if (rc) return rc;
        x = in.normed_out;
    }
    const int ge = epi == EPI_SILU ? 2 : epi == EPI_GELU ? 3 : 0;
    return encode_gemm(s, x, M, w0, w1, ge, reinterpret_cast<__half *>(out0), reinterpret_cast<__half *>(out1),
                       ws);
}

// Split-K over the image in in.hi / in.lo (and hi2 / lo2 for a mixed
// rounding's later segments) when it applies: one matrix with its row
// segments, plain store (partials in stream scratch slot 2).
int try_splitk(imh_stream *s, int nmat, int epi, int N, int K, uint32_t B, const MatPtrs &mp, const ActIn &in,
               bool *used) {
    *used = false;
    const int cus = s->dev->props.multiProcessorCount;
    const int split_rows = (in.round_mode == 2 && mp.seg[0] > 0) ? mp.seg[0] : N;
    if (epi != EPI_STORE || !splitk_applies(nmat, (int)B, N, K, split_rows, cus)) return IMH_OK;
    void *ws = nullptr;
    int rc = imh::stream_scratch(s, 2, splitk_workspace_bytes((int)B, N, split_rows, cus), &ws);
    if (rc) return rc;
    *used = true;
    return launch_splitk(s->stream, cus, N, K, (int)B, mp, in, split_rows, ws);
}

// Plans and launches the matvec kernel for mp (N rows in total, segments
// included): RAW when the workgroups can build the operand image themselves,
// else the prep kernel writes it into stream scratch slot 0 first.
int run_matvec(imh_stream *s, ActIn in, uint32_t B, int nmat, int epi, int N, int K, const MatPtrs &mp,
               const char *who) {
    const bool rn = in.b != nullptr;
    const int cus = s->dev->props.multiProcessorCount;
    {
        bool used = false;
        const int rc = launch_band_matvec(s->stream, cus, (int)B, nmat, epi, N, K, mp, in, &used);
        if (rc || used) return rc;
    }
    if (rn && in.round_mode == 1 && B > 2) {
        // 3-8 rows reading the f16 normed rows: the rows kernel writes the
        // residual and normed rows, then the band kernel projects the normed
        // rows as a plain source (one band launch instead of a prep + tile pair)
        ActIn pin = {};
        pin.a = in.normed_out;
        pin.awq = in.awq;
        bool fits = false;
        int rc = launch_band_matvec(s->stream, cus, (int)B, nmat, epi, N, K, mp, pin, &fits, true);
        if (rc) return rc;
        if (fits) {
            rc = encode_resnorm_rows(s, in.a, in.b, in.gamma, in.eps, in.residual_out, in.normed_out, (int)B, K);
            return rc ? rc : run_matvec(s, pin, B, nmat, epi, N, K, mp, who);
        }
    }
    Plan p;
    int rc = plan_launch(s, nmat, rn, N, K, (int)B, who, p);
    if (rc) return rc;
    if (p.raw) {
        launch_raw(nmat, epi, rn, p.L, mp, in);
        IMH_HIP(hipGetLastError());
        return IMH_OK;
    }
    // IMAGE: the prep kernel writes the image into stream scratch first
    // (two images for a mixed rounding: the unrounded one for the first
    // segment, the rounded one for the rest)
    const bool two = rn && in.round_mode == 2;
    void *scr = nullptr;
    rc = imh::stream_scratch(s, 0, image_bytes(B, K) * (two ? 2 : 1), &scr);
    if (rc) return rc;
    float *rms, *rms2;
    ActIn in2 = in;
    if (two) image_layout(static_cast<uint8_t *>(scr) + image_bytes(B, K), B, K, in2, &rms2);
    image_layout(scr, B, K, in, &rms);
    _Float16 *hi = const_cast<_Float16 *>(in.hi);
    _Float16 *lo = const_cast<_Float16 *>(in.lo);
    float *gs = const_cast<float *>(in.gsum);
    if (rn) {
        const int rounded = in.round_mode;
        const int cpt = resnorm_cpt(K);
        auto kern = cpt == 1 ? int4_prep_resnorm<1>
                    : cpt == 2 ? int4_prep_resnorm<2>
                    : cpt == 4 ? int4_prep_resnorm<4>
                               : int4_prep_resnorm<8>;
        hipLaunchKernelGGL(kern, dim3(B), dim3(256), 0, s->stream, in.a, in.b, in.gamma, in.awq, in.eps,
                           in.residual_out, in.normed_out, hi, lo, gs, rms, K, rounded,
                           const_cast<_Float16 *>(in2.hi), const_cast<_Float16 *>(in2.lo),
                           const_cast<float *>(in2.gsum));
        in.row_scale = rounded == 1 ? nullptr : rms;
        if (two) {
            in.hi2 = in2.hi;
            in.lo2 = in2.lo;
            in.gsum2 = in2.gsum;
        }
    } else {
        dim3 grid((K / 8 + 255) / 256, B);
        hipLaunchKernelGGL(int4_prep_plain, grid, dim3(256), 0, s->stream, in.a, in.awq, hi, lo, gs, K);
    }
    IMH_HIP(hipGetLastError());
    {
        bool used = false;
        rc = try_splitk(s, nmat, epi, N, K, B, mp, in, &used);
        if (rc || used) return rc;
    }
    if (image_da_applies(nmat, (int)B, K)) return launch_image_da(s->stream, nmat, epi, N, K, (int)B, mp, in);
    return launch_image(nmat, epi, p.L, mp, in);
}

// Validates the weights and runs the op: x (plain) or the residual-norm
// inputs (in.b != NULL) -> out0 [, out1].
int run_op(imh_stream *s, ActIn in, uint32_t B, const imh_affine_int4_weight *w0,
           const imh_affine_int4_weight *w1, int epi, uint16_t *out0, uint16_t *out1, const char *who) {
    if (!s || !in.a) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_weight(w0, who);
    if (rc) return rc;
    if (w1) {
        rc = check_weight(w1, who);
        if (rc) return rc;
        if (w1->n != w0->n || w1->k != w0->k)  // D7: the reference assumes N_up == N_gate
            return imh::fail(IMH_EINVAL, std::string(who) + ": gate and up shapes differ");
    }
    if (!out0 || (w1 && epi == EPI_STORE && !out1))
        return imh::fail(IMH_EINVAL, std::string(who) + ": NULL output");
    if (misaligned16(in.a) || misaligned16(in.b) || misaligned16(in.gamma) || misaligned16(in.awq) ||
        misaligned16(in.residual_out) || misaligned16(in.normed_out))
        return imh::fail(IMH_EINVAL, std::string(who) + ": activation vectors must be 16-byte aligned");
    if (B == 0) return IMH_OK;
    rc = imh::use_device(s->dev);
    if (rc) return rc;
    MatPtrs mp = {};
    const imh_affine_int4_weight *ws[2] = {w0, w1};
    for (int i = 0; i < (w1 ? 2 : 1); i++) {
        mp.data[i] = ws[i]->data;
        mp.scales[i] = reinterpret_cast<const __half *>(ws[i]->scales);
        mp.zeros[i] = reinterpret_cast<const __half *>(ws[i]->zeros);
    }
    mp.out[0] = reinterpret_cast<__half *>(out0);
    mp.out[1] = reinterpret_cast<__half *>(out1);
    if ((int)B >= kGemmMinTokens) return run_gemm(s, in, (int)B, w0, w1, epi, out0, out1);
    return run_matvec(s, in, B, w1 ? 2 : 1, epi, (int)w0->n, (int)w0->k, mp, who);
}

// x is divided by the first weight's awq_scales; a gate/up pair shares that
// activation (ops/quantized.rs:218-224), so up's own awq_scales are not read.
ActIn plain_in(const uint16_t *x, const imh_affine_int4_weight *w) {
    ActIn in = {};
    in.a = reinterpret_cast<const __half *>(x);
    in.awq = w ? reinterpret_cast<const __half *>(w->awq_scales) : nullptr;
    return in;
}

MatPtrs mat_ptrs(const imh_affine_int4_weight *w0, const imh_affine_int4_weight *w1, uint16_t *out0) {
    MatPtrs mp = {};
    const imh_affine_int4_weight *ws[2] = {w0, w1};
    for (int i = 0; i < (w1 ? 2 : 1); i++) {
        mp.data[i] = ws[i]->data;
        mp.scales[i] = reinterpret_cast<const __half *>(ws[i]->scales);
        mp.zeros[i] = reinterpret_cast<const __half *>(ws[i]->zeros);
    }
    mp.out[0] = reinterpret_cast<__half *>(out0);
    return mp;
}

// An FFN block (gate/up + activation, then down) at 1-8 rows whose gate/up
// runs on the row-band kernel: that launch also writes the down projection's
// operand image (act / down's AWQ scales, split into f16 hi + lo), and the
// down launch stages that image instead of forming it from act -- at 1-2 rows
// the band kernel (whose every workgroup would otherwise divide and split all
// of K), at 3-8 the tile kernel, which then needs no prep launch; either sums
// the groups itself.  gin: the gate/up source (plain, or residual-norm: at
// 3-8 rows the rows kernel writes the residual and normed rows first and
// gate/up read those).  *done false: nothing was launched (the caller runs
// the two ops).
int ffn_band_pair(imh_stream *s, ActIn gin, uint32_t B, const imh_affine_int4_weight *gate,
                  const imh_affine_int4_weight *up, const imh_affine_int4_weight *down, uint16_t *act_out,
                  uint16_t *y, int epi, bool *done) {
    *done = false;
    if (B < 1 || B > 8 || !act_out || !y || misaligned16(act_out)) return IMH_OK;
    if (misaligned16(gin.a) || misaligned16(gin.b) || misaligned16(gin.gamma) || misaligned16(gin.awq) ||
        misaligned16(gin.residual_out) || misaligned16(gin.normed_out) || misaligned16(down->awq_scales))
        return IMH_OK;
    if (check_weight(gate, "") || check_weight(up, "") || check_weight(down, "")) {
        imh::clear_error();
        return IMH_OK;
    }
    if (up->n != gate->n || up->k != gate->k || down->k != gate->n) return IMH_OK;
    const bool rn = gin.b != nullptr;
    if (rn && B > 2 && gin.round_mode != 1) return IMH_OK;
    int rc = imh::use_device(s->dev);
    if (rc) return rc;
    const int cus = s->dev->props.multiProcessorCount;
    const int F = (int)gate->n, H = (int)gate->k, Hd = (int)down->n;
    void *scr = nullptr;
    rc = imh::stream_scratch(s, 0, (size_t)2 * B * F * sizeof(_Float16), &scr);
    if (rc) return rc;
    _Float16 *ihi = static_cast<_Float16 *>(scr), *ilo = ihi + (size_t)B * F;
    MatPtrs gm = mat_ptrs(gate, up, act_out);
    MatPtrs dm = mat_ptrs(down, nullptr, y);
    ActIn pin = gin;   // the source the gate/up launch reads
    if (rn && B > 2) {
        pin = ActIn{};
        pin.a = gin.normed_out;
        pin.awq = gin.awq;
    }
    pin.img_out_hi = ihi;
    pin.img_out_lo = ilo;
    pin.img_awq = reinterpret_cast<const __half *>(down->awq_scales);
    ActIn din = {};
    din.a = reinterpret_cast<const __half *>(act_out);
    din.hi = ihi;
    din.lo = ilo;   // gsum NULL: the down launch sums the groups
    bool fg = false, fd = false;
    Plan p{};
    rc = launch_band_matvec(s->stream, cus, (int)B, 2, epi, F, H, gm, pin, &fg, true);
    if (rc || !fg) return rc;
    if (B <= 2) {
        din.img_src = 1;
        rc = launch_band_matvec(s->stream, cus, (int)B, 1, EPI_STORE, Hd, F, dm, din, &fd, true);
        if (rc || !fd) return rc;
    } else {
        if (plan_launch(s, 1, false, Hd, F, (int)B, "ffn_band_pair", p) || p.raw) {
            imh::clear_error();
            return IMH_OK;   // a RAW down (small K) builds its own operand
        }
        if (splitk_applies(1, (int)B, Hd, F, Hd, cus)) {   // reserve the partials before the first launch
            void *ws = nullptr;
            rc = imh::stream_scratch(s, 2, splitk_workspace_bytes((int)B, Hd, Hd, cus), &ws);
            if (rc) return rc;
        }
    }
    if (rn && B > 2) {
        rc = encode_resnorm_rows(s, gin.a, gin.b, gin.gamma, gin.eps, gin.residual_out, gin.normed_out, (int)B, H);
        if (rc) return rc;
    }
    rc = launch_band_matvec(s->stream, cus, (int)B, 2, epi, F, H, gm, pin, &fg);
    if (rc) return rc;
    if (!fg) return imh::fail(IMH_EDEVICE, "ffn_band_pair: the gate/up launch was refused after its probe");
    if (B <= 2) {
        rc = launch_band_matvec(s->stream, cus, (int)B, 1, EPI_STORE, Hd, F, dm, din, &fd);
        if (rc) return rc;
        if (!fd) return imh::fail(IMH_EDEVICE, "ffn_band_pair: the down launch was refused after its probe");
    } else {
        bool used = false;
        rc = try_splitk(s, 1, EPI_STORE, Hd, F, B, dm, din, &used);
        if (rc) return rc;
        if (!used && image_da_applies(1, (int)B, F)) {
            rc = launch_image_da(s->stream, 1, EPI_STORE, Hd, F, (int)B, dm, din);
            if (rc) return rc;
            used = true;
        }
        if (!used) {
            rc = launch_image(1, EPI_STORE, p.L, dm, din);
            if (rc) return rc;
            IMH_HIP(hipGetLastError());
        }
    }
    *done = true;
    return IMH_OK;
}

}  // namespace

namespace imh {

int encode_segmented_matvec_int4(imh_stream *s, const uint16_t *x, const imh_fused_residual_norm_params *rn,
                                 uint32_t B, int nseg, const imh_affine_int4_weight *const *w,
                                 uint16_t *const *out) {
    const char *who = "encode_segmented_matvec_int4";
    if (!s || (!x && !rn) || !w || !out || nseg < 1 || nseg > 3)
        return fail(IMH_EINVAL, std::string(who) + ": bad argument");
    int N = 0;
    for (int i = 0; i < nseg; i++) {
        int rc = check_weight(w[i], who);
        if (rc) return rc;
        if (!out[i]) return fail(IMH_EINVAL, std::string(who) + ": NULL output");
        if (w[i]->k != w[0]->k || w[i]->awq_scales != w[0]->awq_scales)
            return fail(IMH_EINVAL, std::string(who) + ": segments must share k and the AWQ scales");
        if (i + 1 < nseg && w[i]->n % 16)
            return fail(IMH_EINVAL, std::string(who) + ": segment rows must be a multiple of 16");
        N += (int)w[i]->n;
    }
    ActIn in = plain_in(x, w[0]);
    if (rn) {
        if (!rn->a || !rn->b || !rn->norm_weight || !rn->residual_output || !rn->normed_output)
            return fail(IMH_EINVAL, std::string(who) + ": NULL argument");
        in.a = reinterpret_cast<const __half *>(rn->a);
        in.b = reinterpret_cast<const __half *>(rn->b);
        in.gamma = reinterpret_cast<const __half *>(rn->norm_weight);
        in.residual_out = reinterpret_cast<__half *>(rn->residual_output);
        in.normed_out = reinterpret_cast<__half *>(rn->normed_output);
        in.eps = rn->eps;
    }
    if (rn && nseg > 1 && (int)B < kGemmMinTokens) {
        // the first segment projects r * gamma * rms_inv unrounded (the fused
        // residual-norm projection); the others read the f16 normed rows, as
        // they would after a separate norm (RAW: each workgroup builds the
        // operand its segment reads; IMAGE: the prep kernel writes both)
        in.round_mode = 2;
    }
    if ((int)B >= kGemmMinTokens || nseg == 1) {   // one op per weight, the later ones on the normed rows
        int rc = run_op(s, in, B, w[0], nullptr, EPI_STORE, out[0], nullptr, who);
        const uint16_t *xn = rn ? rn->normed_output : x;
        for (int i = 1; i < nseg && !rc; i++)
            rc = run_op(s, plain_in(xn, w[0]), B, w[i], nullptr, EPI_STORE, out[i], nullptr, who);
        return rc;
    }
    if (misaligned16(in.a) || misaligned16(in.b) || misaligned16(in.gamma) || misaligned16(in.awq) ||
        misaligned16(in.residual_out) || misaligned16(in.normed_out))
        return fail(IMH_EINVAL, std::string(who) + ": activation vectors must be 16-byte aligned");
    if (B == 0) return IMH_OK;
    int rc = use_device(s->dev);
    if (rc) return rc;
    MatPtrs mp = {};
    int row = 0;
    for (int i = 0; i < nseg; i++) {
        mp.data[i] = w[i]->data;
        mp.scales[i] = reinterpret_cast<const __half *>(w[i]->scales);
        mp.zeros[i] = reinterpret_cast<const __half *>(w[i]->zeros);
        mp.out[i] = reinterpret_cast<__half *>(out[i]);
        if (i) mp.seg[i - 1] = row;
        row += (int)w[i]->n;
    }
    return run_matvec(s, in, B, 1, EPI_STORE, N, (int)w[0]->k, mp, who);
}

int encode_resnorm_gate_up_act_int4(imh_stream *s, const imh_fused_residual_norm_params *rn, uint32_t B,
                                    const imh_affine_int4_weight *gate, const imh_affine_int4_weight *up,
                                    uint16_t *out, int use_gelu) {
    const char *who = "encode_resnorm_gate_up_act_int4";
    if (!s || !rn || !rn->a || !rn->b || !rn->norm_weight || !rn->residual_output || !rn->normed_output || !gate ||
        !up || !out)
        return fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    ActIn in = plain_in(nullptr, gate);
    in.a = reinterpret_cast<const __half *>(rn->a);
    in.b = reinterpret_cast<const __half *>(rn->b);
    in.gamma = reinterpret_cast<const __half *>(rn->norm_weight);
    in.residual_out = reinterpret_cast<__half *>(rn->residual_output);
    in.normed_out = reinterpret_cast<__half *>(rn->normed_output);
    in.eps = rn->eps;
    in.round_mode = 1;   // gate and up read the f16 normed rows
    return run_op(s, in, B, gate, up, use_gelu ? EPI_GELU : EPI_SILU, out, nullptr, who);
}

int encode_resnorm_ffn_block_int4(imh_stream *s, const imh_fused_residual_norm_params *rn, uint32_t B,
                                  const imh_affine_int4_weight *gate, const imh_affine_int4_weight *up,
                                  const imh_affine_int4_weight *down, uint16_t *act, uint16_t *y, int use_gelu) {
    if (s && rn && rn->a && rn->b && rn->norm_weight && rn->residual_output && rn->normed_output && gate && up &&
        down) {
        ActIn in = plain_in(nullptr, gate);
        in.a = reinterpret_cast<const __half *>(rn->a);
        in.b = reinterpret_cast<const __half *>(rn->b);
        in.gamma = reinterpret_cast<const __half *>(rn->norm_weight);
        in.residual_out = reinterpret_cast<__half *>(rn->residual_output);
        in.normed_out = reinterpret_cast<__half *>(rn->normed_output);
        in.eps = rn->eps;
        in.round_mode = 1;
        bool done = false;
        const int rc = ffn_band_pair(s, in, B, gate, up, down, act, y, use_gelu ? EPI_GELU : EPI_SILU, &done);
        if (rc || done) return rc;
    }
    const int rc = encode_resnorm_gate_up_act_int4(s, rn, B, gate, up, act, use_gelu);
    return rc ? rc : imh_encode_affine_projection_int4(s, act, B, down, y);
}

}  // namespace imh

extern "C" {

int imh_encode_affine_projection_int4(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                      const imh_affine_int4_weight *w, uint16_t *y) {
    return run_op(stream, plain_in(x, w), token_count, w, nullptr, EPI_STORE, y, nullptr,
                  "imh_encode_affine_projection_int4");
}

int imh_encode_batched_affine_matvec_int4(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                          const imh_affine_int4_weight *gate, uint16_t *gate_out,
                                          const imh_affine_int4_weight *up, uint16_t *up_out) {
    const char *who = "imh_encode_batched_affine_matvec_int4";
    if (!gate_out || !up_out || !up) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    return run_op(stream, plain_in(x, gate), token_count, gate, up, EPI_STORE, gate_out, up_out, who);
}

int imh_encode_fused_ffn_gate_up_act_int4(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                                          const imh_affine_int4_weight *gate,
                                          const imh_affine_int4_weight *up, uint16_t *out,
                                          int use_gelu) {
    const char *who = "imh_encode_fused_ffn_gate_up_act_int4";
    if (!out || !up) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    return run_op(stream, plain_in(x, gate), token_count, gate, up, use_gelu ? EPI_GELU : EPI_SILU, out,
                  nullptr, who);
}

int imh_encode_ffn_block_int4(imh_stream *stream, const uint16_t *x, uint32_t token_count,
                              const imh_affine_int4_weight *gate, const imh_affine_int4_weight *up,
                              const imh_affine_int4_weight *down, uint16_t *act_out, uint16_t *y, int use_gelu) {
    const char *who = "imh_encode_ffn_block_int4";
    if (!stream || !x || !act_out || !y || !gate || !up || !down)
        return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_weight(down, who);
    if (rc) return rc;
    if (down->k != gate->n)
        return imh::fail(IMH_EINVAL, std::string(who) + ": down.k must equal the intermediate size (gate.n)");
    {
        bool done = false;
        rc = ffn_band_pair(stream, plain_in(x, gate), token_count, gate, up, down, act_out, y,
                           use_gelu ? EPI_GELU : EPI_SILU, &done);
        if (rc || done) return rc;
    }
    rc = run_op(stream, plain_in(x, gate), token_count, gate, up, use_gelu ? EPI_GELU : EPI_SILU, act_out, nullptr,
                who);
    return rc ? rc : run_op(stream, plain_in(act_out, down), token_count, down, nullptr, EPI_STORE, y, nullptr, who);
}

int imh_encode_fused_residual_norm_affine_matvec_int4(imh_stream *stream,
                                                      const imh_fused_residual_norm_params *p) {
    const char *who = "imh_encode_fused_residual_norm_affine_matvec_int4";
    if (!stream || !p || !p->a || !p->b || !p->norm_weight || !p->residual_output || !p->output ||
        !p->normed_output)
        return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    ActIn in = plain_in(p->a, p->weight);
    in.b = reinterpret_cast<const __half *>(p->b);
    in.gamma = reinterpret_cast<const __half *>(p->norm_weight);
    in.residual_out = reinterpret_cast<__half *>(p->residual_output);
    in.normed_out = reinterpret_cast<__half *>(p->normed_output);
    in.eps = p->eps;
    return run_op(stream, in, p->token_count, p->weight, nullptr, EPI_STORE, p->output, nullptr, who);
}

}  // extern "C"
