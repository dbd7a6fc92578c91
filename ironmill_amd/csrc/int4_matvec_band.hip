// int4_matvec_band.hip -- the INT4-affine (group 128) decode matvec for one
// or two batch rows over a grid balanced on the compute units.
//
// Same semantics and arithmetic as int4_matvec_kernel (int4_matvec_kernel.h):
//     y[m][r] = sum_g s[r][g] * (sum_{k in g} xe[m][k] q[r][k] - z[r][g] sum xe),
// xe = x / awq, the raw code bytes entering v_mfma_f32_16x16x32_f16 as f16
// denormals against the slot-ordered activation split into f16 hi + lo, the
// zero point applied to the per-group operand sums, f32 accumulation.  What
// differs is the shape of the work, taken from the streaming probe
// (imh_diag_stream_read): one launch moves the most bytes when every compute
// unit gets the same share (grids of a multiple of the CU count beat the
// 608 / 160 workgroups that one 16-row tile per workgroup gives the Qwen3-4B
// gate+up / down weights), and a wave-wide load of 8 rows x 128 contiguous
// bytes beats 16 rows x 64.
//
//  * Workgroup b of NWG owns the row band [N b / NWG, N (b+1) / NWG) of each
//    matrix (one matrix, or the gate/up pair whose rows the epilogue joins),
//    cut into tiles of 8 rows (the last one masked).  Its waves split the K
//    groups of every tile: wave (mat, part) takes group pairs [p0, p0 + np)
//    of matrix mat in every tile, all of its weight loads issued up front.
//  * MFMA mapping.  B column j = r + 8h: row r of the tile, group h of the
//    pair (one 16-byte load per lane: row j & 7, group j >> 3, quarter lane >>
//    4).  A row i = 8h + 4·plane + b: batch row b, f16 hi (plane 0) or lo
//    (plane 1) half of group h's operand.  Of the 16 x 16 result only the
//    entries whose row and column share h are used; lane l holds rows
//    4(l >> 4) .. +3 of column l & 15, i.e. the batch rows of one (h, plane)
//    for one (r, h) when (l >> 5) == ((l >> 3) & 1).
//  * The activation operand image (all of K) and the band's scales / zeros
//    are staged once per workgroup in LDS, from loads issued ahead of the
//    weight loads; one barrier, then the MFMAs consume the weights as they
//    arrive; a second barrier joins the waves' partial rows (in part order:
//    deterministic).
//  * Residual-norm source (RN): r = a + b, every workgroup reduces the row's
//    sum of squares itself (per-group sums through LDS, one barrier, then
//    each thread adds them in the order of int4_matvec_kernel's row_rms) and
//    builds the operand r * gamma (round_mode 0, rms_inv scaling the output)
//    or f16(r * rms_inv * gamma) (round_mode 1) divided by awq; workgroup 0
//    also writes residual_out = f16(r) and normed_out = f16(r * rms_inv *
//    gamma).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <type_traits>

#include "imh_internal.h"
#include "int4_matvec_kernel.h"

namespace imh_int4 {

namespace {

constexpr int kRS = kGS + 8;   // halfs per operand row in LDS (16-byte pad)
constexpr int kSZC = 2;        // scale/zero words per thread loaded ahead of the weights

struct BandLds {
    size_t img, gs, sz, rsq, red, total;
};

__host__ __device__ inline BandLds band_lds(int G, int BM, int NMAT, int TM, int waves, bool rn) {
    BandLds L;
    const int NH = (BM + 3) / 4;   // MFMA passes of up to 4 batch rows
    L.img = 0;
    L.gs = L.img + (size_t)G * 2 * BM * kRS * 2;
    L.sz = L.gs + (size_t)G * 2 * BM * 4;
    L.rsq = L.sz + (size_t)NMAT * G * TM * 8 * 4;
    L.red = L.rsq + (rn ? (size_t)G * BM * 4 + (size_t)BM * 4 : 0);
    L.red = (L.red + 15) & ~(size_t)15;
    L.total = L.red + (size_t)waves * TM * 8 * 16 * NH;
    return L;
}

// grid NWG; block 64 * NMAT * W.
// Leading arguments: what the loads ahead of the issue-order barrier need,
// which the dispatcher preloads into SGPRs (14 at most) before the first
// instruction -- so those loads do not wait for the argument memory:
//   plain (and MB): x, awq, scales / zeros of matrix 0, then those of matrix
//                   1 (two matrices) or matrix 0's weights (one);
//   residual-norm:  a, b, gamma, awq, scales / zeros of matrix 0;
//   image:          hi, lo, scales / zeros, weights;
// and the dimensions in two words, nwb = N | W << 20 | B << 24 and kg = K |
// NWG << 16 (the grid and block sizes would be argument loads of their own).
// The rest comes from mp / in.  (Eight pointers of 48 bits with the
// dimensions in their high halves, seven words, measured no faster: gate+up
// B=1 7.96 -> 7.91 us, down 6.46 -> 6.57.)
struct BandLead {
    const void *p[6];
    uint32_t nwb, kg;
};
template <int NMAT, int EPI, int TM, int NP, int BM, int XC, bool RN, bool IMG = false, int PD = 1, bool MB = false>
__global__ void __launch_bounds__(512) int4_band_kernel(const void *l0, const void *l1, const void *l2,
                                                        const void *l3, const void *l4, const void *l5, uint32_t nwb,
                                                        uint32_t kg, MatPtrs mp, const ActIn in) {
    const int N = (int)(nwb & 0xFFFFFu), W = (int)((nwb >> 20) & 0xFu), B = (int)(nwb >> 24);
    const int K = (int)(kg & 0xFFFFu), nwg = (int)(kg >> 16);
    const __half *__restrict__ x = static_cast<const __half *>(l0);   // plain: x; RN: a
    const __half *__restrict__ awq = static_cast<const __half *>(RN ? l3 : IMG ? nullptr : l1);
    const __half *__restrict__ xb = static_cast<const __half *>(l1);  // RN: b
    const __half *__restrict__ gam = static_cast<const __half *>(l2);  // RN: gamma
    const _Float16 *__restrict__ ihi = static_cast<const _Float16 *>(l0), *__restrict__ ilo =
        static_cast<const _Float16 *>(l1);   // IMG
    const __half *sc0 = static_cast<const __half *>(RN ? l4 : l2), *zr0 = static_cast<const __half *>(RN ? l5 : l3);
    const __half *sc1 = (NMAT == 2 && !RN) ? static_cast<const __half *>(l4) : mp.scales[1];
    const __half *zr1 = (NMAT == 2 && !RN) ? static_cast<const __half *>(l5) : mp.zeros[1];
    const uint8_t *wd0 = (NMAT == 1 && !RN) ? static_cast<const uint8_t *>(l4) : mp.data[0];
    const uint8_t *wd1 = mp.data[1];
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_b[];
    const int tid = threadIdx.x, nthr = 64 * NMAT * W;
    // the wave index as a scalar, so the weight pointer it selects is uniform
    // and the buffer resources stay in scalar registers
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), waves = nthr >> 6;
    const int mat = wave / W, part = wave - mat * W;
    const int G = K / kGS, P = G / 2;
    const int p0 = (part * P) / W;
    const int np = ((part + 1) * P) / W - p0;
    // (the host keeps N * NWG below 2^32)
    const int RB = (int)(((uint32_t)N * blockIdx.x) / (uint32_t)nwg);
    const int RE = (int)(((uint32_t)N * (blockIdx.x + 1)) / (uint32_t)nwg);
    const int RT = TM * 8;                     // band rows held in LDS (padded)
    // MB: the band [RB, RE) in blocks of RT rows, one after the other over the
    // operand image staged once (tall matrices at 3-8 rows); else one block
    const int nblk = MB ? (RE - RB + RT - 1) / RT : 1;
    int rb = RB;
    int nrows = MB ? min(RT, RE - RB) : RE - RB;

    const BandLds L = band_lds(G, BM, NMAT, TM, waves, RN);
    _Float16 *img = reinterpret_cast<_Float16 *>(lds_b + L.img);
    float *gsl = reinterpret_cast<float *>(lds_b + L.gs);
    uint32_t *szs = reinterpret_cast<uint32_t *>(lds_b + L.sz);
    float *rsq = reinterpret_cast<float *>(lds_b + L.rsq);
    float *rinv = rsq + G * BM;   // RN: rms_inv per batch row (the epilogue's copy)
    float4_t *red = reinterpret_cast<float4_t *>(lds_b + L.red);
    constexpr int NH = (BM + 3) / 4, BMH = BM < 4 ? BM : 4;   // MFMA passes, batch rows per pass

    // (a) activation chunks: chunk c = group c >> 4, elements (c & 15) * 8 ..
    // +7; 16 consecutive threads (one DPP row) hold one group
    // Loads that may have nothing to read go through buffer resources (an
    // out-of-range lane reads zeros and touches no memory): a branch around a
    // load makes the compiler wait for every load in flight where it joins.
    constexpr uint32_t kRsrcWord3 = 0x00020000u;
    const int nchunks = G * 16;
    const __amdgpu_buffer_rsrc_t awq_r =
        __builtin_amdgcn_make_buffer_rsrc((void *)awq, 0, awq ? K * 2 : 0, kRsrcWord3);
    u32x4_t xv[XC][BM], wv[XC];
    u32x4_t bv[RN ? XC : 1][BM], gv[RN ? XC : 1];   // RN: b rows and gamma
    u32x4_t lv[IMG ? XC : 1][BM];                    // IMG: the lo halves (xv: hi)
#pragma unroll
    for (int i = 0; i < XC; i++) {
        const int c = min(i * nthr + tid, nchunks - 1);
        const size_t e = (size_t)c * 8;
        if constexpr (IMG) {
#pragma unroll
            for (int b = 0; b < BM; b++) {
                const size_t o = (size_t)min(b, B - 1) * K + (size_t)img_chunk(c) * 8;
                xv[i][b] = *reinterpret_cast<const u32x4_t *>(ihi + o);
                lv[i][b] = *reinterpret_cast<const u32x4_t *>(ilo + o);
            }
            continue;
        }
#pragma unroll
        for (int b = 0; b < BM; b++) xv[i][b] = *reinterpret_cast<const u32x4_t *>(x + (size_t)min(b, B - 1) * K + e);
        if (RN) {
#pragma unroll
            for (int b = 0; b < BM; b++)
                bv[i][b] = *reinterpret_cast<const u32x4_t *>(xb + (size_t)min(b, B - 1) * K + e);
            gv[i] = *reinterpret_cast<const u32x4_t *>(gam + e);
        }
        wv[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(awq_r, (int)(e * 2), 0, 0));
    }
    // (b) scale / zero words of the block: word w of matrix m covers groups
    // 2p, 2p + 1 of block row w / P (the block's rows are contiguous)
    int szw = nrows * P;
    uint32_t sv[kSZC], zv[kSZC];
    auto load_sz = [&](int rb_, int szw_) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kSZC; i++) {
            const int w = min(i * nthr + tid, NMAT * szw_ - 1);
            const int m = (NMAT == 2 && w >= szw_) ? 1 : 0;
            const size_t src = (size_t)rb_ * P + (w - m * szw_);
            sv[i] = reinterpret_cast<const uint32_t *>(m ? sc1 : sc0)[src];
            zv[i] = reinterpret_cast<const uint32_t *>(m ? zr1 : zr0)[src];
        }
    };
    load_sz(rb, szw);
    // image output: the AWQ scale of the next projection at this thread's
    // first epilogue row, loaded with the small loads -- read in the
    // epilogue it put a memory round trip after the join (rows past the band,
    // and launches without an image output, read zeros)
    float img_w0 = 0.0f;
    if constexpr (EPI != EPI_STORE && !MB) {
        const bool iw = in.img_out_hi && in.img_awq;
        const __amdgpu_buffer_rsrc_t ia_r = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(reinterpret_cast<const char *>(in.img_awq) + (iw ? (size_t)RB * 2 : 0)), 0, iw ? nrows * 2 : 0,
            kRsrcWord3);
        img_w0 = __half2float(__builtin_bit_cast(
            __half, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(ia_r, (tid % RT) * 2, 0, 0)));
    }
    // issue order: every wave's small loads ahead of any weight load in the
    // CU's memory pipeline, which returns them in order (an execution barrier
    // only: nothing waits for the loads here)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // (c) weights: lane (j = lane & 15, kq = lane >> 4), row j & 7 of each
    // tile, group j >> 3 of each pair; rows past the band load nothing
    const int jr = lane & 7, jh = (lane >> 3) & 1, kq = lane >> 4;
    const uint8_t *wdata = (NMAT == 2 && mat) ? wd1 : wd0;
    // Issued pair by pair, tiles inner (the order the MFMAs consume them):
    // the first PD pairs now, each later one PD pairs ahead of its MFMAs, so
    // the MFMAs run while the rest streams in (a wave whose next load cannot
    // issue waits there, in order).
    const __amdgpu_buffer_rsrc_t w_r = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(wdata + (size_t)RB * (K / 2)), 0, (RE - RB) * (K / 2), kRsrcWord3);
    const int woff = jr * (K / 2) + jh * 64 + kq * 16;
    u32x4_t wq[TM][NP];
    // pair i of the block at row offset bo (from RB) into slot i
    // slots past the wave's own pairs: a plain one-matrix launch in 2-tile
    // bands of 5 pair slots (down) loads them past the resource's range
    // (zeros, no memory access) rather than re-reading its last pair -- down
    // B=1 6.56 -> 6.20 us.  Elsewhere the select on every load's offset cost
    // more than it saved (6144 x 2560 in 3-tile bands, no spare slot: 5.69 ->
    // 6.36 us; with two matrices, an image or residual-norm source or the
    // multi-block mode the decode step measured 1.608 -> 1.617 ms at B=1),
    // so those re-read.  The MFMAs skip the spare slots either way.
    constexpr int kPastRange = 0x40000000;
    auto load_pair_at = [&](int bo, int i) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TM; t++)
            wq[t][i] = __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                             w_r,
                             (NMAT == 1 && !IMG && !RN && !MB && TM == 2 && NP == 5) ? (i < np ? woff + (bo + t * 8) * (K / 2) + (p0 + i) * 128 : kPastRange)
                                       : woff + (bo + t * 8) * (K / 2) + (p0 + min(i, np - 1)) * 128,
                             0, 0));
    };
    auto load_pair = [&](int i) __attribute__((always_inline)) { load_pair_at(rb - RB, i); };
#pragma unroll
    for (int i = 0; i < PD && i < NP; i++) load_pair(i);

    // (d) scale/zero words -> LDS [mat][g][band row] (s | z << 16)
    auto sz_store = [&](int w, uint32_t s2, uint32_t z2) __attribute__((always_inline)) {
        const int m = (NMAT == 2 && w >= szw) ? 1 : 0;
        const int wl = w - m * szw;
        const int rr = wl / P, p = wl - rr * P;
        szs[(m * G + 2 * p) * RT + rr] = (s2 & 0xFFFFu) | (z2 << 16);
        szs[(m * G + 2 * p + 1) * RT + rr] = (s2 >> 16) | (z2 & 0xFFFF0000u);
    };
#pragma unroll
    for (int i = 0; i < kSZC; i++) sz_store(min(i * nthr + tid, NMAT * szw - 1), sv[i], zv[i]);   // host: all fit
    // (e) RN: r = a + b, per-group sums of r^2 -> LDS, then every thread's
    // rms_inv per batch row (groups j, j + 8, .. summed in order, then the
    // eight partial sums pairwise: row_rms's order)
    float ri[BM];
    const bool rnd = RN && in.round_mode == 1;
    if (RN) {
#pragma unroll
        for (int i = 0; i < XC; i++) {
            const int c = min(i * nthr + tid, nchunks - 1);
            const bool live = i * nthr + tid < nchunks;
#pragma unroll
            for (int b = 0; b < BM; b++) {
                const _Float16 *ah = reinterpret_cast<const _Float16 *>(&xv[i][b]);
                const _Float16 *bh = reinterpret_cast<const _Float16 *>(&bv[i][b]);
                float sq = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float r = (float)ah[e] + (float)bh[e];
                    sq = __builtin_fmaf(r, r, sq);
                }
                sq = row16_sum(sq);
                if (live && (c & 15) == 0) rsq[(c >> 4) * BM + b] = sq;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        // lane 8 b + j (j < 8) sums groups j, j + 8, .. of batch row b in
        // order, xor shuffles add the eight partial sums pairwise, and every
        // thread takes each row's sum from lane 8 b (one chain of G / 8 LDS
        // reads per lane: eight serial chains per thread took ~1.3 us)
        {
            const int rr = lane >> 3, j = lane & 7;
            float ss = 0.0f;
            if (rr < BM)
                for (int g = j; g < G; g += 8) ss += rsq[g * BM + rr];
            ss += __shfl_xor(ss, 1);
            ss += __shfl_xor(ss, 2);
            ss += __shfl_xor(ss, 4);
#pragma unroll
            for (int b = 0; b < BM; b++) ri[b] = 1.0f / __builtin_sqrtf(__shfl(ss, 8 * b) / (float)K + in.eps);
        }
        if (BM > 2 && tid < BM) {
            float r = ri[0];
#pragma unroll
            for (int b = 1; b < BM; b++) r = tid == b ? ri[b] : r;
            rinv[tid] = r;
        }
    }
    // (f) operand image -> LDS [g][plane][b][kRS], group sums [g][plane][b];
    // RN: workgroup 0 writes the residual and normed rows
#pragma unroll
    for (int i = 0; i < XC; i++) {
        const int c = min(i * nthr + tid, nchunks - 1);
        const bool live = i * nthr + tid < nchunks;   // uniform over the 16-thread row
        const int g = c >> 4;
        const _Float16 *wh = reinterpret_cast<const _Float16 *>(&wv[i]);
#pragma unroll
        for (int b = 0; b < BM; b++) {
            const _Float16 *xh = reinterpret_cast<const _Float16 *>(&xv[i][b]);
            half8_t hi, lo;
            float sh, sl;
            if constexpr (IMG) {
                hi = __builtin_bit_cast(half8_t, xv[i][b]);
                lo = __builtin_bit_cast(half8_t, lv[i][b]);
                chunk_sums(hi, lo, sh, sl);
            } else {
            float v[8];
            if (RN) {
                const _Float16 *bh = reinterpret_cast<const _Float16 *>(&bv[i][b]);
                const _Float16 *gh = reinterpret_cast<const _Float16 *>(&gv[i]);
                half8_t res, nrm;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float r = (float)xh[e] + (float)bh[e];
                    res[e] = (_Float16)r;
                    nrm[e] = (_Float16)(r * ri[b] * (float)gh[e]);
                    v[e] = rnd ? (float)nrm[e] : r * (float)gh[e];
                }
                if (blockIdx.x == 0 && live && b < B) {
                    const size_t off = (size_t)b * K + (size_t)c * 8;
                    *reinterpret_cast<half8_t *>(in.residual_out + off) = res;
                    *reinterpret_cast<half8_t *>(in.normed_out + off) = nrm;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = (float)xh[e];
            }
            if (awq) {
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = div_awq(v[e], (float)wh[e]);
            }
            chunk_operands(v, hi, lo, sh, sl);
            }
            _Float16 *dst = img + ((size_t)(g * 2) * BM + b) * kRS + (c & 15) * 8;
            if (live) {
                *reinterpret_cast<half8_t *>(dst) = hi;
                *reinterpret_cast<half8_t *>(dst + BM * kRS) = lo;
            }
            sh = row16_sum(sh);
            sl = row16_sum(sl);
            if (live && (c & 15) == 0) {
                gsl[(g * 2) * BM + b] = sh * kTwoM24;
                gsl[(g * 2 + 1) * BM + b] = sl * kTwoM24;
            }
        }
    }
    // LDS-only barrier: the weight loads stay in flight across it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

    // (g) MFMA.  A row of this lane: i = lane & 15 -> (ah, aplane, ab); the
    // lane's result rows: (h, plane) = (lane >> 5, (lane >> 4) & 1).  Above 4
    // batch rows the MFMAs run in passes of 4 (pass ph: batch rows 4 ph ..),
    // each weight operand used by every pass.
    const int ai = lane & 15;
    const int ah = ai >> 3, aplane = (ai >> 2) & 1, ab = ai & 3;
    const bool a_live = ab < BMH;
    const int dplane = (lane >> 4) & 1;
    for (int blk = 0; blk < nblk; blk++) {
    if (MB && blk > 0) {
        // the previous block's MFMAs are done with szs and its epilogue with
        // red (the barrier before that epilogue, and this one): this block's
        // scale / zero words in
#pragma unroll
        for (int i = 0; i < kSZC; i++) sz_store(min(i * nthr + tid, NMAT * szw - 1), sv[i], zv[i]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    const int ntile = (nrows + 7) >> 3;
    float acc[TM][BM];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int b = 0; b < BM; b++) acc[t][b] = 0.0f;
#pragma unroll
    for (int i = 0; i < NP; i++) {
        if (i + PD < NP) load_pair(i + PD);
        if (i < np) {
            const int g = 2 * (p0 + i) + jh;             // this lane's column group
            const int ga = 2 * (p0 + i) + ah;            // this lane's A-row group
            half8_t av[NH][4];
#pragma unroll
            for (int ph = 0; ph < NH; ph++) {
                const _Float16 *xa =
                    img + ((size_t)(ga * 2 + aplane) * BM + min(4 * ph + ab, BM - 1)) * kRS + kq * 32;
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    av[ph][m] = *reinterpret_cast<const half8_t *>(xa + m * 8);
                    if (!a_live) av[ph][m] = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
                }
            }
            const float *gp = gsl + (g * 2 + dplane) * BM;
            float gsv[BM];
#pragma unroll
            for (int b = 0; b < BM; b++) gsv[b] = gp[b];
#pragma unroll
            for (int t = 0; t < TM; t++) {
                if (t < ntile) {
                    const uint32_t sz = szs[(mat * G + g) * RT + t * 8 + jr];
                    const float s24 = (float)__builtin_bit_cast(_Float16, (uint16_t)(sz & 0xFFFFu)) * kTwo24;
                    const float z = (float)__builtin_bit_cast(_Float16, (uint16_t)(sz >> 16));
                    u32x4_t bq[4];
#pragma unroll
                    for (int m = 0; m < 4; m++) {
                        const uint32_t w = wq[t][i][m];
                        const uint32_t q0 = __builtin_amdgcn_perm(w, 0u, 0x0C050C04u);  // b0, b1
                        const uint32_t q1 = __builtin_amdgcn_perm(w, 0u, 0x0C070C06u);  // b2, b3
                        bq[m] = (u32x4_t){q0, q1, q0 & 0x00F000F0u, q1 & 0x00F000F0u};
                    }
#pragma unroll
                    for (int ph = 0; ph < NH; ph++) {
                        float4_t accg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int m = 0; m < 4; m++)
                            accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[ph][m], __builtin_bit_cast(half8_t, bq[m]),
                                                                          accg, 0, 0, 0);
#pragma unroll
                        for (int b = 0; b < BMH; b++)
                            acc[t][4 * ph + b] =
                                __builtin_fmaf(s24, __builtin_fmaf(-z, gsv[4 * ph + b], accg[b]), acc[t][4 * ph + b]);
                    }
                }
            }
        }
        if constexpr (MB) {
            // the next block's first pairs into the slots this one is done
            // with, and its scale / zero words into registers
            if (blk + 1 < nblk && i + PD >= NP) load_pair_at(rb + RT - RB, i + PD - NP);
            if (blk + 1 < nblk && i == 0) load_sz(rb + RT, min(RT, RE - rb - RT) * P);
        }
    }
    // (h) rows r = lane & 7 of each tile sit at lanes r (h 0, hi), r + 16
    // (h 0, lo), r + 40 (h 1, hi), r + 56 (h 1, lo)
#pragma unroll
    for (int t = 0; t < TM; t++) {
#pragma unroll
        for (int ph = 0; ph < NH; ph++) {
            float4_t v = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int b = 0; b < BMH; b++) {
                float a = acc[t][4 * ph + b];
                a += __shfl_down(a, 16);
                a += __shfl_down(a, 40);
                v[b] = a;
            }
            if (lane < 8) red[((wave * TM + t) * NH + ph) * 8 + lane] = v;
        }
    }
    __syncthreads();
    // the row's sums over the waves' parts (in part order), per matrix: the
    // W <= 8 / NMAT reads issued together, then added in order (a loop to
    // the runtime W waited for each read in turn)
    auto row_sums = [&](int r, int b, float *sum) __attribute__((always_inline)) {
        const int t = r >> 3, rl = r & 7;
        constexpr int WM = 8 / NMAT;   // the host keeps W <= 8 / NMAT
        // part 0 of matrix 0 for this (row, batch row); parts TM * NH * 8
        // float4s apart (a uniform offset per part)
        const float *r0 = reinterpret_cast<const float *>(red + (t * NH + (b >> 2)) * 8 + rl) + (b & 3);
        constexpr int pst = TM * NH * 8 * 4;
        // W <= 4: the reads of 2 or 4 parts (clamped to the last) issued
        // together, then added in order; W > 4 (down: 8) the loop, which the
        // compiler unrolls by 8 with one wait (left as a loop to the runtime
        // W, W <= 4 waited for each read in turn)
        auto parts_sum = [&](int mt, auto n) __attribute__((always_inline)) {
            constexpr int PN = decltype(n)::value;
            const float *rm = r0 + mt * W * pst;
            float pv[PN];
#pragma unroll
            for (int p = 0; p < PN; p++) pv[p] = rm[min(p, W - 1) * pst];
            float s = 0.0f;
#pragma unroll
            for (int p = 0; p < PN; p++)
                if (p < W) s += pv[p];
            return s;
        };
#pragma unroll
        for (int mt = 0; mt < NMAT; mt++) {
            float s = 0.0f;
            if (W <= 2) {
                s = parts_sum(mt, std::integral_constant<int, 2>{});
            } else if (WM <= 4 || W <= 4) {
                s = parts_sum(mt, std::integral_constant<int, WM < 4 ? WM : 4>{});
            } else {
                for (int p = 0; p < W; p++) s += r0[(mt * W + p) * pst];
            }
            // round_mode 0: the row's rms_inv scales both projections, ahead of the activation
            sum[mt] = (RN && !rnd) ? s * (BM <= 2 ? (b == 0 ? ri[0] : ri[BM - 1]) : rinv[b]) : s;
        }
    };
    if constexpr (EPI == EPI_SILU || EPI == EPI_GELU) {
        // with img_out the row pair (r, r + 1) is also the element pair
        // (v[2i], v[2i + 1]) of the next projection's operand image: the two
        // rows sit in adjacent lanes (the host guarantees even band starts and
        // lengths), so the even lane takes its neighbour's value by a shuffle
        for (int o0 = 0; o0 < RT * BM; o0 += nthr) {
            const int o = o0 + tid;
            const int r = o % RT, b = o / RT;
            const bool live = o < RT * BM && r < nrows && b < B;
            float v = 0.0f;
            if (live) {
                float sum[NMAT];
                row_sums(r, b, sum);
                const float g = sum[0], u = sum[NMAT - 1];
                float act;
                if (EPI == EPI_SILU) {
                    act = g / (1.0f + __expf(-g));
                } else {
                    float inner = 0.7978845608f * (g + 0.044715f * g * g * g);
                    inner = fminf(fmaxf(inner, -10.0f), 10.0f);
                    act = 0.5f * g * (1.0f + tanhf(inner));
                }
                const __half h = __float2half(act * u);
                mp.out[0][(size_t)b * N + rb + r] = h;
                v = __half2float(h);
                if (in.img_out_hi && in.img_awq)
                    v = div_awq(v, o0 == 0 ? img_w0 : __half2float(in.img_awq[rb + r]));
            }
            if (in.img_out_hi) {   // uniform
                const float v1 = __shfl_xor(v, 1);
                if (live && (r & 1) == 0) {
                    const int k = rb + r;
                    _Float16 ah, al, ch, cl;
                    pair_operands(v, v1, ah, al, ch, cl);
                    const size_t base = (size_t)b * N + (size_t)img_chunk(k >> 3) * 8;
                    const int i = (k & 7) >> 1;
                    in.img_out_hi[base + i] = ah;
                    in.img_out_hi[base + 4 + i] = ch;
                    in.img_out_lo[base + i] = al;
                    in.img_out_lo[base + 4 + i] = cl;
                }
            }
        }
    } else {
        for (int o = tid; o < RT * BM; o += nthr) {
            const int r = o % RT, b = o / RT;
            if (r >= nrows || b >= B) continue;
            float sum[NMAT];
            row_sums(r, b, sum);
#pragma unroll
            for (int mt = 0; mt < NMAT; mt++) mp.out[mt][(size_t)b * N + rb + r] = __float2half(sum[mt]);
        }
    }
    if constexpr (MB) {
        rb += RT;
        nrows = min(RT, RE - rb);
        szw = nrows * P;
    }
    }   // blocks
}

struct BandLaunch {
    dim3 grid, block;
    size_t lds;
    hipStream_t st;
    BandLead a;
    bool dry;   // only check that the instantiation accepts its LDS size
};
#define IMH_BAND_ARGS(L) \
    L.a.p[0], L.a.p[1], L.a.p[2], L.a.p[3], L.a.p[4], L.a.p[5], L.a.nwb, L.a.kg

// Above 64 KB of LDS a kernel must be allowed the larger size first (gfx950
// has 160 KB per CU); false if the runtime refuses.
template <typename F>
bool allow_lds(F kernel, size_t lds) {
    if (lds <= 64 * 1024 || hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess)
        return true;
    (void)hipGetLastError();   // the refusal is not an error of the op: a fallback runs it
    return false;
}

template <int NMAT, int EPI, int TM, int NP, int BM, bool RN, bool IMG>
bool launch_xc(int xc, const BandLaunch &L, const MatPtrs &mp, const ActIn &in) {
    if (xc == 1) {
        if (!allow_lds(int4_band_kernel<NMAT, EPI, TM, NP, BM, 1, RN, IMG>, L.lds)) return false;
        if (!L.dry)
            hipLaunchKernelGGL((int4_band_kernel<NMAT, EPI, TM, NP, BM, 1, RN, IMG>), L.grid, L.block, L.lds, L.st,
                               IMH_BAND_ARGS(L), mp, in);
    } else if (BM <= 2) {   // three activation chunks per thread: 1-2 batch rows only
        if (!allow_lds(int4_band_kernel<NMAT, EPI, TM, NP, BM, BM <= 2 ? 3 : 1, RN, IMG>, L.lds)) return false;
        if (!L.dry)
            hipLaunchKernelGGL((int4_band_kernel<NMAT, EPI, TM, NP, BM, BM <= 2 ? 3 : 1, RN, IMG>), L.grid, L.block,
                               L.lds, L.st, IMH_BAND_ARGS(L), mp, in);
    }
    return true;
}

// batch rows per instantiation: 1, 2, 4 (3-4 rows) and 8 (5-8 rows; plain
// sources only); an image source at 1-2 rows
template <int NMAT, int EPI, int TM, int NP, bool RN, bool IMG>
bool launch_bm(int bm, int xc, const BandLaunch &L, const MatPtrs &mp, const ActIn &in) {
    if (bm == 1) return launch_xc<NMAT, EPI, TM, NP, 1, RN, IMG>(xc, L, mp, in);
    if (bm == 2) return launch_xc<NMAT, EPI, TM, NP, 2, RN, IMG>(xc, L, mp, in);
    if constexpr (!RN && !IMG) {
        if (bm == 4) return launch_xc<NMAT, EPI, TM, NP, 4, RN, IMG>(xc, L, mp, in);
        return launch_xc<NMAT, EPI, TM, NP, 8, RN, IMG>(xc, L, mp, in);
    }
    return false;
}

// Tall matrices at 3-8 rows: 5-tile blocks, two pairs per wave, both issued
// ahead (and the next block's two while the last ones compute).
template <int BM>
bool launch_mb(const BandLaunch &L, const MatPtrs &mp, const ActIn &in) {
    if (!allow_lds(int4_band_kernel<1, EPI_STORE, 5, 2, BM, 1, false, false, 2, true>, L.lds)) return false;
    if (!L.dry)
        hipLaunchKernelGGL((int4_band_kernel<1, EPI_STORE, 5, 2, BM, 1, false, false, 2, true>), L.grid, L.block,
                           L.lds, L.st, IMH_BAND_ARGS(L), mp, in);
    return true;
}

// (TM, NP) instantiated: (2, 2), (2, 5), (3, 5) and (5, 3); the host picks
// the smallest TM that holds the band, and (2, 2) when its waves hold at most
// two pairs (O and K/V-sized matrices on eight waves): a wave loads a slot for
// every NP, re-reading its last pair for the slots past its own -- with (2, 5)
// three of O's five loads per tile were such re-reads (O B=1 4.77 -> 4.18 us).
template <int NMAT, int EPI, bool RN, bool IMG = false>
bool launch_shape(int tm, int bm, int xc, const BandLaunch &L, const MatPtrs &mp, const ActIn &in, int np = 5) {
    if (tm <= 2 && np <= 2) return launch_bm<NMAT, EPI, 2, 2, RN, IMG>(bm, xc, L, mp, in);
    if (tm <= 2) return launch_bm<NMAT, EPI, 2, 5, RN, IMG>(bm, xc, L, mp, in);
    if (tm <= 3) return launch_bm<NMAT, EPI, 3, 5, RN, IMG>(bm, xc, L, mp, in);
    return launch_bm<NMAT, EPI, 5, 3, RN, IMG>(bm, xc, L, mp, in);
}

}  // namespace

// Launches the band kernel when it applies (B <= 8, no row segments, an even
// number of groups, the shape within the instantiated tiles and the LDS
// budget -- 64 KB for 1-2 batch rows, 160 KB with one activation chunk per
// thread above; an operand image source (in.img_src, 1-2 batch rows) or
// output (in.img_out_hi, every band on even rows); a
// residual-norm source only at 1-2 batch rows, with
// round_mode 0 or 1, as nmat 1 with EPI_STORE or nmat 2 with an activation);
// *used reports whether it did.  probe: only whether it would apply (nothing
// is launched; the LDS size is checked with the runtime as for a launch).
int launch_band_matvec(hipStream_t st, int cus, int B, int nmat, int epi, int N, int K, const MatPtrs &mp,
                       const ActIn &in, bool *used, bool probe) {
    *used = false;
    const bool rn = in.b != nullptr;
    const int G = K / kGS;
    if (B < 1 || B > 8 || mp.seg[0] != 0 || G % 2 || G < 2) return IMH_OK;
    const int bm = B <= 2 ? B : B <= 4 ? 4 : 8;
    // an image source: one matrix, no norm, 1-2 rows; an image output: a
    // gate/up pair with an activation
    if (in.img_src && (rn || nmat != 1 || epi != EPI_STORE || bm > 2 || !in.hi || !in.lo)) return IMH_OK;
    if (in.img_out_hi && (nmat != 2 || epi == EPI_STORE || !in.img_out_lo)) return IMH_OK;
    // above two rows every workgroup would redo the whole residual + norm of
    // every row (measured slower than the rows kernel + the plain band)
    if (bm > 2 && rn) return IMH_OK;
    if (rn && (in.round_mode > 1 || (nmat == 2) != (epi != EPI_STORE))) return IMH_OK;
    for (int i = 0; i < nmat; i++)
        if ((reinterpret_cast<uintptr_t>(mp.scales[i]) | reinterpret_cast<uintptr_t>(mp.zeros[i])) & 3) return IMH_OK;
    const int P = G / 2;
    const int ntiles = (N + 7) / 8;
    // workgroups: one band per CU, more (bands of up to 5 tiles) for tall
    // matrices -- except at 3-8 rows (one plain-source matrix), where every
    // workgroup would stage the operand image of all of K for 40 rows: there
    // one band per CU, walked in blocks of 5 tiles over one staging (mb)
    const bool mb = bm > 2 && !rn && !in.img_src && nmat == 1 && epi == EPI_STORE && (ntiles + 4) / 5 > cus;
    // tall matrices at 1-2 rows (the LM head): bands of 3 tiles, two waves of
    // five pairs each -- 37.5 against 38.4 us with 5-tile bands of four waves
    // (151936 x 2560 at one row, A/B on one box)
    const bool tall12 = bm <= 2 && nmat == 1 && (ntiles + 4) / 5 > cus;
    const int nwg = mb ? cus : std::min(std::max(cus, tall12 ? (ntiles + 2) / 3 : (ntiles + 4) / 5), N);
    if ((uint64_t)N * nwg >= (1ull << 32)) return IMH_OK;
    const int rows = mb ? 40 : (N + nwg - 1) / nwg;   // mb: rows per block
    const int tm = (rows + 7) / 8;
    if (tm > 5) return IMH_OK;
    if (in.img_out_hi) {
        // the epilogue writes element pairs: every band must start on an even row
        // and hold an even number of rows
        for (int b = 0; b <= nwg; b++)
            if ((int)(((uint32_t)N * (uint32_t)b) / (uint32_t)nwg) % 2) return IMH_OK;
    }
    const int TM = tm <= 2 ? 2 : tm <= 3 ? 3 : 5, NPmax = mb ? 2 : tm <= 3 ? 5 : 3;
    // waves per matrix: as few as keep each wave within NPmax pairs (1-2
    // rows); all eight above, so one activation chunk per thread covers K
    // at 1-2 rows, 2-tile bands one per CU (O, K/V-sized and the down
    // projection): all eight waves, fewer pairs each -- O (2560 x 4096) B=1
    // 5.19 -> 4.77 us with 8 waves of 2 pairs instead of 4 of 4; 3-tile
    // bands (6144 x 2560) measured slower that way and keep the fewest waves
    int W = bm > 2 ? std::min(8 / nmat, P) : std::min((P + NPmax - 1) / NPmax, 8 / nmat);
    if (bm <= 2 && !tall12 && nwg <= cus && TM == 2) W = std::min(8 / nmat, P);
    // multi-block (3-8 rows, tall): the fewest waves that keep eight waves'
    // pair count, so every wave holds the same -- the LM head's 10 pairs on
    // five waves of two, not eight of one or two (B=4 / 8 68.8 / 94.2 ->
    // 63.2 / 84.7 us)
    if (mb) {
        const int npw = (P + 7) / 8;
        W = (P + npw - 1) / npw;
    }
    const int np = (P + W - 1) / W;
    if (np > NPmax) return IMH_OK;
    const int nthr = 64 * W * nmat;
    const int xc = (G * 16 + nthr - 1) / nthr;
    if (xc > 3 || (bm > 2 && xc > 1) || nmat * rows * P > kSZC * nthr) return IMH_OK;
    const size_t lds = band_lds(G, bm, nmat, TM, W * nmat, rn).total;
    if (lds > (bm <= 2 ? 64 : 160) * 1024) return IMH_OK;
    // a probe takes the same dispatch with launches off: the instantiation
    // must still accept its LDS size (hipFuncSetAttribute above 64 KB)
    // the leading arguments (see int4_band_kernel) and the packed dimensions
    if (N >= (1 << 20) || K >= (1 << 16) || nwg >= (1 << 16) || W >= 16 || B >= 16) return IMH_OK;
    BandLead a{};
    if (in.img_src) {
        a = BandLead{{in.hi, in.lo, mp.scales[0], mp.zeros[0], mp.data[0], nullptr}, 0, 0};
    } else if (rn) {
        a = BandLead{{in.a, in.b, in.gamma, in.awq, mp.scales[0], mp.zeros[0]}, 0, 0};
    } else {
        a = BandLead{{in.a, in.awq, mp.scales[0], mp.zeros[0], nmat == 2 ? (const void *)mp.scales[1] : mp.data[0],
                      nmat == 2 ? (const void *)mp.zeros[1] : nullptr},
                     0, 0};
    }
    a.nwb = (uint32_t)N | ((uint32_t)W << 20) | ((uint32_t)B << 24);
    a.kg = (uint32_t)K | ((uint32_t)nwg << 16);
    BandLaunch L{dim3(nwg), dim3(nthr), lds, st, a, probe};
    bool ok;
    if (mb) {
        ok = bm == 4 ? launch_mb<4>(L, mp, in) : launch_mb<8>(L, mp, in);
    } else if (in.img_src) {
        ok = launch_shape<1, EPI_STORE, false, true>(tm, bm, xc, L, mp, in, np);
    } else if (rn) {
        if (nmat == 1)
            ok = launch_shape<1, EPI_STORE, true>(tm, bm, xc, L, mp, in, np);
        else if (epi == EPI_SILU)
            ok = launch_shape<2, EPI_SILU, true>(tm, bm, xc, L, mp, in);
        else
            ok = launch_shape<2, EPI_GELU, true>(tm, bm, xc, L, mp, in);
    } else if (nmat == 1) {
        ok = launch_shape<1, EPI_STORE, false>(tm, bm, xc, L, mp, in, np);
    } else if (epi == EPI_SILU) {
        ok = launch_shape<2, EPI_SILU, false>(tm, bm, xc, L, mp, in);
    } else if (epi == EPI_GELU) {
        ok = launch_shape<2, EPI_GELU, false>(tm, bm, xc, L, mp, in);
    } else {
        ok = launch_shape<2, EPI_STORE, false>(tm, bm, xc, L, mp, in);
    }
    if (!ok) return IMH_OK;   // the LDS size was refused: the tile kernel runs the op
    if (!probe) IMH_HIP(hipGetLastError());
    *used = true;
    return IMH_OK;
}

}  // namespace imh_int4
