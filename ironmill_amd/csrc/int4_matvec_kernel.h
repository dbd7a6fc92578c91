// int4_matvec_kernel.h -- the INT4-affine (group 128) matvec kernel for gfx950,
// shared by the translation units that instantiate it (int4_matvec.hip: image
// sources, one MFMA tile; int4_matvec_mt2.hip: image sources, two tiles;
// int4_matvec_raw.hip: raw sources).
//
// Semantics (dequantize-then-compute, core/dequant.rs:85-180 + the f32 dot of
// the reference kernels, affine_batched.metal:51-90):
//     y[m][r] = sum_k xe[m][k] * (q[r][k] - z[r][g]) * s[r][g],  g = k / 128
// where xe = x / awq (affine_batched.metal:70-79) or, for the fused residual
// norm, xe = (a + b) * gamma / awq and the epilogue multiplies by rms_inv
// (superblock_fused_norm.metal:37-124).
//
// MI355X design:
//  * the contraction runs on the matrix cores (v_mfma_f32_16x16x32_f16), with
//    each group split as
//        y_g = s * (sum_k xe_k q_k - z * sum_k xe_k)
//    so the raw codes enter the MFMA with no per-element zero-point work.  A
//    code byte in the low byte of an f16 whose high byte is zero is the f16
//    denormal byte * 2^-24, exactly, and the matrix cores multiply f16
//    denormals at full precision.  For the 8 codes n0..n7 of one weight dword
//    (byte i = n_2i + 16 n_2i+1) two v_perm_b32 spread the bytes into f16 lanes
//    and two masks keep 16 n_2i+1, giving the B operand
//        {b0, b1, b2, b3, 16 n1, 16 n3, 16 n5, 16 n7} * 2^-24;
//    the activation operand
//        {x0, x2, x4, x6, x1/16 - x0, x3/16 - x2, x5/16 - x4, x7/16 - x6}
//    makes the products sum to x0 n0 + x1 n1 + ... + x7 n7: 4 VALU per 8
//    weights, every product exact, f32 accumulation.
//  * the activation operand values are split into f16 hi + lo halves
//    (~22-bit operands).  In an MFMA tile, A rows 0-7 carry the hi halves of 8
//    batch rows and rows 8-15 their lo halves: one MFMA covers both, and the
//    two halves of a row are added at the end.
//  * the zero point multiplies the per-group sums of the operand values (hi
//    and lo apart, prescaled by 2^-24): two FMAs per output per group.
//  * the operand image (values + group sums) comes from one of two sources:
//    IMAGE -- built by a small prep kernel into memory, then staged into LDS;
//    RAW -- built by every workgroup for its batch rows straight into LDS from
//    x / awq (RAW_RN: from a + b, gamma and awq, with the RMS reduction in the
//    same pass).  RAW saves a launch and is used when the image is small
//    (one or two 8-element chunks per thread); its few VALU overlap the weight
//    loads already in flight.
//  * one workgroup owns one 16-row tile (of each matrix of a gate/up pair);
//    its waves split K, each holding its slice's weights in registers (one
//    16-byte load per lane per group, issued up front), and reduce through
//    LDS in a fixed order: deterministic, no cross-workgroup synchronisation.
//  * activation and scale/zero loads are issued before the weight loads and
//    an LDS-only barrier follows the staging, so the weights stay in flight
//    while the first groups compute.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>

#include "dpp_reduce.h"

namespace imh_int4 {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGS = 128;         // group size the kernels are built for
constexpr int kMaxGroups = 8;    // groups one wave holds per stage (weights stay in registers)
constexpr int kMaxWaves = 16;    // waves per workgroup
constexpr int kSZChunks = 2;     // scale/zero elements per thread loaded ahead of the weights
constexpr int kSXChunks = 2;     // image group sums per thread loaded ahead of the weights
constexpr int kLdsBudget = 64 * 1024;
constexpr float kTwoM24 = 5.9604644775390625e-08f;  // 2^-24
constexpr float kTwo24 = 16777216.0f;               // 2^24

enum Epi : int { EPI_STORE, EPI_SILU, EPI_GELU };
enum Src : int { SRC_IMAGE, SRC_RAW, SRC_RAW_RN };

// Weights and outputs.  NMAT 2: entries 0 and 1 are the pair.  NMAT 1: entry
// 0, or up to three row segments of one launch: the tiles from row seg[0] on
// (seg[1] on) belong to entry 1 (entry 2), rows counted from the segment's
// first row; seg[i] == 0 means no such segment.  Segment starts are multiples
// of 16, so a tile never spans two segments.
struct MatPtrs {
    const uint8_t *data[3];
    const __half *scales[3];
    const __half *zeros[3];
    __half *out[3];
    int seg[2];
};

// Activation source.  IMAGE: hi/lo [B][K] f16 operand values, gsum [B][2][G]
// f32 group sums (prescaled), row_scale [B] or NULL.  RAW: a = x [B][K] and
// awq [K] or NULL.  RAW_RN: r = a + b, operand r * gamma / awq, output scaled
// by rms_inv = 1 / sqrt(mean(r^2) + eps) (round_mode below); the workgroups
// of tile column 0 also write residual_out = f16(r) and normed_out =
// f16(r * rms_inv * gamma).
struct ActIn {
    const _Float16 *hi;
    const _Float16 *lo;
    const float *gsum;
    const float *row_scale;
    const __half *a;
    const __half *b;
    const __half *gamma;
    const __half *awq;
    __half *residual_out;
    __half *normed_out;
    float eps;
    // residual-norm operand: 0 -- r * gamma / awq with rms_inv applied to the
    // output (the fused residual-norm projection); 1 -- the f16-rounded
    // normed row f16(r * rms_inv * gamma) / awq, as a separate RMSNorm feeding
    // the projection would give; 2 -- 0 for the first row segment, 1 for the
    // rest (IMAGE: the second image hi2 / lo2 / gsum2, with no row scale)
    int round_mode;
    const _Float16 *hi2;
    const _Float16 *lo2;
    const float *gsum2;
    // Row-band kernel only.  img_out_hi / img_out_lo (gate/up pair with an
    // activation): also write the activation, divided by img_awq (NULL: not
    // divided), as the operand image [B][N] of the projection that reads it
    // (the down projection of an FFN block).  img_src: hi / lo hold such an
    // image and gsum is NULL -- the kernel sums the groups itself.
    _Float16 *img_out_hi;
    _Float16 *img_out_lo;
    const __half *img_awq;
    int img_src;
};

// Operand images in memory (hi / lo planes [B][K]) hold each group's sixteen
// 8-element chunks as a transposed 4 x 4 block: chunk 4a + b of a group sits
// at position 4b + a (the map is its own inverse).  The direct-operand kernel's
// 16-byte load j of lane quarter kq then reads chunk 4kq + j -- the chunk its
// MFMA slot takes -- and the four quarters of a row read 64 contiguous bytes
// per load; every other reader and writer maps chunk indices through this.
// c: the chunk index along K (element k is in chunk k / 8).
__host__ __device__ __forceinline__ int img_chunk(int c) { return (c & ~15) | ((c & 3) << 2) | ((c >> 2) & 3); }

// Split v into f16 hi + lo with hi + lo == v to ~22 bits.
__device__ __forceinline__ void split_hilo(float v, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// Operand image of one 8-element chunk v[0..7] of xe (natural order): slots
// {v0, v2, v4, v6, v1/16 - v0, v3/16 - v2, v5/16 - v4, v7/16 - v6}, split into
// hi/lo halves.  sh / sl get the chunk's share of the group sums: the codes
// q == z everywhere give sum_i a_i (z + 16 z) + c_i (16 z), so the sum that the
// zero point multiplies is sum_i 17 a_i + 16 c_i, per half.
// Elements (v0, v1) = (v[2i], v[2i + 1]) -> slots i (a) and 4 + i (c).
__device__ __forceinline__ void pair_operands(float v0, float v1, _Float16 &ah, _Float16 &al, _Float16 &ch,
                                              _Float16 &cl) {
    const float c = v1 * 0.0625f - v0;
    split_hilo(v0, ah, al);
    split_hilo(c, ch, cl);
}

// The chunk's share of the group sums, from its operand halves (one order
// for every kernel that forms them: the image writers and the kernels that
// read an image without sums).
__device__ __forceinline__ void chunk_sums(const half8_t &hi, const half8_t &lo, float &sh, float &sl) {
    sh = 0.0f;
    sl = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        sh = sh + __builtin_fmaf(17.0f, (float)hi[i], 16.0f * (float)hi[4 + i]);
        sl = sl + __builtin_fmaf(17.0f, (float)lo[i], 16.0f * (float)lo[4 + i]);
    }
}

__device__ __forceinline__ void chunk_operands(const float v[8], half8_t &hi, half8_t &lo, float &sh,
                                               float &sl) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        _Float16 ah, al, ch, cl;
        pair_operands(v[2 * i], v[2 * i + 1], ah, al, ch, cl);
        hi[i] = ah;
        lo[i] = al;
        hi[4 + i] = ch;
        lo[4 + i] = cl;
    }
    chunk_sums(hi, lo, sh, sl);
}

using imh_dpp::row16_sum;

// v / w to within ~2 ulp (hardware reciprocal, then a multiply); the operand
// keeps ~22 bits, so the difference from a correctly rounded quotient is far
// below the hi/lo resolution.
__device__ __forceinline__ float div_awq(float v, float w) { return v * __builtin_amdgcn_rcpf(w); }

// ---------------------------------------------------------------------------
// main matvec kernel
// ---------------------------------------------------------------------------
// grid (ceil(N/16), ceil(B/16)), block 64 * NMAT * parts.  The workgroup's
// batch rows (up to 16) form MT MFMA tiles of 8 rows.  Wave w works on matrix
// w / parts and, in every K stage, on part w % parts of the stage's groups (at
// most NG of them).  A stage is the range of groups whose activation image
// fits the LDS budget (normally all of K: one stage; RAW sources always use
// one).  Up to XC activation chunks (8 elements of one batch row) per thread
// are loaded ahead of the weights (IMAGE: the rest, if any, after them; RAW:
// the host guarantees there is no rest).
//
// Issue order matters: vector-memory loads of a wave complete in order, so
// the small loads the LDS staging needs are issued first and the weight loads
// right after them, before anything waits.  The first stage is peeled so no
// loop-carried wait sits ahead of the first weight loads.
// Occupancy target (waves per SIMD) the register allocator works to: 6 where
// the live state fits 80 VGPRs without spilling, fewer for the heavier shapes.
// The decode step's instantiations (NG 2) compile without scratch; some raw
// shapes with NG >= 4 spill 12-28 bytes per lane at these targets.
constexpr int waves_per_simd(int NG, int MT, int XC, int SRC) {
    return ((SRC == SRC_RAW_RN && XC == 2) || (NG >= 8 && XC == 2)) ? 4
           : (NG <= 5 && (MT == 1 || XC == 1) && (SRC == SRC_IMAGE || (XC == 1 && SRC == SRC_RAW))) ? 6
                                                                                                   : 5;
}

template <int NMAT, int EPI, int MT, int NG, int XC, int SRC>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(waves_per_simd(NG, MT, XC, SRC))))
int4_matvec_kernel(MatPtrs mp, ActIn in, int Nall, int K, int B, int parts, int SG) {
    constexpr bool RAW = SRC != SRC_IMAGE;
    constexpr bool RN = SRC == SRC_RAW_RN;
    // dynamic LDS: [NMAT][G][16] u32 (scale | zero << 16); [G][MT][16] f32
    // group sums per A row; RN: [G][16] f32 sums of r^2 and [16] rms_inv;
    // then one region holding the activation planes ([2][bc][SG*128 + 8] f16:
    // hi rows, then lo rows) during the stages and the [MT][waves][64] float4
    // partial sums after them
    extern __shared__ __attribute__((aligned(16))) uint32_t lds_dyn[];

    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int waves = nthr >> 6;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int mat = wave / parts;
    const int part = wave - mat * parts;
    const int G = K / kGS;
    const int m0 = blockIdx.y * 16;
    const int bc = min(16, B - m0);
    const int RSX = SG * kGS + 8;        // LDS row stride in halfs (16-byte pad)

    // matrix pointers by select: a dynamic index into the kernel-argument
    // struct would turn into dependent memory loads
    int row0 = blockIdx.x * 16;
    int N = Nall;
    const uint8_t *d0 = mp.data[0], *d1 = mp.data[1];
    const __half *sc0 = mp.scales[0], *sc1 = mp.scales[1];
    const __half *zr0 = mp.zeros[0], *zr1 = mp.zeros[1];
    __half *o0 = mp.out[0], *o1 = mp.out[1];
    int seg_idx = 0;
    if (NMAT == 1 && mp.seg[0] > 0 && row0 < mp.seg[0]) {
        N = mp.seg[0];                                        // first segment: its own row count
    } else if (NMAT == 1 && mp.seg[0] > 0) {                  // uniform over the workgroup
        const bool third = mp.seg[1] > 0 && row0 >= mp.seg[1];
        seg_idx = third ? 2 : 1;
        const int base = third ? mp.seg[1] : mp.seg[0];
        N = (third || mp.seg[1] == 0 ? Nall : mp.seg[1]) - base;
        row0 -= base;
        d0 = third ? mp.data[2] : mp.data[1];
        sc0 = third ? mp.scales[2] : mp.scales[1];
        zr0 = third ? mp.zeros[2] : mp.zeros[1];
        o0 = third ? mp.out[2] : mp.out[1];
    }

    const int n_l = lane & 15;           // weight row within the tile (B column) and A row
    const int kq = lane >> 4;            // 16-byte quarter of a group this lane reads
    const int row = row0 + n_l;
    const int row_c = row < N ? row : N - 1;

    const uint8_t *wdata = (NMAT == 2 && mat) ? d1 : d0;
    // RAW_RN with a rounded operand: the row's rms is reduced before the image is built
    const bool rnd = RN && (in.round_mode == 1 || (in.round_mode == 2 && seg_idx > 0));
    // IMAGE with a rounded second image for the later segments
    const bool img2 = !RAW && in.round_mode == 2 && seg_idx > 0;
    const _Float16 *ihi = img2 ? in.hi2 : in.hi;
    const _Float16 *ilo = img2 ? in.lo2 : in.lo;
    const float *igs = img2 ? in.gsum2 : in.gsum;
    const uint8_t *wrow = wdata + (size_t)row_c * (K / 2) + kq * 16;

    uint32_t *szs = lds_dyn;
    float *sxs = reinterpret_cast<float *>(lds_dyn + NMAT * G * 16);
    float *rsq = sxs + G * MT * 16;
    float *rmsv = rsq + (RN ? G * 16 : 0);
    _Float16 *xs = reinterpret_cast<_Float16 *>(rmsv + (RN ? 16 : 0));
    float4_t *red = reinterpret_cast<float4_t *>(xs);

    // scales/zeros of the tile: per matrix one contiguous run of 16 * G halfs
    // from row0 * G (elements past the last row clamp to it; their rows are
    // never stored); LDS slot [mat][g][row]
    const int per_mat = 16 * G;
    const int sz_total = NMAT * per_mat;
    const size_t sz_last = (size_t)N * G - 1;
    auto sz_elem = [&](int e, const uint16_t *&sp, const uint16_t *&zp, int &dst) {
        const bool second = NMAT == 2 && e >= per_mat;
        const int el = second ? e - per_mat : e;
        sp = reinterpret_cast<const uint16_t *>(second ? sc1 : sc0);
        zp = reinterpret_cast<const uint16_t *>(second ? zr1 : zr0);
        const int rr = el / G;
        dst = ((second ? G : 0) + (el - rr * G)) * 16 + rr;
        return min((size_t)row0 * G + el, sz_last);
    };
    uint32_t sv[kSZChunks], zv[kSZChunks];
    int sd[kSZChunks];
#pragma unroll
    for (int i = 0; i < kSZChunks; i++) {
        const uint16_t *sp, *zp;
        const size_t src = sz_elem(min(i * nthr + tid, sz_total - 1), sp, zp, sd[i]);
        sv[i] = sp[src];
        zv[i] = zp[src];
    }
    // IMAGE group sums: LDS slot e = (g * MT + t) * 16 + a holds A row a of
    // tile t: the hi (a < 8) or lo (a >= 8) sum of batch row 8t + (a & 7),
    // rows past the batch reusing row 0
    const int sx_total = G * MT * 16;
    auto sx_src = [&](int e) {
        const int a = e & 15;
        const int gt = e >> 4;
        const int g = gt / MT;
        const int t = gt - g * MT;
        const int r = 8 * t + (a & 7);
        const int rc = r < bc ? r : 0;
        return (size_t)(m0 + rc) * 2 * G + (a >> 3) * G + g;
    };
    // IMAGE without group sums (igs NULL: an image another launch wrote):
    // each stage forms its groups' sums from the halves it stages; the
    // loads below still go somewhere valid (the image itself, as floats), so
    // no branch sits around them
    const bool isum = !RAW && igs == nullptr;
    const float *igs_ld = isum ? reinterpret_cast<const float *>(ihi) : igs;
    float xsum[RAW ? 1 : kSXChunks];
    if (!RAW) {
#pragma unroll
        for (int i = 0; i < kSXChunks; i++) xsum[i] = igs_ld[sx_src(min(i * nthr + tid, sx_total - 1))];
    }

    // A rows of this lane in each tile: plane n_l >> 3, batch row 8t + (n_l & 7)
    int arow[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int r = 8 * t + (n_l & 7);
        arow[t] = (n_l >> 3) * bc + (r < bc ? r : 0);
    }

    float4_t acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};

    // One activation chunk as loaded: IMAGE (a = hi, b = lo) or RAW (a = x or
    // a, b, g = gamma, w = awq).
    struct Chunk {
        u32x4_t a, b, g, w;
    };
    auto chunk_load = [&](int r, int col, int gs0, Chunk &ch) __attribute__((always_inline)) {
        const size_t e = (size_t)gs0 * kGS + (size_t)col * 8;   // column within the row
        const size_t src = (size_t)(m0 + r) * K + e;
        if (!RAW) {
            const size_t isrc = (size_t)(m0 + r) * K + (size_t)img_chunk(gs0 * 16 + col) * 8;
            ch.a = *reinterpret_cast<const u32x4_t *>(ihi + isrc);
            ch.b = *reinterpret_cast<const u32x4_t *>(ilo + isrc);
            return;
        }
        ch.a = *reinterpret_cast<const u32x4_t *>(in.a + src);
        if (RN) {
            ch.b = *reinterpret_cast<const u32x4_t *>(in.b + src);
            ch.g = *reinterpret_cast<const u32x4_t *>(in.gamma + e);
        }
        if (in.awq) ch.w = *reinterpret_cast<const u32x4_t *>(in.awq + e);
    };
    // Writes the chunk's operand image into the LDS planes.  RAW: builds it;
    // the 16 chunks of a group (16 consecutive lanes -- one DPP row -- all
    // live or all not) sum their shares and the first of them stores the
    // group's sums.
    auto chunk_store = [&](int r, int col, int gs0, const Chunk &ch, bool live) __attribute__((always_inline)) {
        const int off = r * RSX + col * 8;
        if (!RAW) {
            *reinterpret_cast<u32x4_t *>(xs + off) = ch.a;
            *reinterpret_cast<u32x4_t *>(xs + bc * RSX + off) = ch.b;
            if (isum) {   // uniform
                float sh, sl;
                chunk_sums(__builtin_bit_cast(half8_t, ch.a), __builtin_bit_cast(half8_t, ch.b), sh, sl);
                sh = row16_sum(sh);
                sl = row16_sum(sl);
                if (live && (tid & 15) == 0) {
                    float *sx = sxs + ((gs0 + col / 16) * MT + (r >> 3)) * 16 + (r & 7);
                    sx[0] = sh * kTwoM24;
                    sx[8] = sl * kTwoM24;
                }
            }
            return;
        }
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&ch.a);
        float v[8];
        float sq = 0.0f;
        if (RN) {
            const _Float16 *bh = reinterpret_cast<const _Float16 *>(&ch.b);
            const _Float16 *gh = reinterpret_cast<const _Float16 *>(&ch.g);
            const float ri = rnd ? rmsv[r] : 1.0f;   // rms_inv of row r (row_rms, before)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float rr = (float)ah[i] + (float)bh[i];
                sq = __builtin_fmaf(rr, rr, sq);
                v[i] = rnd ? (float)(_Float16)(rr * ri * (float)gh[i]) : rr * (float)gh[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = (float)ah[i];
        }
        if (in.awq) {
            const _Float16 *wh = reinterpret_cast<const _Float16 *>(&ch.w);
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = div_awq(v[i], (float)wh[i]);
        }
        half8_t hi, lo;
        float sh, sl;
        chunk_operands(v, hi, lo, sh, sl);
        *reinterpret_cast<half8_t *>(xs + off) = hi;
        *reinterpret_cast<half8_t *>(xs + bc * RSX + off) = lo;
        sh = row16_sum(sh);
        sl = row16_sum(sl);
        if (RN && !rnd) sq = row16_sum(sq);
        if (live && (tid & 15) == 0) {
            const int g = gs0 + col / 16;
            float *sx = sxs + (g * MT + (r >> 3)) * 16 + (r & 7);
            sx[0] = sh * kTwoM24;
            sx[8] = sl * kTwoM24;
            if (RN && !rnd) rsq[g * 16 + r] = sq;
        }
    };
    // rms_inv of every batch row from the per-group sums of r^2 in LDS, by
    // wave 0: lane (r, j) = (lane >> 3, lane & 7) adds groups j, j + 8, ...
    // of row r, then an xor tree over j (rows <= 8 when RN)
    auto row_rms = [&]() __attribute__((always_inline)) {
        const int r = lane >> 3, j = lane & 7;
        float ss = 0.0f;
        if (r < bc)
            for (int g = j; g < G; g += 8) ss += rsq[g * 16 + r];
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        if (r < bc && j == 0) rmsv[r] = 1.0f / __builtin_sqrtf(ss / (float)K + in.eps);
    };
    // rounded RAW_RN operand: the per-group sums of r^2 first (as chunk_store
    // would store them), then a barrier and row_rms, so every chunk sees its
    // row's rms
    auto chunk_sq = [&](int r, int col, int gs0, const Chunk &ch, bool live) __attribute__((always_inline)) {
        const _Float16 *ah = reinterpret_cast<const _Float16 *>(&ch.a);
        const _Float16 *bh = reinterpret_cast<const _Float16 *>(&ch.b);
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float rr = (float)ah[i] + (float)bh[i];
            sq = __builtin_fmaf(rr, rr, sq);
        }
        sq = row16_sum(sq);
        if (live && (tid & 15) == 0) rsq[(gs0 + col / 16) * 16 + r] = sq;
    };

    auto stage = [&](const int gs0, const bool first) __attribute__((always_inline)) {
        const int SGs = min(SG, G - gs0);
        // (a) activation loads of this stage
        const int cpr = SGs * 16;                  // 8-element chunks per batch row
        const int total = bc * cpr;                // a multiple of 16
        Chunk ch[XC];
#pragma unroll
        for (int i = 0; i < XC; i++) {
            const int c = min(i * nthr + tid, total - 1);
            const int r = c / cpr;
            chunk_load(r, c - r * cpr, gs0, ch[i]);
        }
        // (b) this wave's weights for the stage: unconditional, clamped loads
        const int wg0 = gs0 + (part * SGs) / parts;
        const int ng = gs0 + ((part + 1) * SGs) / parts - wg0;
        u32x4_t wq[NG];
#pragma unroll
        for (int i = 0; i < NG; i++) {
            const int g = min(max(wg0 + min(i, ng - 1), 0), G - 1);
            wq[i] = *reinterpret_cast<const u32x4_t *>(wrow + (size_t)g * 64);
        }
        // (c) scales/zeros (and IMAGE group sums) -> LDS, first stage.  The
        // writes are unconditional -- threads past the end rewrite the last
        // element with its own value -- so the compiler has no branch to sink
        // the loads into behind a wait for the weights.
        if (first) {
#pragma unroll
            for (int i = 0; i < kSZChunks; i++) szs[sd[i]] = sv[i] | (zv[i] << 16);
            for (int e = kSZChunks * nthr + tid; e < sz_total; e += nthr) {
                const uint16_t *sp, *zp;
                int dst;
                const size_t src = sz_elem(e, sp, zp, dst);
                szs[dst] = (uint32_t)sp[src] | ((uint32_t)zp[src] << 16);
            }
            if (!RAW && !isum) {
#pragma unroll
                for (int i = 0; i < kSXChunks; i++) sxs[min(i * nthr + tid, sx_total - 1)] = xsum[i];
                for (int e = kSXChunks * nthr + tid; e < sx_total; e += nthr) sxs[e] = igs[sx_src(e)];
            }
        } else {
            // the previous stage is done with the activation planes
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        }
        // (d) operand image -> LDS (clamped duplicates write identical values)
        if (RN && rnd) {
#pragma unroll
            for (int i = 0; i < XC; i++) {
                const int c = min(i * nthr + tid, total - 1);
                const int r = c / cpr;
                chunk_sq(r, c - r * cpr, gs0, ch[i], i * nthr + tid < total);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            if (wave == 0) row_rms();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        }
#pragma unroll
        for (int i = 0; i < XC; i++) {
            const int c = min(i * nthr + tid, total - 1);
            const int r = c / cpr;
            chunk_store(r, c - r * cpr, gs0, ch[i], i * nthr + tid < total);
        }
        if (!RN) {
            for (int c = XC * nthr + tid; c < total; c += nthr) {  // chunks beyond XC per thread
                const int r = c / cpr;
                Chunk cx;
                chunk_load(r, c - r * cpr, gs0, cx);
                chunk_store(r, c - r * cpr, gs0, cx, true);
            }
        }
        // LDS-only barrier: the weight loads stay in flight across it
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

        // (e) MFMA over the wave's groups
#pragma unroll
        for (int i = 0; i < NG; i++) {
            if (i < ng) {
                const int g = wg0 + i;
                const uint32_t sz = szs[(mat * G + g) * 16 + n_l];
                const float s24 = (float)__builtin_bit_cast(_Float16, (uint16_t)(sz & 0xFFFFu)) * kTwo24;
                const float z = (float)__builtin_bit_cast(_Float16, (uint16_t)(sz >> 16));
                u32x4_t bq[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t w = wq[i][j];
                    const uint32_t p0 = __builtin_amdgcn_perm(w, 0u, 0x0C050C04u);  // b0, b1
                    const uint32_t p1 = __builtin_amdgcn_perm(w, 0u, 0x0C070C06u);  // b2, b3
                    bq[j] = (u32x4_t){p0, p1, p0 & 0x00F000F0u, p1 & 0x00F000F0u};
                }
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const _Float16 *xa = xs + arow[t] * RSX + (g - gs0) * kGS + kq * 32;
                    float4_t accg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const half8_t av = *reinterpret_cast<const half8_t *>(xa + j * 8);
                        accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            av, __builtin_bit_cast(half8_t, bq[j]), accg, 0, 0, 0);
                    }
                    // D rows 4*kq + r of tile t
                    const float4_t sx = *reinterpret_cast<const float4_t *>(sxs + (g * MT + t) * 16 + 4 * kq);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc[t][r] = __builtin_fmaf(s24, __builtin_fmaf(-z, sx[r], accg[r]), acc[t][r]);
                }
            }
        }
    };
    stage(0, true);
    for (int gs0 = SG; gs0 < G; gs0 += SG) stage(gs0, false);

    // reduce: the partial-sum region overlays the activation planes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (RN && !rnd && wave == 0) row_rms();   // (rounded: computed before the operand)
#pragma unroll
    for (int t = 0; t < MT; t++) red[(t * waves + wave) * 64 + lane] = acc[t];
    __syncthreads();
    if (RN && blockIdx.x == 0) {  // residual and normed rows, once per batch tile
        const int cpr = K / 8;
        for (int c = tid; c < bc * cpr; c += nthr) {
            const int r = c / cpr;
            const size_t e = (size_t)(c - r * cpr) * 8;
            const size_t off = (size_t)(m0 + r) * K + e;
            const u32x4_t av = *reinterpret_cast<const u32x4_t *>(in.a + off);
            const u32x4_t bv = *reinterpret_cast<const u32x4_t *>(in.b + off);
            const u32x4_t gv = *reinterpret_cast<const u32x4_t *>(in.gamma + e);
            const _Float16 *ah = reinterpret_cast<const _Float16 *>(&av);
            const _Float16 *bh = reinterpret_cast<const _Float16 *>(&bv);
            const _Float16 *gh = reinterpret_cast<const _Float16 *>(&gv);
            const float ri = rmsv[r];
            half8_t res, nrm;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float rr = (float)ah[i] + (float)bh[i];
                res[i] = (_Float16)rr;
                nrm[i] = (_Float16)(rr * ri * (float)gh[i]);
            }
            *reinterpret_cast<half8_t *>(in.residual_out + off) = res;
            *reinterpret_cast<half8_t *>(in.normed_out + off) = nrm;
        }
    }
    if (wave != 0) return;
    // wave 0: lanes 32t..32t+31 finish tile t.  Lane l of a tile holds D rows
    // 4*(l>>4) + r, r < 4; rows < 8 are hi halves, row + 8 (lane l + 32) the lo
    // halves of the same batch rows.  Parts are summed in part order.
    const int t = lane >> 5;
    if (t >= MT) return;
    const int l2 = lane & 31;
    // parts 1, 2, .. added in order, their reads issued four parts at a time
    // (clamped to the last part) so one wait covers four
    float4_t sum[NMAT];
#pragma unroll
    for (int mt = 0; mt < NMAT; mt++) {
        const float4_t *rp = red + (t * waves + mt * parts) * 64;
        sum[mt] = rp[l2] + rp[l2 + 32];
        for (int p0 = 1; p0 < parts; p0 += 4) {
            float4_t pv[4][2];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int p = min(p0 + j, parts - 1);
                pv[j][0] = rp[p * 64 + l2];
                pv[j][1] = rp[p * 64 + l2 + 32];
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (p0 + j < parts) sum[mt] += pv[j][0] + pv[j][1];
        }
    }
    if (row >= N) return;
    const int mrow = 8 * t + 4 * (l2 >> 4);   // batch row within the tile
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = m0 + mrow + r;
        if (m >= B) break;
        float scale = 1.0f;
        if (RN) scale = rnd ? 1.0f : rmsv[mrow + r];
        else if (!RAW && in.row_scale && !img2) scale = in.row_scale[m];
        if (EPI == EPI_SILU || EPI == EPI_GELU) {
            // the row scale (rms_inv) belongs to both projections, ahead of the activation
            const float g = sum[0][r] * scale, u = sum[NMAT - 1][r] * scale;
            float act;
            if (EPI == EPI_SILU) {
                act = g / (1.0f + __expf(-g));
            } else {
                float inner = 0.7978845608f * (g + 0.044715f * g * g * g);
                inner = fminf(fmaxf(inner, -10.0f), 10.0f);
                act = 0.5f * g * (1.0f + tanhf(inner));
            }
            o0[(size_t)m * N + row] = __float2half(act * u);
        } else {
#pragma unroll
            for (int mt = 0; mt < NMAT; mt++)
                (mt ? o1 : o0)[(size_t)m * N + row] = __float2half(sum[mt][r] * scale);
        }
    }
}

// ---------------------------------------------------------------------------
// host-side launch helpers
// ---------------------------------------------------------------------------
struct Launch {
    dim3 grid, block;
    size_t lds;
    hipStream_t st;
    int N, K, B, parts, SG;
    int ng;    // most groups a wave takes in one stage
    int xc;    // 1 or 2 activation chunks per thread ahead of the weights
    int mt;    // MFMA tiles of 8 batch rows per workgroup (1 or 2)
};

template <int NMAT, int EPI, int MT, int NG, int SRC>
void launch_xc(const Launch &L, const MatPtrs &mp, const ActIn &in) {
    if (L.xc == 1)
        hipLaunchKernelGGL((int4_matvec_kernel<NMAT, EPI, MT, NG, 1, SRC>), L.grid, L.block, L.lds, L.st, mp,
                           in, L.N, L.K, L.B, L.parts, L.SG);
    else
        hipLaunchKernelGGL((int4_matvec_kernel<NMAT, EPI, MT, NG, 2, SRC>), L.grid, L.block, L.lds, L.st, mp,
                           in, L.N, L.K, L.B, L.parts, L.SG);
}

template <int NMAT, int EPI, int MT, int SRC>
void launch_ng(const Launch &L, const MatPtrs &mp, const ActIn &in) {
    if (L.ng <= 2) launch_xc<NMAT, EPI, MT, 2, SRC>(L, mp, in);
    else if (L.ng <= 3) launch_xc<NMAT, EPI, MT, 3, SRC>(L, mp, in);
    else if (L.ng <= 4) launch_xc<NMAT, EPI, MT, 4, SRC>(L, mp, in);
    else if (L.ng <= 5) launch_xc<NMAT, EPI, MT, 5, SRC>(L, mp, in);
    else if (L.ng <= 6) launch_xc<NMAT, EPI, MT, 6, SRC>(L, mp, in);
    else launch_xc<NMAT, EPI, MT, 8, SRC>(L, mp, in);
}

// RAW-source launches (instantiated in int4_matvec_raw.hip): nmat/epi as in
// the kernel, rn selects SRC_RAW_RN (nmat 1 with EPI_STORE, or nmat 2 with
// EPI_SILU / EPI_GELU); L.mt must be 1.
void launch_raw(int nmat, int epi, bool rn, const Launch &L, const MatPtrs &mp, const ActIn &in);
// IMAGE-source launches with two MFMA tiles (int4_matvec_mt2.hip).
void launch_image_mt2(int nmat, int epi, const Launch &L, const MatPtrs &mp, const ActIn &in);
// The CU-balanced row-band kernel at batch 1-2 (int4_matvec_band.hip), for
// plain sources and residual-norm sources of round_mode 0 or 1 (in.b set);
// *used is false where it does not apply.
int launch_band_matvec(hipStream_t st, int cus, int B, int nmat, int epi, int N, int K, const MatPtrs &mp,
                       const ActIn &in, bool *used, bool probe = false);
// The tile grid over an IMAGE source (in.hi / in.lo, in.hi2 / in.lo2 for the
// later segments of round_mode 2, in.row_scale) with the operands read straight
// from the image, 1-8 batch rows (int4_matvec_da.hip); the image's group sums
// are not read (the kernel forms them on the matrix cores).
bool image_da_applies(int nmat, int B, int K);
int launch_image_da(hipStream_t st, int nmat, int epi, int N, int K, int B, const MatPtrs &mp, const ActIn &in);
// Split-K over an IMAGE source (one matrix with its row segments, EPI_STORE,
// 3-8 rows): f32 partials in ws (splitk_workspace_bytes), then a combine
// launch that applies in.row_scale to the rows below split_rows and writes
// each row's segment.  split_rows: the first row of the second image (mixed
// rounding: mp.seg[0]), else N.
bool splitk_applies(int nmat, int B, int N, int K, int split_rows, int cus);
size_t splitk_workspace_bytes(int B, int N, int split_rows, int cus);
int launch_splitk(hipStream_t st, int cus, int N, int K, int B, const MatPtrs &mp, const ActIn &in, int split_rows,
                  void *ws);

}  // namespace imh_int4
