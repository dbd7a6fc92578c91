// tq_kernels.hip -- TurboQuant INT8 KV cache: cache write and GQA decode attention.
//
// Cache write (turboquant.metal:52-170): rotate by R = D.H.D/sqrt(d), L2 norm as
// the per-(token, head) scale, nearest-centroid index by boundary scan; for K
// the 7-bit index is completed by the sign of the QJL projection of the
// residual.  The f32 operation order is fixed (halving-stride tree sums over
// the 128 lanes, fmaf QJL dot in increasing k, no contraction elsewhere) so the
// codes are reproducible bit for bit by the CPU oracle.
//
// Decode attention (turboquant.metal:202-462 semantics; the structure is this
// file's own): one workgroup per (KV split, kv head, sequence) serves all
// query heads of the GQA group, so each KV byte is read once per group instead
// of once per query head.  Per 16-position chunk a wave
//   * builds the dequantized K chunk as MFMA operand B with one LDS lookup per
//     byte (codebook entry as an f16 hi/lo pair) plus the +-1 QJL signs taken
//     straight from bit 7, and runs v_mfma_f32_16x16x32_f16 against the rotated
//     query (hi, lo) and its QJL projection (hi, lo) packed as rows of operand A;
//   * folds the per-position scales in and runs the online softmax of all the
//     group's heads at once with DPP row reductions;
//   * accumulates P.V on v_mfma_f32_16x16x32_f16 (positions as the contraction
//     index, each position twice: against the f16 hi and lo halves of its
//     codebook value) from V codes transposed in registers, with the weights
//     (times the V scale) as f16.
// Waves combine through LDS; with one split the workgroup normalises and
// rotates the result back, with several each publishes its split's partial
// (o, max, sum) and a second kernel merges the splits (log-sum-exp,
// fused_sdpa_reduce, flash_decode.metal:163-215) and rotates back.
#include <hip/hip_runtime.h>
#include <type_traits>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>

#include "dpp_reduce.h"
#include "imh_internal.h"
#include "qk_norm_rope.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

constexpr int kD = 128;          // head_dim the kernels are built for
constexpr int kChunk = 16;       // positions per MFMA block
constexpr int kWaves = 4;        // waves per attention workgroup
constexpr int kSplitQuantum = kChunk * kWaves;
constexpr int kMaxSplits = 512;     // split count cap
constexpr int kAutoSplitLen = 256;  // shortest split the automatic split count makes

// Strides 1..32 of the unnormalised fast Walsh-Hadamard transform of a
// 64-element vector held one element per lane: at stride s the pair (j, j + s)
// becomes (x_j + x_{j+s}, x_j - x_{j+s}), strides in increasing order.
__device__ __forceinline__ float hadamard64(float x, int lane) {
#pragma unroll
    for (int step = 1; step < 64; step *= 2) {
        const float p = __shfl_xor(x, step);
        x = (lane & step) ? p - x : x + p;   // element j + step of the pair: x_j - x_{j+step}
    }
    return x;
}

// IEEE round-to-nearest f32 square root: the hardware v_sqrt_f32 result
// (within 1 ulp) corrected with two fma residuals.  Inputs here are finite
// and >= 1e-20, so no denormal rescaling is needed.
__device__ __forceinline__ float sqrt_rn(float x) {
    float s = __builtin_amdgcn_sqrtf(x);
    const int si = __builtin_bit_cast(int, s);
    const float dn = __builtin_bit_cast(float, si - 1);
    const float up = __builtin_bit_cast(float, si + 1);
    const float r_dn = __builtin_fmaf(-dn, s, x);
    const float r_up = __builtin_fmaf(-up, s, x);
    s = (r_dn <= 0.0f) ? dn : s;
    s = (r_up > 0.0f) ? up : s;
    return s;
}

// ---------------------------------------------------------------------------
// cache write: one wave per (tensor, kv head, token, sequence); lane l holds
// elements l and l + 64.  The Walsh-Hadamard butterfly (strides 1..32 across
// lanes by xor shuffles, 64 inside the lane) and the halving-stride tree sums
// (64 inside the lane, 32..1 by down shuffles) keep the f32 order of a
// 128-element LDS tree bit for bit, with no workgroup barrier.
// ---------------------------------------------------------------------------
struct TqWriteArgs {
    const __half *kv[2];   // [0] K, [1] V projections [batch][tokens][nkv][kD]
    uint8_t *codes[2];
    float *scales[2];
    float *r_norms;        // K only
    const float *codebook[2];
    const float *sorted[2];      // boundaries sorted by value (NaN dropped)
    const int32_t *prefmax[2];   // running max of (original index + 1)
    int n_search[2];
};

// Sum of a 128-element vector held as (element lane, element lane + 64): the
// pair first, then halving strides 32..1 by down shuffles -- the f32 order of
// a 128-element halving tree.  Every lane gets the sum.
__device__ __forceinline__ float tree_sum128(float a, float b) {
#pragma clang fp contract(off)
    float v = a + b;
    for (int sh = 32; sh > 0; sh >>= 1) v = v + __shfl_down(v, sh);
    return __shfl(v, 0);
}

// One vector's TurboQuant codes (turboquant.metal:52-170), held by one wave as
// f0 = element lane, f1 = element lane + 64: rotation, L2 norm as the scale,
// centroid index by the table's own boundary rule; with kcb (K) also the
// residual u - kcb[code] and its norm.  The QJL sign bit is the caller's.
struct TqCodes {
    uint32_t c0, c1;   // codes of elements lane, lane + 64
    float l2;          // scale
    float r0, r1, rn;  // K: residual elements and norm
};
__device__ __forceinline__ TqCodes tq_quantize_vec(float f0, float f1, int lane, float sg0, float sg1,
                                                   const float *bd, const int32_t *pm, int nb,
                                                   const float *kcb) {
#pragma clang fp contract(off)
    const float rscale = 1.0f / sqrtf((float)kD);
    float x0 = f0 * sg0;
    float x1 = f1 * sg1;
    x0 = hadamard64(x0, lane);
    x1 = hadamard64(x1, lane);
    {
        const float lo = x0, hi = x1;   // stride 64: elements lane and lane + 64
        x0 = lo + hi;
        x1 = lo - hi;
    }
    const float xr0 = x0 * (sg0 * rscale), xr1 = x1 * (sg1 * rscale);
    TqCodes r;
    r.l2 = sqrt_rn(fmaxf(tree_sum128(xr0 * xr0, xr1 * xr1), 1e-20f));
    const float inv = __fdiv_rn(1.0f, fmaxf(r.l2, 1e-10f));
    const float u0 = xr0 * inv, u1 = xr1 * inv;
    // 1 + the last j with u >= boundary[j] in the table's own order (0 if
    // none): the boundaries that u passes are a prefix of the sorted ones,
    // so the answer is the prefix max there (turboquant.metal:118-124)
    auto find = [&](float u) {
        int lo = 0, hi = nb;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (u >= bd[mid]) lo = mid + 1;
            else hi = mid;
        }
        return lo == 0 ? 0 : pm[lo - 1];
    };
    r.c0 = (uint32_t)find(u0);
    r.c1 = (uint32_t)find(u1);
    r.r0 = r.r1 = r.rn = 0.0f;
    if (kcb) {
        r.r0 = u0 - kcb[r.c0];
        r.r1 = u1 - kcb[r.c1];
        r.rn = sqrt_rn(fmaxf(tree_sum128(r.r0 * r.r0, r.r1 * r.r1), 1e-20f));
    }
    return r;
}

constexpr int kWriteMaxWaves = 16;

// grid (tokens, batch), block 64 * W with W = min(16, nkv * count): every K
// and V vector of one token, one wave each (looping when there are more than
// 16); vector v is tensor first + v / nkv, kv head v % nkv.  The QJL matrix is
// staged into LDS once per workgroup by all threads (64 KB, one round trip).
__global__ void __launch_bounds__(64 * kWriteMaxWaves) tq_cache_write_kernel(
    const TqWriteArgs a, int first, int count, int tokens, int nkv, int max_seq, int base_pos,
    const int32_t *__restrict__ positions, const float *__restrict__ signs, const float *__restrict__ qjl_t) {
#pragma clang fp contract(off)
    __shared__ float sqt[kD * kD];   // S^T, row k = column k of S
    __shared__ float bnd[2][256];    // sorted boundaries
    __shared__ int32_t bpm[2][256];  // prefix max of index + 1
    __shared__ float res[kWriteMaxWaves][kD];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int W = blockDim.x >> 6;
    const int t = blockIdx.x, b = blockIdx.y;
    const bool has_k = first == 0;
    // this wave's first vector, the signs and the position are loaded before
    // the table staging so that every load of the workgroup is in flight at once
    auto src_of = [&](int v) {
        return a.kv[first + v / nkv] + (((size_t)b * tokens + t) * nkv + v % nkv) * kD;
    };
    const int v0 = wave;
    __half pre0 = __float2half(0.0f), pre1 = __float2half(0.0f);
    if (v0 < nkv * count) {
        pre0 = src_of(v0)[lane];
        pre1 = src_of(v0)[lane + 64];
    }
    const float sg0 = signs[lane], sg1 = signs[lane + 64];
    const long long start = positions ? (long long)positions[b] : (long long)base_pos;
    if (has_k) {
        const float4 *src4 = reinterpret_cast<const float4 *>(qjl_t);
        float4 *dst4 = reinterpret_cast<float4 *>(sqt);
        for (int e = tid; e < kD * kD / 4; e += blockDim.x) dst4[e] = src4[e];
    }
    for (int w = first; w < first + count; w++)
        for (int j = tid; j < a.n_search[w]; j += blockDim.x) {
            bnd[w][j] = a.sorted[w][j];
            bpm[w][j] = a.prefmax[w][j];
        }
    __syncthreads();

    long long pl = (start + t) % max_seq;
    if (pl < 0) pl += max_seq;

    for (int v = wave; v < nkv * count; v += W) {
        const int which = first + v / nkv, h = v % nkv;
        const size_t slot = ((size_t)b * nkv + h) * (size_t)max_seq + (size_t)pl;
        const __half *src = src_of(v);
        float f0 = __half2float(v == v0 ? pre0 : src[lane]);
        float f1 = __half2float(v == v0 ? pre1 : src[lane + 64]);
        const TqCodes qc = tq_quantize_vec(f0, f1, lane, sg0, sg1, bnd[which], bpm[which], a.n_search[which],
                                           which == 0 ? a.codebook[0] : nullptr);
        uint32_t code0 = qc.c0, code1 = qc.c1;
        const float l2 = qc.l2;

        if (which == 0) {
            res[wave][lane] = qc.r0;
            res[wave][lane + 64] = qc.r1;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll 16
            for (int k = 0; k < kD; k++) {
                const float rk = res[wave][k];
                acc0 = __builtin_fmaf(sqt[k * kD + lane], rk, acc0);
                acc1 = __builtin_fmaf(sqt[k * kD + lane + 64], rk, acc1);
            }
            if (acc0 >= 0.0f) code0 |= 0x80u;
            if (acc1 >= 0.0f) code1 |= 0x80u;
            if (lane == 0) a.r_norms[slot] = qc.rn;
            __builtin_amdgcn_wave_barrier();   // res[wave] is rewritten by the next vector
        }
        a.codes[which][slot * kD + lane] = (uint8_t)code0;
        a.codes[which][slot * kD + lane + 64] = (uint8_t)code1;
        if (lane == 0) a.scales[which][slot] = l2;
    }
}

// ---------------------------------------------------------------------------
// decode attention
// ---------------------------------------------------------------------------
// Attention: grid (num_splits, num_kv_heads, batch), block 64 * kWaves.  Each
// wave walks its split in 16-position chunks; the codes and per-position
// scales of the next chunk are loaded before the current one is computed.
//
// Register layout.  Head hh of the group owns rows 4hh..4hh+3 of the 16-row
// MFMA operands, so in every 16x16 result lane group g = lane >> 4 holds head
// g: the scores of one head are one DPP row (softmax reductions serve all
// heads at once) and the running max, sum and rescale are per lane.  P.V runs
// on v_mfma_f32_16x16x32_f16 with the positions as the contraction index:
// result column c of block j is dim 8c + j, so lane (c, g) loads V codes of
// positions 4g..4g+3 at dims 8c..8c+7 (four 8-byte row loads, coalesced
// across the 16 lanes of a row) and its B operand for block j is the
// codebook values (f16 hi, lo) of byte j of the four rows -- a register
// transpose, no LDS staging.  The weights w * v_scale go through a 256-byte
// per-wave LDS buffer into row 4hh of operand A as f16, each weight twice.  Built with -amdgpu-mfma-vgpr-form so the accumulators
// stay in VGPRs (no AGPR round trip around the softmax rescale).
// Optional QK-norm + RoPE of the query ahead of the rotation (head_dim 128 =
// rotary_dim): norm weight [128], cos / sin tables [max_pos][64], the query's
// position positions[b].  norm == NULL: the query is used as given (the other
// pointers still address readable memory: max_pos 1, 64 table entries).
struct QkRope {
    const __half *norm;
    const __half *cos;
    const __half *sin;
    const int32_t *positions;
    int max_pos;
    float eps;
};

// Optional cache write of the step's token in the same launch (k_new == NULL:
// attention only).  The grid then has one more workgroup per (kv head,
// sequence), the last in x: it quantizes the token's K (after the QK-norm +
// RoPE when k_norm is set, with qr's tables) and V as the cache write does,
// stores the codes at row L - 1 (L = the sequence's length with the token),
// and publishes that one position as its split's partial; the other splits
// cover [0, L - 1).  Its work overlaps theirs, and the combine kernel merges
// it like any split.
struct TqFuse {
    const __half *k_new, *v_new;   // [batch][nkv][kD]
    uint8_t *kcodes, *vcodes;      // the cache, writable
    float *kscales, *vscales, *krnorm;
    const float *sorted[2];        // search tables of the cache write
    const int32_t *prefmax[2];
    int n_search[2];
    const __half *k_norm;
    const float *qjl_t;   // S^T again: a separate argument, so its addresses are
                          // not shared with (and held live from) the prologue's
};

// f16 hi + lo pair of a codebook table entry as f32
__device__ __forceinline__ float tab_f32(uint32_t e) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(e & 0xFFFFu)) +
           (float)__builtin_bit_cast(_Float16, (uint16_t)(e >> 16));
}

// Codebook entry c as (f16 hi | f16 lo << 16): the LDS tables of the
// attention kernels (an f16 V entry alone would bias every output by its
// rounding error, a bias that does not average out over positions while the
// output itself shrinks as 1/sqrt(positions): rel-L2 1.9e-3 at 30k positions
// of random V).
__device__ __forceinline__ uint32_t tab_entry(float v) {
    const _Float16 hi = (_Float16)v;
    const _Float16 lo = (_Float16)(v - (float)hi);
    return (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
}

// One 16-position chunk of a (sequence, kv head)'s cache as the attention
// loops read it.  Lane (n, g) = (lane & 15, lane >> 4) takes K code bytes
// 32 g .. 32 g + 31 of position p0 + n and that position's scales, and V code
// bytes 8 n .. 8 n + 7 of positions p0 + 4 g .. p0 + 4 g + 3 (the P.V
// operand's transpose).  Loads go through buffer resources bounded at the
// range's end: rows at or past it read as zeros and fetch nothing.
struct ChunkIn {
    uint4 k0, k1;
    uint2 v[4];
    float ksc, krn, vsc;
};
struct ChunkRsrc {
    __amdgpu_buffer_rsrc_t kc, vc, ks, kr, vs;
};
__device__ __forceinline__ ChunkRsrc chunk_rsrc(const uint8_t *kcodes, const uint8_t *vcodes, const float *kscales,
                                                const float *krnorm, const float *vscales, size_t head_base,
                                                int rows) {
    constexpr uint32_t kRsrcWord3 = 0x00020000u;
    ChunkRsrc r;
    r.kc = __builtin_amdgcn_make_buffer_rsrc((void *)(kcodes + head_base * kD), 0, rows * kD, kRsrcWord3);
    r.vc = __builtin_amdgcn_make_buffer_rsrc((void *)(vcodes + head_base * kD), 0, rows * kD, kRsrcWord3);
    r.ks = __builtin_amdgcn_make_buffer_rsrc((void *)(kscales + head_base), 0, rows * 4, kRsrcWord3);
    r.kr = __builtin_amdgcn_make_buffer_rsrc((void *)(krnorm + head_base), 0, rows * 4, kRsrcWord3);
    r.vs = __builtin_amdgcn_make_buffer_rsrc((void *)(vscales + head_base), 0, rows * 4, kRsrcWord3);
    return r;
}
__device__ __forceinline__ void load_chunk(const ChunkRsrc &r, int p0, int n_l, int kg, ChunkIn &c) {
    const int koff = (p0 + n_l) * kD + kg * 32;
    c.k0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r.kc, koff, 0, 0));
    c.k1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r.kc, koff + 16, 0, 0));
    const int voff = (p0 + 4 * kg) * kD + n_l * 8;
#pragma unroll
    for (int i = 0; i < 4; i++)
        c.v[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r.vc, voff + i * kD, 0, 0));
    const int soff = (p0 + n_l) * 4;
    c.ksc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r.ks, soff, 0, 0));
    c.krn = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r.kr, soff, 0, 0));
    c.vsc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r.vs, soff, 0, 0));
}

// Score operands B of k-slice j from the lane's code words kw[2j], kw[2j+1]
// (dims 32 g + 8 j .. + 7, k-slot order {0, 2, 1, 3} within each word): the
// codebook entries' f16 hi and lo parts (one LDS lookup per byte) and the
// +-1 QJL signs straight from bit 7.
// Codebook tables spread over the LDS banks (the lookups of 64 lanes with
// random codes conflicted on ~55 % of the LDS's active cycles): row c of 256
// bytes holds the K entry of code byte c in words 0..31 and the V entry in
// words 32..63, and lane l reads copy l & 31, so the 32 lanes of a half-wave
// hit 32 different banks whatever their codes.  The byte offset of code byte
// k of w is one v_perm: (byte << 8) | lane offset (4 (l & 31), + 128 for V).
constexpr int kTabRowBytes = 256;
constexpr int kSpreadMinLen = 1024;   // positions per split from which the decode loop uses them
constexpr int kLazyMinLen = 1024;     // positions per split from which the rescale is lazy
constexpr int kTabBytes = 256 * kTabRowBytes;
__device__ __forceinline__ uint32_t tab_read(const uint8_t *tabs, uint32_t w, int k, uint32_t lane_off) {
    const uint32_t off = __builtin_amdgcn_perm(w, lane_off, 0x0C0C0000u | ((4u + (uint32_t)k) << 8));
    return *reinterpret_cast<const uint32_t *>(tabs + off);
}
// tabs <- 32 copies of each entry of ktab / vtab (256 threads, wave w,
// instruction i: rows 16 i + 4 w + (lane >> 4), 16 bytes per lane)
__device__ __forceinline__ void spread_tables(uint8_t *tabs, const uint32_t *ktab, const uint32_t *vtab, int lane,
                                              int wave) {
    const int chunk = lane & 15;
    const uint32_t *src = chunk < 8 ? ktab : vtab;
#pragma unroll 4
    for (int i = 0; i < 16; i++) {
        const int r = 16 * i + 4 * wave + (lane >> 4);
        const uint32_t v = src[r];
        *reinterpret_cast<uint4 *>(tabs + r * kTabRowBytes + chunk * 16) = make_uint4(v, v, v, v);
    }
}

// The loops' view of the tables: entries of code byte k of a word, K or V.
// TabOne: the single 256-entry copies; TabSpread: the bank-spread copies.
struct TabOne {
    const uint32_t *kt, *vt;
    __device__ __forceinline__ uint32_t k(uint32_t w, int b) const { return kt[(w >> (8 * b)) & 0xFF]; }
    __device__ __forceinline__ uint32_t v(uint32_t w, int b) const { return vt[(w >> (8 * b)) & 0xFF]; }
};
struct TabSpread {
    const uint8_t *t;
    uint32_t lk, lv;
    __device__ __forceinline__ uint32_t k(uint32_t w, int b) const { return tab_read(t, w, b, lk); }
    __device__ __forceinline__ uint32_t v(uint32_t w, int b) const { return tab_read(t, w, b, lv); }
};

template <class Tab>
__device__ __forceinline__ void k_operands(const uint32_t *kw2, const Tab &tab, half8_t &Bh, half8_t &Bl,
                                           half8_t &Bs) {
    uint32_t bh[4], bl[4], bs[4];
#pragma unroll
    for (int hw = 0; hw < 2; hw++) {
        const uint32_t w = kw2[hw];
        const uint32_t t0 = tab.k(w, 0);
        const uint32_t t1 = tab.k(w, 1);
        const uint32_t t2 = tab.k(w, 2);
        const uint32_t t3 = tab.k(w, 3);
        bh[2 * hw] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
        bl[2 * hw] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
        bh[2 * hw + 1] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
        bl[2 * hw + 1] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
        // +1 (0x3C00) where bit 7 of the code is set, -1 (0xBC00) where not
        bs[2 * hw] = ((w << 8) & 0x80008000u) ^ 0xBC00BC00u;
        bs[2 * hw + 1] = (w & 0x80008000u) ^ 0xBC00BC00u;
    }
    Bh = __builtin_bit_cast(half8_t, make_uint4(bh[0], bh[1], bh[2], bh[3]));
    Bl = __builtin_bit_cast(half8_t, make_uint4(bl[0], bl[1], bl[2], bl[3]));
    Bs = __builtin_bit_cast(half8_t, make_uint4(bs[0], bs[1], bs[2], bs[3]));
}

// Score operand B of code word w (dims 4t .. 4t + 3 of the lane's 32): the
// four bytes' codebook entries as they sit in the table, (f16 hi, f16 lo)
// pairs, so each k pair of the contraction is one dim's hi and lo part and no
// repacking is needed (the operand A row that takes q_hi twice gives
// q_hi (K_hi + K_lo), the row that takes q_lo and 0 gives q_lo K_hi).
template <class Tab>
__device__ __forceinline__ half8_t k_pair_operand(uint32_t w, const Tab &tab) {
    return __builtin_bit_cast(half8_t, make_uint4(tab.k(w, 0), tab.k(w, 1), tab.k(w, 2), tab.k(w, 3)));
}
// The +-1 QJL signs of code words kw2[0], kw2[1] from bit 7, k-slot order
// {0, 2, 1, 3} within each word.
__device__ __forceinline__ half8_t k_sign_operand(const uint32_t *kw2) {
    uint32_t bs[4];
#pragma unroll
    for (int hw = 0; hw < 2; hw++) {
        const uint32_t w = kw2[hw];
        // +1 (0x3C00) where bit 7 of the code is set, -1 (0xBC00) where not
        bs[2 * hw] = ((w << 8) & 0x80008000u) ^ 0xBC00BC00u;
        bs[2 * hw + 1] = (w & 0x80008000u) ^ 0xBC00BC00u;
    }
    return __builtin_bit_cast(half8_t, make_uint4(bs[0], bs[1], bs[2], bs[3]));
}

// P.V operand B of dim block j: codebook values (hi, lo) of byte j of the
// lane's four V position rows
template <class Tab>
__device__ __forceinline__ half8_t v_operand(const ChunkIn &c, int j, const Tab &tab) {
    uint32_t e[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t word = j < 4 ? c.v[i].x : c.v[i].y;
        e[i] = tab.v(word, j & 3);
    }
    return __builtin_bit_cast(half8_t, make_uint4(e[0], e[1], e[2], e[3]));
}

// Occupancy: 3 waves per SIMD (168 VGPRs); the fused token writer's extra
// live state needs more than that, so it runs at 2 rather than spill.
// LAZY: the softmax rescale of the output accumulators is skipped for chunks
// where no head's running maximum grew (chosen for splits of kLazyMinLen
// positions or more).
template <int GQA, bool FUSED, bool SPREAD, bool LAZY>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(FUSED ? 2 : 3))) tq_attention_kernel(
    const __half *__restrict__ q, int nh, int nkv, int max_seq, int seq_len, int T,
    const int32_t *__restrict__ seq_lens, float attn_scale, const float *__restrict__ signs,
    const float *__restrict__ qjl_t, const float *__restrict__ kcb, const float *__restrict__ vcb,
    const uint8_t *__restrict__ kcodes, const uint8_t *__restrict__ vcodes,
    const float *__restrict__ kscales, const float *__restrict__ vscales,
    const float *__restrict__ krnorm, int split_len, float *__restrict__ part_o,
    float *__restrict__ part_m, float *__restrict__ part_l,
    __half *__restrict__ out, const QkRope qr, const TqFuse fz) {
    __shared__ float qs[GQA][2][kD];
    __shared__ float wtab[2][256];     // token writer: sorted boundaries
    __shared__ int32_t wpm[2][256];    // token writer: prefix maxima
    __shared__ uint32_t ktab[256];   // entry c & 0x7F, indexed by the whole code byte
    __shared__ uint32_t vtab[256];   // V entry c, same packing as ktab
    // P.V weights of a chunk, each f16 twice (hi and lo slots of operand A)
    __shared__ __attribute__((aligned(16))) uint32_t wbuf[kWaves][4][16];
    // SPREAD: the spread tables of the KV loop; the waves' partial outputs om
    // use the same bytes before the tables are built and after the loop
    __shared__ __attribute__((aligned(16))) uint8_t tabs[SPREAD ? kTabBytes : kWaves * GQA * kD * 4];
    float(*om)[GQA][kD] = reinterpret_cast<float(*)[GQA][kD]>(tabs);
    __shared__ float mm[kWaves][GQA];
    __shared__ float ll[kWaves][GQA];
    __shared__ float wres[2][kD];      // token writer: K residual, then its QJL projection

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    // S = gridDim.x through an asm that also takes every kernel argument the
    // prologue reads: the compiler loads them all in one trip before it
    // (otherwise in dependent batches).  Not volatile and no memory operand,
    // so loads after it still count as unclobbered (scalar loads).
    int S;
    asm("" : "=s"(S) : "0"(gridDim.x), "s"(gridDim.y), "s"(gridDim.z), "s"(q), "s"(nh), "s"(nkv), "s"(max_seq),
        "s"(seq_len), "s"(T), "s"(seq_lens), "s"(attn_scale), "s"(signs), "s"(qjl_t), "s"(kcb), "s"(vcb));
    int S2;
    asm("" : "=s"(S2) : "0"(S), "s"(kcodes), "s"(vcodes), "s"(kscales), "s"(vscales), "s"(krnorm), "s"(split_len),
        "s"(qr.norm), "s"(qr.cos), "s"(qr.sin), "s"(qr.positions), "s"(qr.max_pos), "s"(qr.eps));
    S = S2;
    // With the token writers (FUSED): the grid in dispatch order is every
    // group's S - 1 splits first, then the groups' writers, so the streaming
    // workgroups spread evenly over the CUs (two per CU at ~512) and the
    // short-lived writers take spare slots.
    // z = b * T + t: query token t of sequence b (T tokens per sequence)
    int split = blockIdx.x, kvh = blockIdx.y, z = blockIdx.z;
    if (FUSED) {
        const int i = (blockIdx.z * gridDim.y + blockIdx.y) * S + blockIdx.x;
        const int sa = S - 1, streaming = sa * (int)(gridDim.y * gridDim.z);
        const int g = i < streaming ? i / sa : i - streaming;
        split = i < streaming ? i - g * sa : sa;
        kvh = g % (int)gridDim.y;
        z = g / (int)gridDim.y;
    }
    // uniform (scalar loads of the per-sequence values below)
    const int b = __builtin_amdgcn_readfirstlane(z / T), tq = z - b * T;
    const bool writer = FUSED && split == S - 1;   // the step's token (uniform per workgroup)

    // with seq_lens, seq_len is the bound every length is clamped to; the
    // sequence's RoPE position is read in the same trip
    const int32_t pos_b = qr.positions[b];
    int L = seq_lens ? min(seq_lens[b], seq_len) : seq_len;
    L = L < 0 ? 0 : (L > max_seq ? max_seq : L);
    // causal (turboquant.metal:268): token t of T sees positions < L - T + t + 1
    L -= T - 1 - tq;
    L = L < 0 ? 0 : L;
    const int L_tok = L;               // with the fused write: the token is row L_tok - 1
    if (FUSED) L = L > 0 ? L - 1 : 0;
    const int p_begin = split * split_len;
    const int p_end = min(p_begin + split_len, L);
    const size_t head_base = ((size_t)b * nkv + kvh) * (size_t)max_seq;
    const int n_l = lane & 15;   // score layout: position; P.V layout: column c
    const int kg = lane >> 4;    // lane group: K dims block / head / V position quad

    // loads bounded at p_end: rows at or past the split's end read as zeros
    // (their weights are zero), so no clamping, and each lane's offsets
    // advance by one add per chunk
    const ChunkRsrc crs = chunk_rsrc(kcodes, vcodes, kscales, krnorm, vscales, head_base, p_end > 0 ? p_end : 0);
    // wave w takes chunks p_begin + 16 w + 64 i of the split, one chunk in
    // flight; loads past the split's end read zeros and fetch nothing, so
    // they are issued unconditionally
    // Prologue loads go first: a wave's loads return in issue order, so the
    // query, tables and S^T issued ahead of the first chunk are not held
    // behind it.  S^T (128 x 128 f32, L2-resident) is read as float4s: thread
    // (kr, dq) = (tid >> 5, tid & 31) takes rows 16 kr .. 16 kr + 15 at
    // columns 4 dq .. 4 dq + 3.
    static_assert(kWaves == 4 && GQA <= kWaves, "query prep maps 256 threads and one wave per head");
    const float rscale = 1.0f / sqrtf((float)kD);
    const int kr = tid >> 5, dq = tid & 31;
    const int qhead = kvh * GQA + (wave < GQA ? wave : 0);
    const __half *qh = q + ((size_t)z * nh + qhead) * kD;
    const __half q0 = qh[lane], q1 = qh[lane + 64];
    const float sg0 = signs[lane], sg1 = signs[lane + 64];
    // QK-norm + RoPE operands, loaded unconditionally (a branch here would
    // make the compiler wait for them before the loads below issue)
    const __half *qnw = qr.norm ? qr.norm : qh;
    const long rp = imh_qk::clamp_pos(pos_b, qr.max_pos);
    const __half qw0 = qnw[lane], qw1 = qnw[lane + 64];
    const __half qc = qr.cos[rp * (kD / 2) + lane], qsn = qr.sin[rp * (kD / 2) + lane];
    const float kc = kcb[tid & 0x7F], vc = vcb[tid];
    float4 st[16];
    {
        const float4 *s4 = reinterpret_cast<const float4 *>(qjl_t) + (size_t)kr * 16 * (kD / 4) + dq;
#pragma unroll
        for (int i = 0; i < 16; i++) st[i] = s4[(size_t)i * (kD / 4)];
    }
    ChunkIn cur;
    const int p_first = p_begin + wave * kChunk;
    load_chunk(crs, p_first, n_l, kg, cur);
    __builtin_amdgcn_sched_barrier(0);   // every load above issues before the first wait

    // tables: K and V codebooks as f16 hi + lo pairs
    ktab[tid] = tab_entry(kc);
    vtab[tid] = tab_entry(vc);
    // q_rot = D.H.D/sqrt(d) q: wave hh rotates head hh in registers (lane
    // holds elements lane and lane + 64; butterfly strides 1..32 by xor
    // shuffles, stride 64 in the lane) into qs[hh][0]
    if (wave < GQA) {
        float f0 = __half2float(q0), f1 = __half2float(q1);
        if (qr.norm)
            imh_qk::norm_rope_128(f0, f1, __half2float(qw0), __half2float(qw1), __half2float(qc), __half2float(qsn),
                                  qr.eps);
        float x0 = f0 * sg0, x1 = f1 * sg1;
        x0 = hadamard64(x0, lane);
        x1 = hadamard64(x1, lane);
        qs[wave][0][lane] = (x0 + x1) * (sg0 * rscale);
        qs[wave][0][lane + 64] = (x0 - x1) * (sg1 * rscale);
    }
    __syncthreads();
    // its QJL projection s_q[d] = sum_k S[d][k] q_rot[k] into qs[hh][1]:
    // 16-row partial sums, the two of a wave added by a shuffle, the four
    // waves' through LDS (om is free until the loop ends)
    {
        float4 pr[GQA];
#pragma unroll
        for (int hh = 0; hh < GQA; hh++) pr[hh] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int i = 0; i < 16; i++) {
#pragma unroll
            for (int hh = 0; hh < GQA; hh++) {
                const float qv = qs[hh][0][kr * 16 + i];
                pr[hh].x = __builtin_fmaf(st[i].x, qv, pr[hh].x);
                pr[hh].y = __builtin_fmaf(st[i].y, qv, pr[hh].y);
                pr[hh].z = __builtin_fmaf(st[i].z, qv, pr[hh].z);
                pr[hh].w = __builtin_fmaf(st[i].w, qv, pr[hh].w);
            }
        }
#pragma unroll
        for (int hh = 0; hh < GQA; hh++) {
            pr[hh].x += __shfl_xor(pr[hh].x, 32);
            pr[hh].y += __shfl_xor(pr[hh].y, 32);
            pr[hh].z += __shfl_xor(pr[hh].z, 32);
            pr[hh].w += __shfl_xor(pr[hh].w, 32);
            if (lane < 32) reinterpret_cast<float4 *>(&om[wave][hh][0])[dq] = pr[hh];
        }
    }
    __syncthreads();
    for (int e = tid; e < GQA * kD; e += 64 * kWaves) {
        const int hh = e / kD, d = e % kD;
        qs[hh][1][d] = (om[0][hh][d] + om[1][hh][d]) + (om[2][hh][d] + om[3][hh][d]);
    }
    __syncthreads();

    const float qjl_factor = sqrtf(2.0f / 3.14159265f) / (float)kD;
    if constexpr (!FUSED) (void)fz;
    if (FUSED && writer) {
        // ---- the step's token: cache write and its one-position partial ----
        // the lane id again, from mbcnt: values derived from `lane` in the
        // prologue (shuffle addresses) would otherwise be shared with this
        // path and held across the loop's registers
        const int wl = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        const bool has = L_tok > 0;
        const int row = L_tok - 1;
        // thread (kr, dq)'s S^T block again (L2 hits; holding the prologue's
        // copy across the branch would cost the loop registers)
        float4 sw[16];
        {
            const float4 *s4 = reinterpret_cast<const float4 *>(fz.qjl_t) + (size_t)kr * 16 * (kD / 4) + dq;
#pragma unroll
            for (int i = 0; i < 16; i++) sw[i] = s4[(size_t)i * (kD / 4)];
        }
        for (int w = 0; w < 2; w++)
            for (int j = tid; j < fz.n_search[w]; j += 64 * kWaves) {
                wtab[w][j] = fz.sorted[w][j];
                wpm[w][j] = fz.prefmax[w][j];
            }
        float f0 = 0.0f, f1 = 0.0f;
        if (wave < 2 && has) {   // wave 0: K, wave 1: V
            const __half *src = (wave == 0 ? fz.k_new : fz.v_new) + ((size_t)b * nkv + kvh) * kD;
            f0 = __half2float(src[wl]);
            f1 = __half2float(src[wl + 64]);
            if (wave == 0 && fz.k_norm) {
                const long rpk = imh_qk::clamp_pos(row, qr.max_pos);
                imh_qk::norm_rope_128(f0, f1, wl, fz.k_norm, qr.cos + rpk * (kD / 2), qr.sin + rpk * (kD / 2),
                                      qr.eps);
            }
        }
        __syncthreads();   // search tables staged
        TqCodes tc{};
        if (wave < 2 && has) {
            tc = tq_quantize_vec(f0, f1, wl, sg0, sg1, wtab[wave], wpm[wave], fz.n_search[wave],
                                 wave == 0 ? kcb : nullptr);
            if (wave == 0) {
                wres[0][wl] = tc.r0;
                wres[0][wl + 64] = tc.r1;
            }
        }
        __syncthreads();
        // QJL signs of the K residual: s[d] = sum_k S[d][k] r[k] as one fmaf
        // chain per d in increasing k, the cache write's order (bit-exact sign
        // bits).  Thread (kr, dq) holds S^T rows 16 kr .. 16 kr + 15 at columns
        // 4 dq .. 4 dq + 3 in sw[]; row block kr continues the chains of block
        // kr - 1 through LDS.
        for (int blk = 0; blk < 8; blk++) {
            if (kr == blk) {
                float4 a4 = blk == 0 ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                     : reinterpret_cast<const float4 *>(wres[1])[dq];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float rk = wres[0][16 * blk + i];
                    a4.x = __builtin_fmaf(sw[i].x, rk, a4.x);
                    a4.y = __builtin_fmaf(sw[i].y, rk, a4.y);
                    a4.z = __builtin_fmaf(sw[i].z, rk, a4.z);
                    a4.w = __builtin_fmaf(sw[i].w, rk, a4.w);
                }
                reinterpret_cast<float4 *>(wres[1])[dq] = a4;
            }
            __syncthreads();
        }
        const size_t slot = head_base + (size_t)(has ? row : 0);
        if (wave == 0 && has) {
            const uint32_t c0 = tc.c0 | (wres[1][wl] >= 0.0f ? 0x80u : 0u);
            const uint32_t c1 = tc.c1 | (wres[1][wl + 64] >= 0.0f ? 0x80u : 0u);
            fz.kcodes[slot * kD + wl] = (uint8_t)c0;
            fz.kcodes[slot * kD + wl + 64] = (uint8_t)c1;
            if (wl == 0) {
                fz.kscales[slot] = tc.l2;
                fz.krnorm[slot] = tc.rn;
            }
            // each head's score against the dequantized K, the loop's terms
            const float k0 = tab_f32(ktab[c0]), k1 = tab_f32(ktab[c1]);
            const float g0 = (c0 & 0x80u) ? 1.0f : -1.0f, g1 = (c1 & 0x80u) ? 1.0f : -1.0f;
            const float qw = tc.rn * qjl_factor * tc.l2;
#pragma unroll
            for (int hh = 0; hh < GQA; hh++) {
                const float t1 = imh_qk::wave_sum64(__builtin_fmaf(qs[hh][0][wl + 64], k1, qs[hh][0][wl] * k0));
                const float t2 = imh_qk::wave_sum64(__builtin_fmaf(qs[hh][1][wl + 64], g1, qs[hh][1][wl] * g0));
                if (wl == 0) {
                    mm[0][hh] = attn_scale * (t1 * tc.l2 + t2 * qw);
                    ll[0][hh] = 1.0f;
                }
            }
        } else if (wave == 1 && has) {
            fz.vcodes[slot * kD + wl] = (uint8_t)tc.c0;
            fz.vcodes[slot * kD + wl + 64] = (uint8_t)tc.c1;
            if (wl == 0) fz.vscales[slot] = tc.l2;
            // weight 1 at its own maximum: the partial output is the value
            const float v0 = tab_f32(vtab[tc.c0]) * tc.l2, v1 = tab_f32(vtab[tc.c1]) * tc.l2;
#pragma unroll
            for (int hh = 0; hh < GQA; hh++) {
                om[0][hh][wl] = v0;
                om[0][hh][wl + 64] = v1;
            }
        }
        if ((wave != 0 || !has) && wl < GQA) {
            mm[wave][wl] = -INFINITY;
            ll[wave][wl] = 0.0f;
        }
    } else {
        // SPREAD: the spread codebook tables of the loop (their bytes held
        // om's partial sums of the query projection, reduced above)
        using Tab = typename std::conditional<SPREAD, TabSpread, TabOne>::type;
        Tab tab;
        if constexpr (SPREAD) {
            spread_tables(tabs, ktab, vtab, lane, wave);
            __syncthreads();
            tab.t = tabs;
            tab.lk = 4u * (uint32_t)(lane & 31);
            tab.lv = tab.lk + 128u;
        } else {
            tab.kt = ktab;
            tab.vt = vtab;
        }
        // score operands A.  Rows 4h..4h+3 carry head h.  Against the table
        // pairs of word t (k pair i/2 = dim 32 g + 4 t + i/2, hi then lo):
        // aq[t] = {q_hi, q_hi} in row 4h and {q_lo, 0} in row 4h + 1; against
        // the QJL signs of words 2j, 2j + 1 (k-slot order {0, 2, 1, 3} within
        // each word): aqs[j] = s_hi in row 4h + 2, s_lo in row 4h + 3.  Lane
        // group h's four accumulator registers then hold q_hi.K + q_hi.K_lo,
        // q_lo.K_hi (ds) and s_hi.sgn, s_lo.sgn (dg).
        const int am = lane & 15;
        const int ah = am >> 2, ar = am & 3;
        const bool arow = ah < GQA;
        half8_t aq[8], aqs[4];
        const _Float16 z = (_Float16)0.0f;
    #pragma unroll
        for (int t = 0; t < 8; t++) {
    #pragma unroll
            for (int i = 0; i < 4; i++) {
                const float vq = arow ? qs[ah][0][kg * 32 + 4 * t + i] : 0.0f;
                const _Float16 qh = (_Float16)vq;
                const _Float16 ql = (_Float16)(vq - (float)qh);
                aq[t][2 * i] = ar == 0 ? qh : (ar == 1 ? ql : z);
                aq[t][2 * i + 1] = ar == 0 ? qh : z;
            }
        }
        constexpr int slot_byte[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    #pragma unroll
        for (int j = 0; j < 4; j++) {
    #pragma unroll
            for (int i = 0; i < 8; i++) {
                const float vs = arow ? qs[ah][1][kg * 32 + j * 8 + slot_byte[i]] : 0.0f;
                const _Float16 sh = (_Float16)vs;
                const _Float16 sl = (_Float16)(vs - (float)sh);
                aqs[j][i] = ar == 2 ? sh : (ar == 3 ? sl : z);
            }
        }

        float m_run = -INFINITY, l_run = 0.0f;   // of head kg (rows of one DPP row)
        float4_t acc[8];
    #pragma unroll
        for (int j = 0; j < 8; j++) acc[j] = float4_t{0, 0, 0, 0};

        auto process = [&](const ChunkIn &c, const int p0) __attribute__((always_inline)) {
            // ---- scores S[h][n] for 16 positions via MFMA ----
            const uint32_t kw[8] = {c.k0.x, c.k0.y, c.k0.z, c.k0.w, c.k1.x, c.k1.y, c.k1.z, c.k1.w};
            float4_t ds = {0, 0, 0, 0}, dg = {0, 0, 0, 0};
    #pragma unroll
            for (int j = 0; j < 4; j++) {
                ds = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[2 * j], k_pair_operand(kw[2 * j], tab), ds, 0, 0, 0);
                dg = __builtin_amdgcn_mfma_f32_16x16x32_f16(aqs[j], k_sign_operand(&kw[2 * j]), dg, 0, 0, 0);
                ds = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[2 * j + 1], k_pair_operand(kw[2 * j + 1], tab), ds, 0,
                                                           0, 0);
            }
            // lane (n, g): ds[0..1], dg[2..3] = the four partial products of head g at position p0 + n
            const bool valid = (p0 + n_l) < p_end;
            const float qw = c.krn * qjl_factor * c.ksc;
            const float sc = valid ? attn_scale * ((ds[0] + ds[1]) * c.ksc + (dg[2] + dg[3]) * qw) : -INFINITY;
            const float cm = imh_dpp::row16_max_full(sc);
            const float nm = fmaxf(m_run, cm);
            const bool live = nm != -INFINITY;   // a head with no position yet keeps weight 0
            const float corr = live ? __expf(m_run - nm) : 1.0f;
            const float w = live ? __expf(sc - nm) : 0.0f;
            l_run = l_run * corr + imh_dpp::row16_sum_full(w);
            m_run = nm;
            // LAZY: only when some head's maximum grew, which on long splits
            // is rare after the first chunks; on short splits the test and
            // its branch cost more than the eight multiplies they skip
            if (!LAZY || __builtin_amdgcn_ballot_w64(corr != 1.0f)) {
    #pragma unroll
                for (int j = 0; j < 8; j++) acc[j][0] *= corr;
            }
            // weights * v_scale as f16, each twice (against the V entries' hi
            // and lo), transposed through LDS into operand A
            const uint32_t wh = __builtin_bit_cast(uint16_t, (_Float16)(w * c.vsc));
            wbuf[wave][kg][n_l] = wh | (wh << 16);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            half8_t wa = {0, 0, 0, 0, 0, 0, 0, 0};
            if (arow && ar == 0) wa = *reinterpret_cast<const half8_t *>(&wbuf[wave][ah][4 * kg]);
            // ---- o += W . V: operand B of block j = codebook values (hi, lo) of
            // byte j of the four position rows ----
    #pragma unroll
            for (int j = 0; j < 8; j++) {
                const half8_t bv = v_operand(c, j, tab);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, bv, acc[j], 0, 0, 0);
            }
            __builtin_amdgcn_wave_barrier();   // wbuf is rewritten next chunk
        };
        for (int p0 = p_first; p0 < p_end; p0 += kChunk * kWaves) {
            const ChunkIn c = cur;
            load_chunk(crs, p0 + kChunk * kWaves, n_l, kg, cur);
            process(c, p0);
        }
        if constexpr (SPREAD) __syncthreads();   // every wave is done with the tables: om takes their bytes

        // lane (c, g): acc[j][0] = o[head g][dim 8c + j]
        if (kg < GQA) {
            float4 *dst = reinterpret_cast<float4 *>(&om[wave][kg][n_l * 8]);
            dst[0] = make_float4(acc[0][0], acc[1][0], acc[2][0], acc[3][0]);
            dst[1] = make_float4(acc[4][0], acc[5][0], acc[6][0], acc[7][0]);
            if (n_l == 0) {
                mm[wave][kg] = m_run;
                ll[wave][kg] = l_run;
            }
        }
    }
    __syncthreads();
    // combine the waves; with one split normalise here, else publish the
    // split's partial (o unnormalised, running max, sum)
    for (int e = tid; e < GQA * kD; e += 64 * kWaves) {
        const int hh = e / kD, d = e % kD;
        float M = -INFINITY;
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, mm[w][hh]);
        float ov = 0.0f, lv = 0.0f;
        if (M != -INFINITY) {
            for (int w = 0; w < kWaves; w++) {
                if (mm[w][hh] == -INFINITY) continue;
                const float f = __expf(mm[w][hh] - M);
                ov += om[w][hh][d] * f;
                lv += ll[w][hh] * f;
            }
        }
        if (S == 1) {
            qs[hh][0][d] = (ov / fmaxf(lv, 1e-10f)) * signs[d];
        } else {
            // the split's partial; tq_split_combine_kernel merges the splits
            const size_t pidx = ((size_t)z * nh + kvh * GQA + hh) * S + split;
            part_o[pidx * kD + d] = ov;
            if (d == 0) {
                part_m[pidx] = M;
                part_l[pidx] = lv;
            }
        }
    }
    if (S > 1) return;   // uniform: no workgroup barrier follows for these
    __syncthreads();
    // rotate back: o = D.H.D/sqrt(d) o_rot, wave hh on head hh in registers
    // (lane id from mbcnt, so the prologue's shuffle addresses are not held
    // to here across the loop)
    if (wave < GQA) {
        const int ol = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        const float sg0 = signs[ol], sg1 = signs[ol + 64];
        float x0 = qs[wave][0][ol], x1 = qs[wave][0][ol + 64];
        x0 = hadamard64(x0, ol);
        x1 = hadamard64(x1, ol);
        __half *o = out + ((size_t)z * nh + kvh * GQA + wave) * kD;
        o[ol] = __float2half((x0 + x1) * (sg0 * rscale));
        o[ol + 64] = __float2half((x0 - x1) * (sg1 * rscale));
    }
}

// ---------------------------------------------------------------------------
// Attention of a prefill chunk (token_count > 1).  The decode kernel fills the
// 16 rows of its score MFMA with one token's GQA heads times four partial
// products (query hi / lo against codebook hi / lo, QJL hi / lo), and uses 4
// of the 16 rows of its P.V MFMA; it runs once per query token, decoding and
// reading every KV chunk T times.  Here the 16 MFMA rows are 16 / GQA
// consecutive tokens x the GQA heads: a KV chunk's codes are looked up once
// for all of them, the partial products go to separate MFMAs (20 per chunk
// instead of 12 per token), and P.V fills every row.
//   * tq_query_prep_kernel rotates each query row and projects it onto the
//     QJL matrix (the decode prologue's arithmetic, same f32 order) and
//     stores the four f16 operand planes q_hi, q_lo, s_hi, s_lo in MFMA
//     k-slot order;
//   * tq_prefill_attention_kernel<GQA>, one workgroup per (split, kv head,
//     token block of a sequence), keeps a per-row online softmax; each row
//     has its own causal bound (turboquant.metal:268);
//   * with several splits, tq_split_combine_kernel merges the partials
//     (log-sum-exp, fused_sdpa_reduce, flash_decode.metal:163-215) and
//     rotates back; with one, the attention kernel does.
// ---------------------------------------------------------------------------
constexpr int kQPlanes = 4;   // q_hi, q_lo, s_hi, s_lo, kD halfs each

// element p of an operand plane holds dimension (p & ~7) | slot(p & 7): the
// k-slot order {0, 2, 1, 3, 4, 6, 5, 7} of the code-byte unpack (bits 0 and 1
// swapped)
__device__ __forceinline__ int plane_dim(int p) { return (p & ~7) | ((p & 1) << 1) | ((p >> 1) & 1) | (p & 4); }

// grid ceil(rows / 4), block 256: wave w rotates query row 4 blockIdx.x + w
// (rows = batch x tokens x heads, [row][kD] f16), then the workgroup projects
// its four rows and writes their planes ([row][kQPlanes][kD] f16).
__global__ void __launch_bounds__(256) tq_query_prep_kernel(const __half *__restrict__ q, int rows,
                                                            const float *__restrict__ signs,
                                                            const float *__restrict__ qjl_t,
                                                            _Float16 *__restrict__ planes) {
    __shared__ float qs[4][2][kD];
    __shared__ float om[4][4][kD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.x * 4;
    const int kr = tid >> 5, dq = tid & 31;
    const float rscale = 1.0f / sqrtf((float)kD);
    const __half *qh = q + (size_t)min(row0 + wave, rows - 1) * kD;
    const float sg0 = signs[lane], sg1 = signs[lane + 64];
    float x0 = __half2float(qh[lane]) * sg0, x1 = __half2float(qh[lane + 64]) * sg1;
    float4 st[16];
    {
        const float4 *s4 = reinterpret_cast<const float4 *>(qjl_t) + (size_t)kr * 16 * (kD / 4) + dq;
#pragma unroll
        for (int i = 0; i < 16; i++) st[i] = s4[(size_t)i * (kD / 4)];
    }
    x0 = hadamard64(x0, lane);
    x1 = hadamard64(x1, lane);
    qs[wave][0][lane] = (x0 + x1) * (sg0 * rscale);
    qs[wave][0][lane + 64] = (x0 - x1) * (sg1 * rscale);
    __syncthreads();
    float4 pr[4];
#pragma unroll
    for (int hh = 0; hh < 4; hh++) pr[hh] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < 16; i++) {
#pragma unroll
        for (int hh = 0; hh < 4; hh++) {
            const float qv = qs[hh][0][kr * 16 + i];
            pr[hh].x = __builtin_fmaf(st[i].x, qv, pr[hh].x);
            pr[hh].y = __builtin_fmaf(st[i].y, qv, pr[hh].y);
            pr[hh].z = __builtin_fmaf(st[i].z, qv, pr[hh].z);
            pr[hh].w = __builtin_fmaf(st[i].w, qv, pr[hh].w);
        }
    }
#pragma unroll
    for (int hh = 0; hh < 4; hh++) {
        pr[hh].x += __shfl_xor(pr[hh].x, 32);
        pr[hh].y += __shfl_xor(pr[hh].y, 32);
        pr[hh].z += __shfl_xor(pr[hh].z, 32);
        pr[hh].w += __shfl_xor(pr[hh].w, 32);
        if (lane < 32) reinterpret_cast<float4 *>(&om[wave][hh][0])[dq] = pr[hh];
    }
    __syncthreads();
    for (int e = tid; e < 4 * kD; e += 256) {
        const int hh = e / kD, d = e % kD;
        qs[hh][1][d] = (om[0][hh][d] + om[1][hh][d]) + (om[2][hh][d] + om[3][hh][d]);
    }
    __syncthreads();
    for (int e = tid; e < 4 * kD; e += 256) {
        const int hh = e / kD, p = e % kD;
        if (row0 + hh >= rows) continue;
        const int d = plane_dim(p);
        const float vq = qs[hh][0][d], vs = qs[hh][1][d];
        const _Float16 qhi = (_Float16)vq, shi = (_Float16)vs;
        _Float16 *dst = planes + (size_t)(row0 + hh) * kQPlanes * kD + p;
        dst[0] = qhi;
        dst[kD] = (_Float16)(vq - (float)qhi);
        dst[2 * kD] = shi;
        dst[3 * kD] = (_Float16)(vs - (float)shi);
    }
}

// grid (S, nkv, batch x ceil(T / TB)), block 256; TB = 16 / GQA tokens per
// workgroup.  MFMA row r = TB-local token r / GQA, head r % GQA; lane (n, g)
// holds output rows 4 g .. 4 g + 3 at column n.
template <int GQA>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2))) tq_prefill_attention_kernel(
    const _Float16 *__restrict__ planes, int nh, int nkv, int max_seq, int seq_len, int T,
    const int32_t *__restrict__ seq_lens, float attn_scale, const float *__restrict__ signs,
    const float *__restrict__ kcb, const float *__restrict__ vcb, const uint8_t *__restrict__ kcodes,
    const uint8_t *__restrict__ vcodes, const float *__restrict__ kscales, const float *__restrict__ vscales,
    const float *__restrict__ krnorm, int split_len, float *__restrict__ part_o, float *__restrict__ part_m,
    float *__restrict__ part_l, __half *__restrict__ out) {
    constexpr int TB = 16 / GQA;
    __shared__ uint32_t ktab[256];
    __shared__ uint32_t vtab[256];
    __shared__ _Float16 wbuf[kWaves][16][16];
    // the spread codebook tables of the loop; the waves' partial outputs om
    // take the same bytes after it
    __shared__ __attribute__((aligned(16))) uint8_t tabs[kTabBytes];
    float(*om)[16][kD] = reinterpret_cast<float(*)[16][kD]>(tabs);
    __shared__ float mm[kWaves][16];
    __shared__ float ll[kWaves][16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int S = gridDim.x, split = blockIdx.x, kvh = blockIdx.y;
    const int ntb = (T + TB - 1) / TB;
    const int b = blockIdx.z / ntb;
    const int t0 = (blockIdx.z - b * ntb) * TB;
    int L = seq_lens ? min(seq_lens[b], seq_len) : seq_len;
    L = L < 0 ? 0 : (L > max_seq ? max_seq : L);
    // token t sees positions < L - T + t + 1 (turboquant.metal:268)
    auto bound = [&](int r) {
        const int t = t0 + r / GQA;
        return t < T ? max(0, L - (T - 1 - t)) : 0;
    };
    const int Lmax = max(0, L - (T - min(t0 + TB, T)));
    const int p_begin = split * split_len;
    const int p_end = min(p_begin + split_len, Lmax);
    const size_t head_base = ((size_t)b * nkv + kvh) * (size_t)max_seq;
    const int n_l = lane & 15;
    const int kg = lane >> 4;
    const ChunkRsrc crs = chunk_rsrc(kcodes, vcodes, kscales, krnorm, vscales, head_base, p_end > 0 ? p_end : 0);

    // operands A: row am = lane & 15, k-slice j = the 8 halfs at plane
    // offset 32 g + 8 j (rows past the chunk's tokens repeat the last one and
    // are masked)
    const int am = lane & 15;
    const int at = min(t0 + am / GQA, T - 1);
    const _Float16 *pa =
        planes + (((size_t)b * T + at) * nh + kvh * GQA + am % GQA) * (kQPlanes * kD) + kg * 32;
    half8_t aqh[4], aql[4], ash[4], asl[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        aqh[j] = *reinterpret_cast<const half8_t *>(pa + 8 * j);
        aql[j] = *reinterpret_cast<const half8_t *>(pa + kD + 8 * j);
        ash[j] = *reinterpret_cast<const half8_t *>(pa + 2 * kD + 8 * j);
        asl[j] = *reinterpret_cast<const half8_t *>(pa + 3 * kD + 8 * j);
    }
    const float kc = kcb[tid & 0x7F], vc = vcb[tid];
    ChunkIn cur, nxt;
    const int p_first = p_begin + wave * kChunk;
    load_chunk(crs, p_first, n_l, kg, cur);
    __builtin_amdgcn_sched_barrier(0);   // every load above issues before the first wait
    ktab[tid] = tab_entry(kc);
    vtab[tid] = tab_entry(vc);
    int bnd[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) bnd[rr] = min(bound(4 * kg + rr), p_end);
    __syncthreads();
    spread_tables(tabs, ktab, vtab, lane, wave);
    __syncthreads();
    TabSpread tab;
    tab.t = tabs;
    tab.lk = 4u * (uint32_t)(lane & 31);
    tab.lv = tab.lk + 128u;

    // scores in log2 units (attn_scale * log2(e) folded into the per-position
    // scales): the softmax exponentials are single exp2s
    const float sl2 = attn_scale * 1.44269504f;
    const float qf2 = sqrtf(2.0f / 3.14159265f) / (float)kD * sl2;
    // per row: the running maximum (uniform over the row's 16 lanes) and this
    // lane's share of the running sum (the row's sum is reduced once, after
    // the loop: every lane of a row rescales by the same factor)
    float m_run[4], l_run[4];
    float4_t acc[8];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
        m_run[rr] = -INFINITY;
        l_run[rr] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = float4_t{0, 0, 0, 0};

    auto process = [&](const ChunkIn &c, const int p0) __attribute__((always_inline)) {
        // ---- scores of 16 rows x 16 positions ----
        const uint32_t kw[8] = {c.k0.x, c.k0.y, c.k0.z, c.k0.w, c.k1.x, c.k1.y, c.k1.z, c.k1.w};
        float4_t dq = {0, 0, 0, 0}, ds = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            half8_t Bh, Bl, Bs;
            k_operands(&kw[2 * j], tab, Bh, Bl, Bs);
            dq = __builtin_amdgcn_mfma_f32_16x16x32_f16(aqh[j], Bh, dq, 0, 0, 0);
            ds = __builtin_amdgcn_mfma_f32_16x16x32_f16(ash[j], Bs, ds, 0, 0, 0);
            dq = __builtin_amdgcn_mfma_f32_16x16x32_f16(aqh[j], Bl, dq, 0, 0, 0);
            ds = __builtin_amdgcn_mfma_f32_16x16x32_f16(asl[j], Bs, ds, 0, 0, 0);
            dq = __builtin_amdgcn_mfma_f32_16x16x32_f16(aql[j], Bh, dq, 0, 0, 0);
        }
        const float ks2 = c.ksc * sl2;
        const float qw2 = c.krn * qf2 * c.ksc;
        float corr[4];
        bool grew = false;
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const bool valid = (p0 + n_l) < bnd[rr];
            const float sc = valid ? __builtin_fmaf(dq[rr], ks2, ds[rr] * qw2) : -INFINITY;
            const float nm = fmaxf(m_run[rr], imh_dpp::row16_max(sc));
            const bool live = nm != -INFINITY;   // a row with no position yet keeps weight 0
            corr[rr] = live ? __builtin_amdgcn_exp2f(m_run[rr] - nm) : 1.0f;
            const float w = live ? __builtin_amdgcn_exp2f(sc - nm) : 0.0f;
            l_run[rr] = __builtin_fmaf(l_run[rr], corr[rr], w);
            m_run[rr] = nm;
            grew |= corr[rr] != 1.0f;
            wbuf[wave][4 * kg + rr][n_l] = (_Float16)(w * c.vsc);
        }
        if (__builtin_amdgcn_ballot_w64(grew)) {   // some row's max grew
#pragma unroll
            for (int j = 0; j < 8; j++)
#pragma unroll
                for (int rr = 0; rr < 4; rr++) acc[j][rr] *= corr[rr];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // operand A of P.V: row am's weights at positions 4 g .. 4 g + 3, each
        // twice (against the V entries' hi and lo halves)
        const half4_t w4 = *reinterpret_cast<const half4_t *>(&wbuf[wave][am][4 * kg]);
        const half8_t wa = {w4[0], w4[0], w4[1], w4[1], w4[2], w4[2], w4[3], w4[3]};
#pragma unroll
        for (int j = 0; j < 8; j++)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, v_operand(c, j, tab), acc[j], 0, 0, 0);
        __builtin_amdgcn_wave_barrier();   // wbuf is rewritten next chunk
    };
    // two chunk register sets in turn (no copies): the next chunk's loads are
    // in flight while one is processed
    constexpr int kStep = kChunk * kWaves;
    for (int p0 = p_first; p0 < p_end; p0 += 2 * kStep) {
        load_chunk(crs, p0 + kStep, n_l, kg, nxt);
        process(cur, p0);
        if (p0 + kStep >= p_end) break;
        load_chunk(crs, p0 + 2 * kStep, n_l, kg, cur);
        process(nxt, p0 + kStep);
    }
#pragma unroll
    for (int rr = 0; rr < 4; rr++) l_run[rr] = imh_dpp::row16_sum(l_run[rr]);
    __syncthreads();   // every wave is done with the tables: om takes their bytes

    // lane (c, g): acc[j][rr] = o[row 4 g + rr][dim 8 c + j]
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
        float4 *dst = reinterpret_cast<float4 *>(&om[wave][4 * kg + rr][n_l * 8]);
        dst[0] = make_float4(acc[0][rr], acc[1][rr], acc[2][rr], acc[3][rr]);
        dst[1] = make_float4(acc[4][rr], acc[5][rr], acc[6][rr], acc[7][rr]);
        if (n_l == 0) {
            mm[wave][4 * kg + rr] = m_run[rr];
            ll[wave][4 * kg + rr] = l_run[rr];
        }
    }
    __syncthreads();
    // combine the waves (maxima in log2 units); with one split normalise (in
    // place: element (r, d) of om[0] is read and written by one thread), else
    // publish the partial
    for (int e = tid; e < 16 * kD; e += 64 * kWaves) {
        const int r = e / kD, d = e % kD;
        float M = -INFINITY;
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, mm[w][r]);
        float ov = 0.0f, lv = 0.0f;
        if (M != -INFINITY) {
            for (int w = 0; w < kWaves; w++) {
                if (mm[w][r] == -INFINITY) continue;
                const float f = __builtin_amdgcn_exp2f(mm[w][r] - M);
                ov += om[w][r][d] * f;
                lv += ll[w][r] * f;
            }
        }
        if (S == 1) {
            om[0][r][d] = (ov / fmaxf(lv, 1e-10f)) * signs[d];
        } else if (t0 + r / GQA < T) {
            const size_t pidx = (((size_t)b * T + t0 + r / GQA) * nh + kvh * GQA + r % GQA) * S + split;
            part_o[pidx * kD + d] = ov;
            if (d == 0) {
                part_m[pidx] = M;
                part_l[pidx] = lv;
            }
        }
    }
    if (S > 1) return;
    __syncthreads();
    // rotate back: o = D.H.D/sqrt(d) o_rot, wave w on rows w, w + 4, ..
    const float rscale = 1.0f / sqrtf((float)kD);
    const float sg0 = signs[lane], sg1 = signs[lane + 64];
    for (int r = wave; r < 16; r += kWaves) {
        const int t = t0 + r / GQA;
        if (t >= T) break;   // rows grow with t
        float x0 = om[0][r][lane], x1 = om[0][r][lane + 64];
        x0 = hadamard64(x0, lane);
        x1 = hadamard64(x1, lane);
        __half *o = out + (((size_t)b * T + t) * nh + kvh * GQA + r % GQA) * kD;
        o[lane] = __float2half((x0 + x1) * (sg0 * rscale));
        o[lane + 64] = __float2half((x0 - x1) * (sg1 * rscale));
    }
}

// grid rows, block 256: one workgroup merges the S split partials of its row
// ([row][S] maxima -- in log2 units for the prefill kernel, natural for the
// decode kernel -- and sums, [row][S][kD] outputs) and rotates the result
// back into out[row].  Split s weighs exp(m_s - M); wave w sums the splits
// w, w + 4, .. (the first sixteen of them loaded together with the maxima), the
// four partial sums are added in wave order through LDS, and wave 0
// normalises and rotates.
template <bool LOG2>
__global__ void __launch_bounds__(256) tq_split_combine_kernel(const float *__restrict__ part_o,
                                                               const float *__restrict__ part_m,
                                                               const float *__restrict__ part_l, int rows, int S,
                                                               const float *__restrict__ signs,
                                                               __half *__restrict__ out) {
    __shared__ float osum[4][kD];
    __shared__ float lsums[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = blockIdx.x;
    const float *pm = part_m + (size_t)row * S;
    const float *pl = part_l + (size_t)row * S;
    const float *po = part_o + (size_t)row * S * kD;
    // the maxima for the row maximum, then the wave's first kR splits (every
    // load issued before the first wait: one memory latency for S <= 4 kR)
    constexpr int kR = 16;
    float mx = pm[lane < S ? lane : 0];
    mx = lane < S ? mx : -INFINITY;
    float mv[kR], lv[kR], ov0[kR], ov1[kR];
#pragma unroll
    for (int i = 0; i < kR; i++) {
        const int sp = min(wave + 4 * i, S - 1);
        mv[i] = pm[sp];
        lv[i] = pl[sp];
        ov0[i] = po[(size_t)sp * kD + lane];
        ov1[i] = po[(size_t)sp * kD + lane + 64];
    }
    for (int sp = lane + 64; sp < S; sp += 64) mx = fmaxf(mx, pm[sp]);
#pragma unroll
    for (int st = 32; st >= 1; st >>= 1) mx = fmaxf(mx, __shfl_xor(mx, st));
    float o0 = 0.0f, o1 = 0.0f, ls = 0.0f;
    auto add = [&](float m, float l, float a0, float a1) __attribute__((always_inline)) {
        const float f = (mx == -INFINITY || m == -INFINITY) ? 0.0f
                                                            : (LOG2 ? __builtin_amdgcn_exp2f(m - mx) : __expf(m - mx));
        ls = __builtin_fmaf(f, l, ls);
        o0 = __builtin_fmaf(a0, f, o0);
        o1 = __builtin_fmaf(a1, f, o1);
    };
    // splits in the order wave, wave + 4, .. (the sums' order does not depend
    // on how the loads were batched)
#pragma unroll
    for (int i = 0; i < kR; i++)
        if (wave + 4 * i < S) add(mv[i], lv[i], ov0[i], ov1[i]);
#pragma unroll 4
    for (int sp = wave + 4 * kR; sp < S; sp += 4)
        add(pm[sp], pl[sp], po[(size_t)sp * kD + lane], po[(size_t)sp * kD + lane + 64]);
    osum[wave][lane] = o0;
    osum[wave][lane + 64] = o1;
    if (lane == 0) lsums[wave] = ls;
    __syncthreads();
    if (wave != 0) return;
    o0 = ((osum[0][lane] + osum[1][lane]) + osum[2][lane]) + osum[3][lane];
    o1 = ((osum[0][lane + 64] + osum[1][lane + 64]) + osum[2][lane + 64]) + osum[3][lane + 64];
    const float lsum = ((lsums[0] + lsums[1]) + lsums[2]) + lsums[3];
    const float inv = 1.0f / fmaxf(lsum, 1e-10f);
    const float sg0 = signs[lane], sg1 = signs[lane + 64];
    float x0 = o0 * inv * sg0, x1 = o1 * inv * sg1;
    x0 = hadamard64(x0, lane);
    x1 = hadamard64(x1, lane);
    const float rscale = 1.0f / sqrtf((float)kD);
    out[(size_t)row * kD + lane] = __float2half((x0 + x1) * (sg0 * rscale));
    out[(size_t)row * kD + lane + 64] = __float2half((x0 - x1) * (sg1 * rscale));
}

int check_cache(const imh_tq_tables *t, const imh_tq_kv_cache *c, const char *who) {
    if (!t || !c) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL tables or cache");
    if (!c->k_codes || !c->v_codes || !c->k_scales || !c->v_scales || !c->k_r_norms)
        return imh::fail(IMH_EINVAL, std::string(who) + ": a cache array is NULL");
    if (c->head_dim != t->head_dim)
        return imh::fail(IMH_EINVAL, std::string(who) + ": cache head_dim differs from the tables'");
    if (c->head_dim != kD)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": kernels are built for head_dim 128");
    if (c->batch == 0 || c->num_kv_heads == 0 || c->max_seq_len == 0)
        return imh::fail(IMH_EINVAL, std::string(who) + ": empty cache shape");
    if ((reinterpret_cast<uintptr_t>(c->k_codes) | reinterpret_cast<uintptr_t>(c->v_codes)) & 15)
        return imh::fail(IMH_EINVAL, std::string(who) + ": code arrays must be 16-byte aligned");
    return IMH_OK;
}

}  // namespace

extern "C" {

static int launch_cache_write(imh_stream *stream, const imh_tq_tables *t, const imh_tq_kv_cache *cache,
                              const uint16_t *k_proj, const uint16_t *v_proj, uint32_t token_count,
                              uint32_t base_pos, const int32_t *positions, const char *who) {
    int rc = check_cache(t, cache, who);
    if (rc) return rc;
    if (token_count == 0) return IMH_OK;
    rc = imh::use_device(stream->dev);
    if (rc) return rc;
    TqWriteArgs a{};
    a.kv[0] = reinterpret_cast<const __half *>(k_proj);
    a.kv[1] = reinterpret_cast<const __half *>(v_proj);
    a.codes[0] = cache->k_codes;
    a.codes[1] = cache->v_codes;
    a.scales[0] = cache->k_scales;
    a.scales[1] = cache->v_scales;
    a.r_norms = cache->k_r_norms;
    a.codebook[0] = t->k_codebook;
    a.codebook[1] = t->v_codebook;
    a.sorted[0] = t->k_sorted;
    a.sorted[1] = t->v_sorted;
    a.prefmax[0] = t->k_prefmax;
    a.prefmax[1] = t->v_prefmax;
    a.n_search[0] = t->k_search;
    a.n_search[1] = t->v_search;
    const int first = k_proj ? 0 : 1;
    const int count = (k_proj ? 1 : 0) + (v_proj ? 1 : 0);
    const int waves = (int)std::min<uint32_t>(kWriteMaxWaves, cache->num_kv_heads * count);
    if (cache->batch > 65535) return imh::fail(IMH_EINVAL, std::string(who) + ": batch above 65535");
    dim3 grid(token_count, cache->batch);
    hipLaunchKernelGGL(tq_cache_write_kernel, grid, dim3(64 * waves), 0, stream->stream, a, first, count,
                       (int)token_count, (int)cache->num_kv_heads, (int)cache->max_seq_len, (int)base_pos,
                       positions, t->signs, t->qjl_t);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

int imh_encode_turboquant_cache_write(imh_stream *stream, const imh_tq_tables *t,
                                      const imh_tq_kv_cache *cache, const uint16_t *kv_proj,
                                      uint32_t token_count, uint32_t base_pos,
                                      const int32_t *positions, int is_k) {
    const char *who = "imh_encode_turboquant_cache_write";
    if (!stream || !kv_proj) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    return launch_cache_write(stream, t, cache, is_k ? kv_proj : nullptr, is_k ? nullptr : kv_proj, token_count,
                              base_pos, positions, who);
}

int imh_encode_turboquant_cache_write_kv(imh_stream *stream, const imh_tq_tables *t,
                                         const imh_tq_kv_cache *cache, const uint16_t *k_proj,
                                         const uint16_t *v_proj, uint32_t token_count, uint32_t base_pos,
                                         const int32_t *positions) {
    const char *who = "imh_encode_turboquant_cache_write_kv";
    if (!stream || !k_proj || !v_proj) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    return launch_cache_write(stream, t, cache, k_proj, v_proj, token_count, base_pos, positions, who);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Fixed scratch of imh_encode_turboquant_attention_noalloc: split partials
// (o, max, sum per query row, head and split), in one device array per GPU,
// held until the process ends.  Host
// code never passes the array's name to a kernel (on the host it is only a
// stand-in); it uses the address hipGetSymbolAddress returns for the current
// device, looked up once per device when the device is opened.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocPartBytes = size_t(4) << 20;   // partials
static __device__ __align__(256) uint8_t scratch[kNoAllocPartBytes];

constexpr int kMaxDevices = 64;
static void *g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

namespace imh {

int noalloc_scratch_init(int ordinal) {
    if (ordinal < 0 || ordinal >= kMaxDevices)
        return fail(IMH_EUNSUPPORTED, "device ordinal above the library's limit of 64");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[ordinal]) return IMH_OK;
    int cur = -1;
    IMH_HIP(hipGetDevice(&cur));
    if (cur != ordinal) IMH_HIP(hipSetDevice(ordinal));
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(IMH_EDEVICE, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[ordinal] = ptr;
    return IMH_OK;
}

}  // namespace imh

extern "C" {

// token_count > 1: query prep, the token-block kernel and, with several
// splits, the combine.  Splits as for decode (~512 workgroups, none shorter
// than 256 positions unless num_splits asks), over the longest causal range.
static int run_prefill_attention(imh_stream *stream, const imh_tq_tables *t, const imh_tq_kv_cache *cache,
                                 const uint16_t *q, uint32_t num_heads, uint32_t gqa, uint32_t L,
                                 const int32_t *seq_lens, float attn_scale, uint16_t *out,
                                 uint32_t num_splits, uint32_t T, const char *who) {
    const uint32_t nkv = cache->num_kv_heads;
    const uint32_t TB = 16 / gqa;
    const uint32_t ntb = (T + TB - 1) / TB;
    if ((uint64_t)cache->batch * ntb > 65535)
        return imh::fail(IMH_EINVAL, std::string(who) + ": batch x token blocks above 65535");
    const size_t rows = (size_t)cache->batch * T * num_heads;
    if (rows > (size_t)INT32_MAX / 4)
        return imh::fail(IMH_EINVAL, std::string(who) + ": batch x token_count x num_heads too large");
    uint32_t want = num_splits;
    if (want == 0) {
        const uint32_t groups = cache->batch * ntb * nkv;
        want = std::min<uint32_t>((512 + groups - 1) / groups, std::max<uint32_t>(1, L / kAutoSplitLen));
    }
    const uint32_t max_splits = std::max<uint32_t>(1, (L + kSplitQuantum - 1) / kSplitQuantum);
    want = std::max<uint32_t>(1, std::min(want, std::min<uint32_t>(max_splits, kMaxSplits)));
    uint32_t split_len = (L + want - 1) / want;
    split_len = std::max<uint32_t>(kSplitQuantum, (split_len + kSplitQuantum - 1) / kSplitQuantum * kSplitQuantum);
    const uint32_t S = std::max<uint32_t>(1, (L + split_len - 1) / split_len);

    void *pl_scr = nullptr, *part = nullptr;
    int rc = imh::stream_scratch(stream, 0, rows * kQPlanes * kD * sizeof(_Float16), &pl_scr);
    if (rc) return rc;
    float *po = nullptr, *pm = nullptr, *pls = nullptr;
    if (S > 1) {
        rc = imh::stream_scratch(stream, 1, rows * S * (kD + 2) * sizeof(float), &part);
        if (rc) return rc;
        po = static_cast<float *>(part);
        pm = po + rows * S * kD;
        pls = pm + rows * S;
    }
    _Float16 *planes = static_cast<_Float16 *>(pl_scr);
    const unsigned qblocks = (unsigned)((rows + 3) / 4);
    hipLaunchKernelGGL(tq_query_prep_kernel, dim3(qblocks), dim3(256), 0, stream->stream,
                       reinterpret_cast<const __half *>(q), (int)rows, t->signs, t->qjl_t, planes);
    IMH_HIP(hipGetLastError());
    dim3 grid(S, nkv, cache->batch * ntb);
#define IMH_TQ_PREFILL(G)                                                                                       \
    hipLaunchKernelGGL((tq_prefill_attention_kernel<G>), grid, dim3(64 * kWaves), 0, stream->stream, planes,      \
                       (int)num_heads, (int)nkv, (int)cache->max_seq_len, (int)L, (int)T, seq_lens, attn_scale,   \
                       t->signs, t->k_codebook, t->v_codebook, cache->k_codes, cache->v_codes, cache->k_scales,   \
                       cache->v_scales, cache->k_r_norms, (int)split_len, po, pm, pls,                           \
                       reinterpret_cast<__half *>(out))
    if (gqa == 4) IMH_TQ_PREFILL(4);
    else if (gqa == 2) IMH_TQ_PREFILL(2);
    else IMH_TQ_PREFILL(1);
#undef IMH_TQ_PREFILL
    IMH_HIP(hipGetLastError());
    if (S > 1) {
        hipLaunchKernelGGL(tq_split_combine_kernel<true>, dim3((unsigned)rows), dim3(256), 0, stream->stream, po, pm, pls,
                           (int)rows, (int)S, t->signs, reinterpret_cast<__half *>(out));
        IMH_HIP(hipGetLastError());
    }
    return IMH_OK;
}

// fixed_scratch: the no-alloc entry point's per-device array (NULL: the
// stream's scratch slots, grown on demand)
static int run_attention(imh_stream *stream, const imh_tq_tables *t, const imh_tq_kv_cache *cache,
                         const uint16_t *q, uint32_t num_heads, uint32_t seq_len, const int32_t *seq_lens,
                         float attn_scale, uint16_t *out, uint32_t num_splits, const char *who,
                         const imh_qk_norm_rope_params *qk, const uint16_t *k_new = nullptr,
                         const uint16_t *v_new = nullptr, uint32_t token_count = 1,
                         void *fixed_scratch = nullptr) {
    if (!stream || !q || !out) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    const bool fused = k_new != nullptr;   // the token's cache write in the same launch
    int rc = check_cache(t, cache, who);
    if (rc) return rc;
    const uint32_t nkv = cache->num_kv_heads;
    if (num_heads == 0 || num_heads % nkv != 0)
        return imh::fail(IMH_EINVAL, std::string(who) + ": num_heads must be a multiple of num_kv_heads");
    const uint32_t gqa = num_heads / nkv;
    if (gqa != 1 && gqa != 2 && gqa != 4)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": GQA group of " + std::to_string(gqa) +
                                               " heads not built (1, 2, 4)");
    if (seq_len > cache->max_seq_len)
        return imh::fail(IMH_ERANGE, std::string(who) + ": seq_len " + std::to_string(seq_len) +
                                         " exceeds max_seq_len " + std::to_string(cache->max_seq_len));
    rc = imh::use_device(stream->dev);
    if (rc) return rc;

    // KV split: by default ~512 workgroups, but no split shorter than 256
    // positions (the combining workgroup's work grows with the split count;
    // measured best at ctx 8k and 32k, batch 1 to 16).  Explicit num_splits
    // may go down to 64 positions per split.  With per-sequence lengths the
    // splits span the bound (0 = max_seq_len).
    const uint32_t L = seq_lens && seq_len == 0 ? cache->max_seq_len : seq_len;
    if (token_count == 0 || (token_count > 1 && (fused || qk)))
        return imh::fail(IMH_EINVAL, std::string(who) + ": token_count must be 1 with the cache write or "
                                                         "QK-norm, and at least 1");
    if (token_count > 1)
        return run_prefill_attention(stream, t, cache, q, num_heads, gqa, L, seq_lens, attn_scale, out,
                                     num_splits, token_count, who);
    // query rows: token t of sequence b is row b * token_count + t
    const uint32_t B = cache->batch * token_count;
    if (B > 65535) return imh::fail(IMH_EINVAL, std::string(who) + ": batch x token_count above 65535");
    uint32_t want = num_splits;
    if (want == 0) {
        const uint32_t groups = B * nkv;
        want = std::min<uint32_t>((512 + groups - 1) / groups, std::max<uint32_t>(1, L / kAutoSplitLen));
    }
    const uint32_t max_splits = std::max<uint32_t>(1, (L + kSplitQuantum - 1) / kSplitQuantum);
    want = std::max<uint32_t>(1, std::min(want, std::min<uint32_t>(max_splits, kMaxSplits - (fused ? 1 : 0))));
    uint32_t split_len = (L + want - 1) / want;
    split_len = std::max<uint32_t>(kSplitQuantum,
                                   (split_len + kSplitQuantum - 1) / kSplitQuantum * kSplitQuantum);
    // <= kMaxSplits, with the token writer's split
    const uint32_t S = std::max<uint32_t>(1, (L + split_len - 1) / split_len) + (fused ? 1 : 0);

    // scratch: split partials (none for one split); every workgroup of the
    // attention writes its own, so the fixed array's leftover contents never
    // reach the combine
    const size_t nparts = (size_t)B * num_heads * S;
    float *po = nullptr, *pm = nullptr, *pl = nullptr;
    if (S > 1) {
        void *scr = nullptr;
        const size_t part_bytes = nparts * kD * 4 + nparts * 8 + 512;
        if (fixed_scratch) {
            if (part_bytes > kNoAllocPartBytes)
                return imh::fail(IMH_EINVAL,
                                 std::string(who) + ": needs " + std::to_string(part_bytes) + " bytes of split "
                                 "partials; the fixed scratch holds " + std::to_string(kNoAllocPartBytes) +
                                 " bytes (fewer num_splits or a smaller batch fit)");
            scr = fixed_scratch;
        } else {
            rc = imh::stream_scratch(stream, 1, part_bytes, &scr);
            if (rc) return rc;
        }
        po = static_cast<float *>(scr);
        pm = po + nparts * kD;
        pl = pm + nparts;
    }
    const __half *qh = reinterpret_cast<const __half *>(q);
    dim3 grid(S, nkv, B);
#define IMH_TQ_LAUNCH(G, F, SP, LZ)                                                                            \
    hipLaunchKernelGGL((tq_attention_kernel<G, F, SP, LZ>), grid, dim3(64 * kWaves), 0, stream->stream, qh, (int)num_heads, \
                       (int)nkv, (int)cache->max_seq_len, (int)L, (int)token_count, seq_lens, attn_scale,       \
                       t->signs, t->qjl_t,                                                                      \
                       t->k_codebook, t->v_codebook, cache->k_codes, cache->v_codes, cache->k_scales,           \
                       cache->v_scales, cache->k_r_norms, (int)split_len, po, pm, pl,                           \
                       reinterpret_cast<__half *>(out), qr, fz)
    // without the QK-norm the kernel still reads (and discards) one position
    // and 64 table entries: point them at the codebook
    QkRope qr{nullptr, reinterpret_cast<const __half *>(t->v_codebook),
              reinterpret_cast<const __half *>(t->v_codebook), reinterpret_cast<const int32_t *>(t->v_codebook), 1,
              0.0f};
    if (qk) {   // the query through the QK-norm + RoPE first
        qr.norm = reinterpret_cast<const __half *>(qk->q_norm);
        qr.cos = reinterpret_cast<const __half *>(qk->cos_cache);
        qr.sin = reinterpret_cast<const __half *>(qk->sin_cache);
        qr.positions = qk->positions;
        qr.max_pos = (int)qk->max_pos;
        qr.eps = qk->eps;
    }
    TqFuse fz{};
    if (fused) {
        fz.k_new = reinterpret_cast<const __half *>(k_new);
        fz.v_new = reinterpret_cast<const __half *>(v_new);
        fz.kcodes = cache->k_codes;
        fz.vcodes = cache->v_codes;
        fz.kscales = cache->k_scales;
        fz.vscales = cache->v_scales;
        fz.krnorm = cache->k_r_norms;
        fz.sorted[0] = t->k_sorted;
        fz.sorted[1] = t->v_sorted;
        fz.prefmax[0] = t->k_prefmax;
        fz.prefmax[1] = t->v_prefmax;
        fz.n_search[0] = t->k_search;
        fz.n_search[1] = t->v_search;
        fz.k_norm = qk ? reinterpret_cast<const __half *>(qk->k_norm) : nullptr;
        fz.qjl_t = t->qjl_t;
    }
    // bank-spread tables from kSpreadMinLen positions per split (building
    // them costs more than their lookups save on short splits); not with the
    // token writers, whose workgroups would hold the tables' 64 KB of LDS too
    // and no longer fit beside two streaming workgroups per CU
    const bool spread = !fused && split_len >= kSpreadMinLen;
    // lazy rescale from kLazyMinLen positions per split (decode at batch 8,
    // ctx 8k: 3.51 -> 3.34 ms per step; at batch 1, ~5 chunks per wave, the
    // eager rescale is faster: 1.74 -> 1.72 ms); the spread instantiation
    // always has long splits
    static_assert(kLazyMinLen == kSpreadMinLen, "non-fused: lazy exactly when spread");
    const bool lazy = split_len >= kLazyMinLen;
    if (fused && lazy) {   // the writer workgroups only in these instantiations
        if (gqa == 4) IMH_TQ_LAUNCH(4, true, false, true);
        else if (gqa == 2) IMH_TQ_LAUNCH(2, true, false, true);
        else IMH_TQ_LAUNCH(1, true, false, true);
    } else if (fused) {
        if (gqa == 4) IMH_TQ_LAUNCH(4, true, false, false);
        else if (gqa == 2) IMH_TQ_LAUNCH(2, true, false, false);
        else IMH_TQ_LAUNCH(1, true, false, false);
    } else if (spread) {
        if (gqa == 4) IMH_TQ_LAUNCH(4, false, true, true);
        else if (gqa == 2) IMH_TQ_LAUNCH(2, false, true, true);
        else IMH_TQ_LAUNCH(1, false, true, true);
    } else {
        if (gqa == 4) IMH_TQ_LAUNCH(4, false, false, false);
        else if (gqa == 2) IMH_TQ_LAUNCH(2, false, false, false);
        else IMH_TQ_LAUNCH(1, false, false, false);
    }
#undef IMH_TQ_LAUNCH
    IMH_HIP(hipGetLastError());
    if (S > 1) {   // the splits' merge, in stream order after every partial
        const int rows = (int)(B * num_heads);
        hipLaunchKernelGGL(tq_split_combine_kernel<false>, dim3((unsigned)rows), dim3(256), 0, stream->stream, po, pm,
                           pl, rows, (int)S, t->signs, reinterpret_cast<__half *>(out));
        IMH_HIP(hipGetLastError());
    }
    return IMH_OK;
}

int imh_encode_turboquant_attention(imh_stream *stream, const imh_tq_tables *t,
                                    const imh_tq_kv_cache *cache, const uint16_t *q,
                                    uint32_t num_heads, uint32_t seq_len, const int32_t *seq_lens,
                                    float attn_scale, uint16_t *out, uint32_t num_splits) {
    return run_attention(stream, t, cache, q, num_heads, seq_len, seq_lens, attn_scale, out, num_splits,
                         "imh_encode_turboquant_attention", nullptr);
}

int imh_encode_turboquant_attention_noalloc(imh_stream *stream, const imh_tq_tables *t,
                                            const imh_tq_kv_cache *cache, const uint16_t *q,
                                            uint32_t num_heads, uint32_t seq_len, const int32_t *seq_lens,
                                            float attn_scale, uint16_t *out, uint32_t num_splits) {
    const char *who = "imh_encode_turboquant_attention_noalloc";
    if (!stream) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL stream");
    const int ord = stream->dev->ordinal;
    void *ptr = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        ptr = (ord >= 0 && ord < kMaxDevices) ? g_scratch_ptr[ord] : nullptr;
    }
    if (!ptr) {   // imh_device_open looks it up; a device opened otherwise gets it here
        int rc = imh::use_device(stream->dev);
        if (rc) return rc;
        rc = imh::noalloc_scratch_init(ord);
        if (rc) return rc;
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        ptr = g_scratch_ptr[ord];
    }
    return run_attention(stream, t, cache, q, num_heads, seq_len, seq_lens, attn_scale, out, num_splits, who,
                         nullptr, nullptr, nullptr, 1, ptr);
}

int imh_encode_turboquant_attention_tokens(imh_stream *stream, const imh_tq_tables *t,
                                           const imh_tq_kv_cache *cache, const uint16_t *q, uint32_t num_heads,
                                           uint32_t token_count, uint32_t seq_len, const int32_t *seq_lens,
                                           float attn_scale, uint16_t *out, uint32_t num_splits) {
    return run_attention(stream, t, cache, q, num_heads, seq_len, seq_lens, attn_scale, out, num_splits,
                         "imh_encode_turboquant_attention_tokens", nullptr, nullptr, nullptr, token_count);
}

int imh_encode_kv_cache_and_attention(imh_stream *stream, const imh_tq_tables *t,
                                      const imh_tq_kv_cache *cache, const uint16_t *k_proj,
                                      const uint16_t *v_proj, const uint16_t *q, uint32_t num_heads,
                                      uint32_t seq_pos, float attn_scale, uint16_t *out) {
    const char *who = "imh_encode_kv_cache_and_attention";
    int rc = check_cache(t, cache, who);
    if (rc) return rc;
    if ((uint64_t)seq_pos + 1 > cache->max_seq_len)
        return imh::fail(IMH_ERANGE, std::string(who) + ": position " + std::to_string(seq_pos) +
                                         " is beyond max_seq_len " + std::to_string(cache->max_seq_len));
    if (!k_proj || !v_proj) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    // one launch: the token's K / V are quantized and stored at row seq_pos by
    // one extra workgroup per (kv head, sequence) while the others attend
    // over [0, seq_pos); that workgroup's partial is the token's position
    return run_attention(stream, t, cache, q, num_heads, seq_pos + 1, nullptr, attn_scale, out, 0, who, nullptr,
                         k_proj, v_proj);
}

}  // extern "C"

namespace imh {

// QK-norm + RoPE folded into the cache write (K) and the attention prologue
// (Q); qk must have head_dim = rotary_dim = 128, both norms and positions.
static int check_qk(const imh_qk_norm_rope_params *qk, const char *who) {
    if (!qk || !qk->q_norm || !qk->k_norm || !qk->cos_cache || !qk->sin_cache || !qk->positions)
        return fail(IMH_EINVAL, std::string(who) + ": QK-norm + RoPE needs both norms, the tables and positions");
    if (qk->head_dim != (uint32_t)kD || (qk->rotary_dim != 0 && qk->rotary_dim != (uint32_t)kD) || qk->max_pos == 0)
        return fail(IMH_EUNSUPPORTED, std::string(who) + ": folded QK-norm + RoPE is built for head_dim = "
                                                          "rotary_dim = 128");
    return IMH_OK;
}

int encode_tq_write_attend(imh_stream *stream, const imh_tq_tables *t, const imh_tq_kv_cache *cache,
                           const uint16_t *q, const uint16_t *k_proj, const uint16_t *v_proj, uint32_t num_heads,
                           const int32_t *seq_lens, float attn_scale, uint16_t *out,
                           const imh_qk_norm_rope_params *qk) {
    const char *who = "encode_tq_write_attend";
    if (!k_proj || !v_proj || !seq_lens) return fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    if (qk) {
        int rc = check_qk(qk, who);
        if (rc) return rc;
    }
    return run_attention(stream, t, cache, q, num_heads, 0, seq_lens, attn_scale, out, 0, who, qk, k_proj, v_proj);
}

}  // namespace imh
