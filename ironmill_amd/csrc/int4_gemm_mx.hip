// int4_gemm_mx.hip -- the INT4-affine (group 128) prefill GEMM with bf16 or
// fp8-e4m3 matrix-core operands (superblock_matmul_int4, affine_matmul.metal:
// 10-152, at the bf16 / fp8 precisions of the prefill workload):
//
//     C[m][n] = out( sum_g s[n][g] * sum_{k in g} a[m][k] * (q[n][k] - z[n][g]) ),  f32 accumulate
//
// with a = x / awq rounded once to the operand type (bf16, or e4m3 for the
// fp8 variant) and C rounded to bf16.  The weights are never rounded: the
// codes enter the matrix cores as exact small integers and the group's
// zero-point and scale are applied in f32 to the group's partial sums.
//
// MI355X design (not the Metal kernel's structure):
//  * A -- the activation -- goes through LDS; B -- the INT4 weights -- goes
//    straight from memory into registers in the MFMA operand layout (lane =
//    weight column + 32 x K half, two 16-byte loads per lane per group and
//    32-column fragment) and is expanded there, so a workgroup's weights
//    never touch LDS and each is read once per workgroup.
//  * bf16: a code byte q placed under the bf16 exponent byte 0x43 is the bf16
//    value 128 + q exactly (one v_perm per two codes); the MFMA gives
//    sum a (128 + q) and the group's correction subtracts (128 + z) sum a,
//    with sum a the row's group sum of the rounded operand (exact products,
//    f32 sums).  fp8: the code byte itself, read as e4m3, is q * 2^-9 exactly
//    (subnormals and the first binade), the matrix core's block scale 2^9
//    restores q, and the correction subtracts z sum a.  The correction is one more
//    matrix-core product per tile and group (the row sum split into three
//    exact bf16 pieces against -c; the last of the group's bf16 products),
//    so the fold of a group is one multiply-add.
//  * a prep kernel writes the operand rows (x / awq rounded, each 8-element
//    chunk in the slot order the code unpack produces) and their group sums.
//  * the 32 x 32 matrix-core shapes (v_mfma_f32_32x32x16_bf16,
//    v_mfma_scale_f32_32x32x64_f8f6f4): measured on the MI355X they sustain
//    ~2.3 / ~4.9 PFLOP/s where the 16 x 16 bf16 shape stops at ~1.7.
//  * workgroup tile 64 (M) x 256 columns, four waves each owning 64 x 64
//    (2 x 2 MFMA tiles of 32 x 32); the next group's A (global -> registers
//    -> other LDS buffer) and B (global -> registers) are loaded while the
//    current group computes, their loads issued one or two per k step (a
//    burst of twelve at the group's start held the wave's issue for ~400
//    cycles), unconditionally (the last group re-loads itself), so no wait
//    for them sits inside the compute: one barrier per group.  K is split over
//    workgroups when the tile grid leaves workgroup slots (two per CU) idle
//    and a model of the dispatch says the split pays for its partials; the
//    f32 partials are summed in split order by a second kernel
//    (deterministic).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <string>

#include "dpp_reduce.h"
#include "imh_internal.h"

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kGS = 128;
constexpr int kBM = 64;          // workgroup rows (M)
constexpr int kThreads = 256;    // 4 waves, each owning 64 rows x 64 columns
constexpr int kWaveCols = 64;    // two 32-column B fragments per wave
template <int P> constexpr int wg_cols() { return 4 * kWaveCols; }
constexpr float kE4M3Max = 448.0f;

enum Prec : int { PREC_BF16 = 1, PREC_FP8 = 2 };

// fp8 B operand: a code byte q (0..15) read as OCP E4M3 is q * 2^-9 exactly
// (0..7 are the subnormals m * 2^-9, 8..15 the first binade 2^-6 (1 + m / 8));
// the matrix core's E8M0 block scale 2^9 (exponent 127 + 9) restores q.
constexpr uint32_t kScaleCodesE8m0 = 0x88888888u;
constexpr uint32_t kScaleOneE8m0 = 0x7F7F7F7Fu;

// grid (ceil(K / 8 / 256), M), block 256: chunk c (8 elements) of row m:
// a = x / awq (no awq: x) rounded to the operand type, stored in slot order
// {0, 2, 4, 6, 1, 3, 5, 7}; the 16 chunks of a group (16 consecutive lanes)
// sum their rounded values into gsum[m][g].
template <int P>
__global__ void __launch_bounds__(256) gemm_mx_prep_kernel(const __bf16 *__restrict__ x,
                                                           const __half *__restrict__ awq,
                                                           uint8_t *__restrict__ aop, float *__restrict__ gsum,
                                                           int K) {
    const int m = blockIdx.y;
    const int c_raw = blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = c_raw * 8 < K;
    const int c = live ? c_raw : 0;
    const size_t off = (size_t)m * K + (size_t)c * 8;
    const u32x4_t xv = *reinterpret_cast<const u32x4_t *>(x + off);
    const __bf16 *xb = reinterpret_cast<const __bf16 *>(&xv);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (float)xb[i];
    if (awq) {
        const u32x4_t wv = *reinterpret_cast<const u32x4_t *>(awq + (size_t)c * 8);
        const _Float16 *wh = reinterpret_cast<const _Float16 *>(&wv);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = v[i] / (float)wh[i];
    }
    constexpr int kSlot[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    float sum = 0.0f;
    if (P == PREC_BF16) {
        bf16x8_t o;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            o[i] = (__bf16)v[kSlot[i]];
            sum += (float)o[i];
        }
        if (live) *reinterpret_cast<bf16x8_t *>(aop + off * 2) = o;
    } else {
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float e[4];
#pragma unroll
            for (int i = 0; i < 4; i++) e[i] = fminf(fmaxf(v[kSlot[4 * h + i]], -kE4M3Max), kE4M3Max);
            uint32_t p = __builtin_amdgcn_cvt_pk_fp8_f32(e[0], e[1], 0, false);
            p = __builtin_amdgcn_cvt_pk_fp8_f32(e[2], e[3], p, true);
            w[h] = p;
            // the rounded values, back from the encoding
            const float2_t r0 = __builtin_amdgcn_cvt_pk_f32_fp8(p, false);
            const float2_t r1 = __builtin_amdgcn_cvt_pk_f32_fp8(p, true);
            sum += r0[0];
            sum += r0[1];
            sum += r1[0];
            sum += r1[1];
        }
        if (live) *reinterpret_cast<uint2 *>(aop + off) = make_uint2(w[0], w[1]);
    }
    sum = imh_dpp::row16_sum(sum);
    if (live && (threadIdx.x & 15) == 0) gsum[(size_t)m * (K / kGS) + (size_t)c / 16] = sum;
}

// Tile order.  Workgroup ids go round-robin over the 8 XCDs, each with its
// own L2, so the linear id is first turned into an index that is contiguous
// per XCD; that index then walks bands of `band` row tiles (M) with the row
// tile fastest, so the workgroups resident on one XCD share both their A rows
// (one band) and their B columns (neighbouring column tiles) in its L2.
struct TileOrder {
    int tiles_m, tiles_n, band, splits;
};
__device__ __forceinline__ void tile_of(const TileOrder &o, int &mt, int &nt, int &split) {
    const int T = o.tiles_m * o.tiles_n * o.splits;
    const int L = blockIdx.x;
    const int x = L & 7, j = L >> 3;
    const int q = T >> 3, r = T & 7;
    const int t = x * q + min(x, r) + j;             // contiguous per XCD
    const int per_split = o.tiles_m * o.tiles_n;
    split = t / per_split;
    const int u = t - split * per_split;
    const int per_band = o.band * o.tiles_n;
    const int b = u / per_band, v = u - b * per_band;
    mt = b * o.band + v % o.band;
    nt = v / o.band;
}

// grid (tiles_m * tiles_n * splits), block 256; tile (mt, nt, split) from
// tile_of.  Split z covers groups [z * per, min((z + 1) * per, G)).  Without a
// split C is stored as bf16; with one the f32 partials go to part[z][M][N].
//
// Operand layouts of the 32 x 32 MFMAs (lane l: n or m = l & 31, h = l >> 5):
//   bf16 32x32x16, k step s (0..7) of a group: lane (n, h) holds the 8 codes
//     [64 h + 8 s, +8) of column n -- dword s of the 32 code bytes
//     [32 h, 32 h + 32) of the group row -- and A lane (m, h) the operand
//     chunk 8 h + s of row m (8 elements in the code unpack's slot order);
//   fp8 32x32x64, k step t (0..1): lane (n, h) the 32 codes [64 t + 32 h, +32)
//     (code bytes [32 t + 16 h, +16)), A lane (m, h) the 32 operand bytes at
//     64 t + 32 h of row m;
//   D: lane l, value i: row 8 (i >> 2) + 4 h + (i & 3), column l & 31.
template <int P>
__global__ void __launch_bounds__(kThreads, 2) gemm_mx_kernel(
    const uint8_t *__restrict__ aop, const float *__restrict__ gsum, const uint8_t *__restrict__ wdata,
    const __half *__restrict__ scales, const __half *__restrict__ zeros, __bf16 *__restrict__ out,
    float *__restrict__ part, int M, int N, int K, int per, TileOrder order) {
    constexpr int EB = P == PREC_BF16 ? 2 : 1;     // operand bytes per element
    constexpr int RB = kGS * EB + 16;              // LDS row bytes of one group (16-byte pad)
    constexpr int ACH = kBM * kGS * EB / 16 / kThreads;   // 16-byte A chunks per thread per group
    // A stages: [stage buffer][group of the stage] -- GPB groups per barrier:
    // two at bf16, four at fp8 (its operand is half the bytes: the same LDS)
    constexpr int GPB = P == PREC_BF16 ? 2 : 4;
    __shared__ __attribute__((aligned(16))) uint8_t As[2][GPB][kBM * RB];
    __shared__ __attribute__((aligned(16))) float Gs[2][GPB][kBM];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nl = lane & 31, h = lane >> 5;
    int mt, nt, split;
    tile_of(order, mt, nt, split);
    const int m0 = mt * kBM;
    const int n0 = nt * wg_cols<P>() + wave * kWaveCols;
    const int G = K / kGS;
    const int g_begin = split * per;
    const int g_end = min(g_begin + per, G);

    // B rows of this lane: fragment j holds column n0 + 32 j + nl (clamped)
    const uint8_t *brow[2];
    size_t szrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = min(n0 + 32 * j + nl, N - 1);
        brow[j] = wdata + (size_t)n * (K / 2) + (P == PREC_BF16 ? 32 * h : 16 * h);
        szrow[j] = (size_t)n * G;
    }
    // A staging: chunk c = i * 256 + tid of the group's 64 x (128 * EB) bytes
    auto load_a1 = [&](int g, int i, u32x4_t *ar) __attribute__((always_inline)) {
        const int c = i * kThreads + tid;
        const int r = c / (kGS * EB / 16), cc = c - r * (kGS * EB / 16);
        const int m = min(m0 + r, M - 1);
        ar[i] = *reinterpret_cast<const u32x4_t *>(aop + ((size_t)m * K + (size_t)g * kGS) * EB + cc * 16);
    };
    auto load_gs = [&](int g, float &gs) __attribute__((always_inline)) {
        gs = tid < kBM ? gsum[(size_t)min(m0 + tid, M - 1) * G + g] : 0.0f;
    };
    auto load_a = [&](int g, u32x4_t *ar, float &gs) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < ACH; i++) load_a1(g, i, ar);
        load_gs(g, gs);
    };
    auto store_a = [&](int sb, int part, const u32x4_t *ar, float gs) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int c = i * kThreads + tid;
            const int r = c / (kGS * EB / 16), cc = c - r * (kGS * EB / 16);
            *reinterpret_cast<u32x4_t *>(&As[sb][part][r * RB + cc * 16]) = ar[i];
        }
        if (tid < kBM) Gs[sb][part][tid] = gs;
    };
    // B codes (32 bytes per fragment and lane), scales and zero-points of
    // group g; the scale and zero stay apart until used
    struct BRegs {
        u32x4_t w[2][2];
        uint16_t s[2], z[2];
    };
    auto load_b1 = [&](int g, int j, BRegs &b) __attribute__((always_inline)) {
        {
            const uint8_t *p = brow[j] + (size_t)g * 64;
            b.w[j][0] = *reinterpret_cast<const u32x4_t *>(p);
            b.w[j][1] = *reinterpret_cast<const u32x4_t *>(p + (P == PREC_BF16 ? 16 : 32));
            b.s[j] = reinterpret_cast<const uint16_t *>(scales)[szrow[j] + g];
            b.z[j] = reinterpret_cast<const uint16_t *>(zeros)[szrow[j] + g];
        }
    };
    auto load_b = [&](int g, BRegs &b) __attribute__((always_inline)) {
        load_b1(g, 0, b);
        load_b1(g, 1, b);
    };

    float16_t acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[mi][j][i] = 0.0f;

    // One group: the MFMAs of the four 32 x 32 tiles over the group's k
    // steps, then each tile's group partial folded into acc with the scale
    // and zero-point of the lane's column and the group sums of its rows.
    // hook(st) runs at k step st: it issues the next group's loads.
    auto compute = [&](int sb, int part, const BRegs &b, auto &&hook) __attribute__((always_inline)) {
        const uint8_t *Ab = As[sb][part];
        // The group's zero-point correction -c * rowsum (c = 128 + z for the
        // bf16 codes, which carry 128; z for fp8) is added to each tile's
        // group accumulator on the matrix core: A lane (m, 0) holds the row sum
        // split into three bf16 pieces (hi + mid + lo == rowsum exactly), B
        // lane (n, 0) -c three times (exact in bf16), all other k slots zero
        // -- so the fold is one multiply-add per output.
        bf16x8_t ca[2], cb[2];
        {
            const __bf16 z0 = (__bf16)0.0f;
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                const float rs = Gs[sb][part][32 * mi + nl];
                const __bf16 r0 = (__bf16)rs;
                const float e1 = rs - (float)r0;
                const __bf16 r1 = (__bf16)e1;
                const __bf16 r2 = (__bf16)(e1 - (float)r1);
                ca[mi] = h == 0 ? (bf16x8_t){r0, r1, r2, z0, z0, z0, z0, z0} : (bf16x8_t){z0, z0, z0, z0, z0, z0, z0, z0};
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const __bf16 c = (__bf16)((P == PREC_BF16 ? -128.0f : 0.0f) - (float)__builtin_bit_cast(_Float16, b.z[j]));
                cb[j] = h == 0 ? (bf16x8_t){c, c, c, z0, z0, z0, z0, z0} : (bf16x8_t){z0, z0, z0, z0, z0, z0, z0, z0};
            }
        }
        const float16_t zero16 = {};
        if (P == PREC_BF16) {
            float16_t gg[2][2];
#pragma unroll
            for (int st = 0; st < 8; st++) {
                hook(st);
                bf16x8_t af[2], bf[2];
#pragma unroll
                for (int mi = 0; mi < 2; mi++)
                    af[mi] = *reinterpret_cast<const bf16x8_t *>(&Ab[(32 * mi + nl) * RB + (8 * h + st) * 16]);
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    // 8 codes -> bf16 128 + q in slot order {0, 2, 4, 6, 1, 3, 5, 7}
                    const uint32_t w = b.w[j][st >> 2][st & 3];
                    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
                    const u32x4_t o = {__builtin_amdgcn_perm(lo, 0x43434343u, 0x00050004u),
                                       __builtin_amdgcn_perm(lo, 0x43434343u, 0x00070006u),
                                       __builtin_amdgcn_perm(hi, 0x43434343u, 0x00050004u),
                                       __builtin_amdgcn_perm(hi, 0x43434343u, 0x00070006u)};
                    bf[j] = __builtin_bit_cast(bf16x8_t, o);
                }
#pragma unroll
                for (int mi = 0; mi < 2; mi++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        gg[mi][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mi], bf[j], st == 0 ? zero16 : gg[mi][j],
                                                                            0, 0, 0);
            }
            // the zero-point correction last: its operands (an LDS read and a
            // short VALU chain) are built while the k steps run, not ahead of them
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    gg[mi][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ca[mi], cb[j], gg[mi][j], 0, 0, 0);
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float sj = (float)__builtin_bit_cast(_Float16, b.s[j]);
#pragma unroll
                    for (int i = 0; i < 16; i++) acc[mi][j][i] = __builtin_fmaf(sj, gg[mi][j][i], acc[mi][j][i]);
                }
        } else {
#pragma unroll
            for (int st = 0; st < 6; st++) hook(st);
            // both k steps' A fragments, then per column fragment its B
            // fragments and the two tiles' MFMAs: one tile's partial live at a time
            i32x8_t af[2][2];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int mi = 0; mi < 2; mi++) {
                    const uint8_t *p = &Ab[(32 * mi + nl) * RB + 64 * t + 32 * h];
                    const u32x4_t a0 = *reinterpret_cast<const u32x4_t *>(p);
                    const u32x4_t a1 = *reinterpret_cast<const u32x4_t *>(p + 16);
                    af[mi][t] = (i32x8_t){(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                                          (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
                }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                i32x8_t bf[2];
#pragma unroll
                for (int t = 0; t < 2; t++)
                    // code dword d = codes 8 d .. 8 d + 7 -> the even codes' bytes, then the odd
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const uint32_t w = b.w[j][t][d];
                        bf[t][2 * d] = (int)(w & 0x0F0F0F0Fu);
                        bf[t][2 * d + 1] = (int)((w >> 4) & 0x0F0F0F0Fu);
                    }
                const float sj = (float)__builtin_bit_cast(_Float16, b.s[j]);
#pragma unroll
                for (int mi = 0; mi < 2; mi++) {
                    float16_t g = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ca[mi], cb[j], zero16, 0, 0, 0);
#pragma unroll
                    for (int t = 0; t < 2; t++)
                        // formats 0 / 0: e4m3 x e4m3; A scale x1, B scale x 2^9
                        g = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[mi][t], bf[t], g, 0, 0, 0, kScaleOneE8m0,
                                                                            0, kScaleCodesE8m0);
#pragma unroll
                    for (int i = 0; i < 16; i++) acc[mi][j][i] = __builtin_fmaf(sj, g[i], acc[mi][j][i]);
                }
            }
        }
    };

    // Ping-pong over two B register sets (no copies between iterations), A in
    // stages of two groups with one barrier per stage: group g computes from
    // stage buffer sb (part g & 1 of the stage) while group g + 2's A is
    // loaded into registers and, after g's MFMAs, stored to the other stage
    // buffer -- free since the barrier that closed the stage before (every
    // wave was done reading it) -- and group g + 1's B into the other set.
    // The prefetch is unconditional -- past the last group the last one is
    // loaded again -- so the compiler's wait for the current set never has to
    // cover the prefetch.
    u32x4_t ar[ACH];
    BRegs b0, b1;
    float gsv = 0.0f;
    if (g_begin < g_end) {
        load_a(g_begin, ar, gsv);
        load_b(g_begin, b0);
        store_a(0, 0, ar, gsv);
#pragma unroll
        for (int q = 1; q < GPB; q++) {
            load_a(min(g_begin + q, g_end - 1), ar, gsv);
            store_a(0, q, ar, gsv);
        }
        __syncthreads();
    }
    auto step = [&](int g, int sb, int part, const BRegs &cur, BRegs &nxt) __attribute__((always_inline)) {
        const int ga = min(g + GPB, g_end - 1), gb = min(g + 1, g_end - 1);
        // the loads spread over the k steps: A chunks first (they are stored
        // to LDS after the compute), then B
        compute(sb, part, cur, [&](int st) __attribute__((always_inline)) {
            if (st < ACH) load_a1(ga, st, ar);
            if (st == ACH) load_gs(ga, gsv);
            if (st == 4) load_b1(gb, 0, nxt);
            if (st == 5) load_b1(gb, 1, nxt);
        });
        store_a(sb ^ 1, part, ar, gsv);
    };
    // two stages per iteration: the stage buffers' indices are constants (GPB
    // is even, so group parity and part parity pick the same B set)
    for (int g = g_begin; g < g_end; g += 2 * GPB) {
#pragma unroll
        for (int q = 0; q < GPB; q++) {
            if (g + q >= g_end) break;
            if (q & 1) step(g + q, 0, q, b1, b0);
            else step(g + q, 0, q, b0, b1);
        }
        __syncthreads();
        if (g + GPB < g_end) {
#pragma unroll
            for (int q = 0; q < GPB; q++) {
                if (g + GPB + q >= g_end) break;
                if (q & 1) step(g + GPB + q, 1, q, b1, b0);
                else step(g + GPB + q, 1, q, b0, b1);
            }
            __syncthreads();
        }
    }

    // D of tile (mi, j): lane holds rows 32 mi + 8 (i >> 2) + 4 h + (i & 3), column 32 j + nl
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = n0 + 32 * j + nl;
        if (n >= N) continue;
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = m0 + 32 * mi + 8 * (i >> 2) + 4 * h + (i & 3);
                if (m >= M) continue;
                if (part) part[((size_t)split * M + m) * N + n] = acc[mi][j][i];
                else out[(size_t)m * N + n] = (__bf16)acc[mi][j][i];
            }
    }
}

// Sums the split partials in split order: grid ceil(M * N / 256), block 256.
__global__ void __launch_bounds__(256) gemm_mx_reduce_kernel(const float *__restrict__ part, int splits, size_t count,
                                                             __bf16 *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    float s = part[i];
    for (int z = 1; z < splits; z++) s += part[(size_t)z * count + i];
    out[i] = (__bf16)s;
}

int check_gemm_weight(const imh_affine_int4_weight *w, const char *who) {
    if (!w || !w->data || !w->scales || !w->zeros)
        return imh::fail(IMH_EINVAL, std::string(who) + ": weight or one of its arrays is NULL");
    if (w->group_size != kGS)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": group_size " + std::to_string(w->group_size) +
                                               " not supported (built for 128)");
    if (w->n == 0 || w->k == 0 || w->k % kGS)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": k must be a non-zero multiple of 128, n non-zero");
    if ((reinterpret_cast<uintptr_t>(w->data) & 15) != 0)
        return imh::fail(IMH_EINVAL, std::string(who) + ": weight data must be 16-byte aligned");
    return IMH_OK;
}

// K splits for a grid of `tiles` output tiles (fewer than the slots, two
// per CU).  Workgroups of a launch are dispatched as slots free up, and each
// costs about the same per group: ~2.4 us bf16 / ~1.9 us fp8 with two per
// CU, ~0.9 of that alone on its CU.  So a grid of W workgroups runs full
// rounds of two per CU, then its remainder (one per CU where it fits); a
// split adds the partials' round trip (written during the GEMM, read back by
// the reduce launch at ~4.5 TB/s plus ~2 us).  Measured against the earlier
// rule (as many splits as fill two per CU, rounded up): K 2560 -> N 9728 at
// M = 512 (304 tiles) 1 split instead of 2, 65 -> 57 us (bf16); K 9728 ->
// N 2560 at M = 512 (80 tiles) 6 instead of 7, 72 -> 60 us; at M = 2048
// (320 tiles) 1 split took 200 us against 186 with 2 and 185-191 with 3.
// At least 4 groups per split.
double grid_us(long long W, int per, int cus, double g2) {
    double us = 0.0;
    for (; W > 2 * cus; W -= 2 * cus) us += per * g2;
    return us + per * (W > cus ? g2 : 0.9 * g2);
}
int gemm_splits(int tiles, int G, int M, int N, int cus, int P) {
    const double g2 = P == PREC_BF16 ? 2.4 : 1.9;
    int best = 1;
    double best_us = grid_us(tiles, G, cus, g2);
    for (int s = 2; s <= G / 4; s++) {
        const int per = (G + s - 1) / s;
        if ((G + per - 1) / per != s) continue;
        const double us = grid_us((long long)tiles * s, per, cus, g2) +
                          ((double)s * M * N * 4 + (double)M * N * 2) / 4.5e6 + 2.0;
        if (us < best_us * 0.98) {   // a split must win clearly
            best_us = us;
            best = s;
        }
    }
    return best;
}

}  // namespace

extern "C" {

int imh_affine_gemm_int4(imh_stream *stream, const void *x, uint32_t M, const imh_affine_int4_weight *w, void *y,
                         int precision) {
    const char *who = "imh_affine_gemm_int4";
    if (!stream || !x || !y) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    int rc = check_gemm_weight(w, who);
    if (rc) return rc;
    if (precision == IMH_GEMM_F16) {
        // the f16 path is the projection op (matvec below 32 tokens, f16 GEMM from 32)
        return imh_encode_affine_projection_int4(stream, static_cast<const uint16_t *>(x), M, w,
                                                 static_cast<uint16_t *>(y));
    }
    if (precision != IMH_GEMM_BF16 && precision != IMH_GEMM_FP8_E4M3)
        return imh::fail(IMH_EINVAL, std::string(who) + ": unknown precision " + std::to_string(precision));
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (w->awq_scales && (reinterpret_cast<uintptr_t>(w->awq_scales) & 15)))
        return imh::fail(IMH_EINVAL, std::string(who) + ": x and awq_scales must be 16-byte aligned");
    if (M == 0) return IMH_OK;
    if (M > 65535u) return imh::fail(IMH_EINVAL, std::string(who) + ": M above 65535");
    rc = imh::use_device(stream->dev);
    if (rc) return rc;
    const int N = (int)w->n, K = (int)w->k, G = K / kGS;
    const int P = precision == IMH_GEMM_BF16 ? PREC_BF16 : PREC_FP8;
    const int eb = P == PREC_BF16 ? 2 : 1;
    // K split (fewer tiles than workgroup slots, two per CU)
    const int cus = stream->dev->props.multiProcessorCount;
    const int wgc = P == PREC_BF16 ? wg_cols<PREC_BF16>() : wg_cols<PREC_FP8>();
    const int tiles = ((N + wgc - 1) / wgc) * (((int)M + kBM - 1) / kBM);
    int splits = tiles < 2 * cus ? gemm_splits(tiles, G, (int)M, N, cus, P) : 1;
    const int per = (G + splits - 1) / splits;
    splits = (G + per - 1) / per;
    // scratch slot 0: operand rows + group sums; slot 2: split partials
    const size_t a_bytes = ((size_t)M * K * eb + 255) / 256 * 256;
    void *scr = nullptr;
    rc = imh::stream_scratch(stream, 0, a_bytes + (size_t)M * G * sizeof(float), &scr);
    if (rc) return rc;
    uint8_t *aop = static_cast<uint8_t *>(scr);
    float *gsum = reinterpret_cast<float *>(aop + a_bytes);
    float *part = nullptr;
    if (splits > 1) {
        void *p = nullptr;
        rc = imh::stream_scratch(stream, 2, (size_t)splits * M * N * sizeof(float), &p);
        if (rc) return rc;
        part = static_cast<float *>(p);
    }
    const __bf16 *xb = static_cast<const __bf16 *>(x);
    const __half *awq = reinterpret_cast<const __half *>(w->awq_scales);
    dim3 pgrid((K / 8 + 255) / 256, M);
    if (P == PREC_BF16)
        hipLaunchKernelGGL(gemm_mx_prep_kernel<PREC_BF16>, pgrid, dim3(256), 0, stream->stream, xb, awq, aop, gsum, K);
    else
        hipLaunchKernelGGL(gemm_mx_prep_kernel<PREC_FP8>, pgrid, dim3(256), 0, stream->stream, xb, awq, aop, gsum, K);
    IMH_HIP(hipGetLastError());
    TileOrder order;
    order.tiles_m = ((int)M + kBM - 1) / kBM;
    order.tiles_n = (N + wgc - 1) / wgc;
    order.splits = splits;
    // band: the largest divisor of tiles_m that is at most tiles_m / 8 (so
    // each XCD gets about one band), at least 1
    order.band = 1;
    for (int b = std::max(1, order.tiles_m / 8); b >= 1; b--)
        if (order.tiles_m % b == 0) {
            order.band = b;
            break;
        }
    dim3 grid((unsigned)order.tiles_m * order.tiles_n * splits);
    const __half *sc = reinterpret_cast<const __half *>(w->scales), *zr = reinterpret_cast<const __half *>(w->zeros);
    __bf16 *out = static_cast<__bf16 *>(y);
    if (P == PREC_BF16)
        hipLaunchKernelGGL(gemm_mx_kernel<PREC_BF16>, grid, dim3(kThreads), 0, stream->stream, aop, gsum, w->data, sc, zr,
                           out, part, (int)M, N, K, per, order);
    else
        hipLaunchKernelGGL(gemm_mx_kernel<PREC_FP8>, grid, dim3(kThreads), 0, stream->stream, aop, gsum, w->data, sc, zr,
                           out, part, (int)M, N, K, per, order);
    IMH_HIP(hipGetLastError());
    if (splits > 1) {
        const size_t count = (size_t)M * N;
        hipLaunchKernelGGL(gemm_mx_reduce_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream->stream,
                           part, splits, count, out);
        IMH_HIP(hipGetLastError());
    }
    return IMH_OK;
}

}  // extern "C"
