// int4_matvec_da.hip -- the INT4 matvec over a prebuilt operand image at 1-8
// batch rows with the activation operands read straight from memory.
//
// Same semantics and tile mapping as int4_matvec_kernel (int4_matvec_kernel.h)
// with an IMAGE source: one workgroup per 16-row tile (of each matrix of a
// gate/up pair, or of one row segment), A rows 0-7 the f16 hi halves of the
// batch rows' operand values and rows 8-15 their lo halves, raw code bytes as
// f16 denormals in B.  What differs is where the A operand comes from: the
// LDS kernel stages the image through 64 KB of LDS in stages of groups, each
// stage a dependent load -> barrier -> MFMA round (five of them for K = 9728
// at 8 rows); here lane (i, kq) of a wave loads its own A row's 32 operand
// values of each of its groups from the hi or lo plane -- four 16-byte loads,
// each reading with the row's other three quarters 64 contiguous bytes (the
// image's chunk order, img_chunk) -- together with its weights, so every load
// of a wave is issued up front and nothing waits on the other waves before
// the MFMAs.  The group sums the zero
// point multiplies come from one more MFMA per k slice against the operand of
// codes that are all 1 -- {17, 17, 17, 17, 16, 16, 16, 16} * 2^-24 in the
// B slots -- so they land in the lanes of the result rows they belong to; the
// scale and zero point of a lane's (row, group) are two 2-byte loads issued
// first.  The waves' partial tiles are joined through LDS in part order
// (deterministic), as in the LDS kernel.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>

#include "imh_internal.h"
#include "int4_matvec_kernel.h"

namespace imh_int4 {

namespace {

// grid (tiles), block 64 * NMAT * parts; NG: most groups a wave takes.
template <int NMAT, int EPI, int NG>
__global__ void __launch_bounds__(1024) int4_da_kernel(MatPtrs mp, const ActIn in, int Nall, int K, int B,
                                                       int parts) {
    extern __shared__ __attribute__((aligned(16))) float4_t red[];   // [waves][64]
    const int tid = threadIdx.x;
    const int waves = blockDim.x >> 6;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int mat = wave / parts;
    // the part (group range) this wave takes, rotated by the workgroup index:
    // every tile reads the same operand image, and tiles reading it in the
    // same order at the same time pile onto the same cache lines
    const int part = (wave - mat * parts + (int)blockIdx.x) % parts;
    const int G = K / kGS;

    // the tile's matrix, row segment and image (selects: a dynamic index
    // into the kernel-argument struct would become dependent loads)
    int row0 = blockIdx.x * 16;
    int N = Nall;
    const uint8_t *d0 = mp.data[0], *d1 = mp.data[1];
    const __half *sc0 = mp.scales[0], *sc1 = mp.scales[1];
    const __half *zr0 = mp.zeros[0], *zr1 = mp.zeros[1];
    __half *o0 = mp.out[0], *o1 = mp.out[1];
    int seg_idx = 0;
    if (NMAT == 1 && mp.seg[0] > 0 && row0 < mp.seg[0]) {
        N = mp.seg[0];
    } else if (NMAT == 1 && mp.seg[0] > 0) {
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
    const bool img2 = in.round_mode == 2 && seg_idx > 0;
    const _Float16 *ihi = img2 ? in.hi2 : in.hi;
    const _Float16 *ilo = img2 ? in.lo2 : in.lo;

    const int n_l = lane & 15;   // weight row of the tile (B column) and A row
    const int kq = lane >> 4;    // quarter of a group this lane reads
    const int row = row0 + n_l;
    const int row_c = row < N ? row : N - 1;
    const uint8_t *wdata = (NMAT == 2 && mat) ? d1 : d0;
    const uint16_t *sp = reinterpret_cast<const uint16_t *>((NMAT == 2 && mat) ? sc1 : sc0) + (size_t)row_c * G;
    const uint16_t *zp = reinterpret_cast<const uint16_t *>((NMAT == 2 && mat) ? zr1 : zr0) + (size_t)row_c * G;
    const uint8_t *wrow = wdata + (size_t)row_c * (K / 2) + kq * 16;
    // A row n_l: plane n_l >> 3, batch row n_l & 7 (rows past the batch read
    // row 0; their results are never stored).  Load j of a group reads the
    // chunk at position 4 j + kq, which holds chunk 4 kq + j (img_chunk): the
    // elements 32 kq + 8 j .. + 7 that the weight word j of this lane's
    // 16-byte code load multiplies.
    const int ar = (n_l & 7) < B ? (n_l & 7) : 0;
    const _Float16 *arow = ((n_l >> 3) ? ilo : ihi) + (size_t)ar * K + kq * 8;

    const int g0 = (part * G) / parts;
    const int ng = ((part + 1) * G) / parts - g0;
    // issue order: scales / zero points, then weights and operands, all
    // before the first use (a wave's loads complete in order)
    uint16_t sv[NG], zv[NG];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = g0 + min(i, ng - 1);
        sv[i] = sp[g];
        zv[i] = zp[g];
    }
    u32x4_t wq[NG];
    half8_t av[NG][4];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = g0 + min(i, ng - 1);
        wq[i] = *reinterpret_cast<const u32x4_t *>(wrow + (size_t)g * 64);
#pragma unroll
        for (int j = 0; j < 4; j++) av[i][j] = *reinterpret_cast<const half8_t *>(arow + (size_t)g * kGS + j * 32);
    }
    // all-ones codes: bytes 0x11 (17) in slots 0-3, their high nibbles (16) in 4-7
    const half8_t ones = __builtin_bit_cast(half8_t, (u32x4_t){0x00110011u, 0x00110011u, 0x00100010u, 0x00100010u});

    float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NG; i++) {
        if (i < ng) {
            const float s24 = (float)__builtin_bit_cast(_Float16, sv[i]) * kTwo24;
            const float z = (float)__builtin_bit_cast(_Float16, zv[i]);
            float4_t d = {0.0f, 0.0f, 0.0f, 0.0f}, ds = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t w = wq[i][j];
                const uint32_t q0 = __builtin_amdgcn_perm(w, 0u, 0x0C050C04u);  // b0, b1
                const uint32_t q1 = __builtin_amdgcn_perm(w, 0u, 0x0C070C06u);  // b2, b3
                const u32x4_t bq = {q0, q1, q0 & 0x00F000F0u, q1 & 0x00F000F0u};
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i][j], __builtin_bit_cast(half8_t, bq), d, 0, 0, 0);
                ds = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i][j], ones, ds, 0, 0, 0);
            }
            // D rows 4 kq + r: the group sums of the same A rows
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(s24, __builtin_fmaf(-z, ds[r], d[r]), acc[r]);
        }
    }
    red[(mat * parts + part) * 64 + lane] = acc;   // joined in part order
    __syncthreads();
    if (wave != 0) return;
    // wave 0, lanes 0-31: lane l holds D rows 4 (l >> 4) + r < 8 (hi halves);
    // lane l + 32 the lo halves of the same batch rows.  Parts in part order.
    if (lane >= 32) return;
    float4_t sum[NMAT];
#pragma unroll
    for (int mt = 0; mt < NMAT; mt++) {
        const float4_t *rp = red + (mt * parts) * 64;
        sum[mt] = rp[lane] + rp[lane + 32];
        for (int p = 1; p < parts; p++) sum[mt] += rp[p * 64 + lane] + rp[p * 64 + lane + 32];
    }
    if (row >= N) return;
    const int mrow = 4 * (lane >> 4);   // first batch row of this lane
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = mrow + r;
        if (m >= B) break;
        const float scale = (in.row_scale && !img2) ? in.row_scale[m] : 1.0f;
        if (EPI == EPI_SILU || EPI == EPI_GELU) {
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
            for (int mt = 0; mt < NMAT; mt++) (mt ? o1 : o0)[(size_t)m * N + row] = __float2half(sum[mt][r] * scale);
        }
    }
}

template <int NMAT, int EPI>
void launch_ng_da(int ng, dim3 grid, dim3 block, size_t lds, hipStream_t st, const MatPtrs &mp, const ActIn &in,
                  int N, int K, int B, int parts) {
    if (ng <= 2)
        hipLaunchKernelGGL((int4_da_kernel<NMAT, EPI, 2>), grid, block, lds, st, mp, in, N, K, B, parts);
    else if (ng <= 3)
        hipLaunchKernelGGL((int4_da_kernel<NMAT, EPI, 3>), grid, block, lds, st, mp, in, N, K, B, parts);
    else if (ng <= 4)
        hipLaunchKernelGGL((int4_da_kernel<NMAT, EPI, 4>), grid, block, lds, st, mp, in, N, K, B, parts);
    else
        hipLaunchKernelGGL((int4_da_kernel<NMAT, EPI, 5>), grid, block, lds, st, mp, in, N, K, B, parts);
}

// Split-K over a prebuilt image, 3-8 rows: grid (bands of NT tiles, S
// slices of K).  Workgroup (band, slice) reads the operand of its slice only
// and the weights of its NT x 16 rows in that slice, so a CU moves ~1 / S of
// the image the per-tile kernel reads; the band's f32 partial sums go to
// part[slice][m][row] and int4_splitk_combine_kernel adds the slices in
// slice order (deterministic).  Waves split the slice's groups (<= NG each);
// each wave loads a group's A operand once (the direct-operand layout) and
// uses it for the NT tiles' weights.  Row segments: each tile takes its own
// segment's weights (segment starts are multiples of 16).  Tiles [0, gb) and
// [gb, tiles) are banded apart -- bands0 bands, then the rest -- because with
// a mixed rounding (round_mode 2) the rows from gb on read the second image.
template <int NT, int NG>
__global__ void __launch_bounds__(1024) int4_splitk_kernel(MatPtrs mp, const ActIn in, int N, int K, int B, int S,
                                                           int gb, int bands0, float *__restrict__ part) {
    extern __shared__ __attribute__((aligned(16))) float4_t red[];   // [NT][waves][64]
    const int tid = threadIdx.x;
    const int waves = blockDim.x >> 6;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = K / kGS;
    const int slice = blockIdx.y;
    const int gs0 = (slice * G) / S, gsn = ((slice + 1) * G) / S - gs0;
    const int part_w = (wave + (int)blockIdx.x) % waves;   // rotated, as in the per-tile kernel
    const int g0 = gs0 + (part_w * gsn) / waves;
    const int ng = gs0 + ((part_w + 1) * gsn) / waves - g0;
    const int n_l = lane & 15, kq = lane >> 4;

    const int band = blockIdx.x;
    const bool grp1 = band >= bands0;
    const int tiles = (N + 15) / 16;
    const int tile0 = grp1 ? gb + (band - bands0) * NT : band * NT;
    const int tile_end = grp1 ? tiles : gb;
    const bool img2 = grp1 && in.round_mode == 2;
    // tile t: its segment's weights, scales and zero points, and the lane's
    // row within the segment (tiles past the band's end redo its last tile;
    // they store nothing)
    const uint8_t *wd[NT];
    const uint16_t *sp[NT], *zp[NT];
    int rowc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int r0 = min(tile0 + t, tile_end - 1) * 16;
        const int sg = (mp.seg[0] > 0 && r0 >= mp.seg[0]) ? ((mp.seg[1] > 0 && r0 >= mp.seg[1]) ? 2 : 1) : 0;
        const int base = sg == 0 ? 0 : (sg == 1 ? mp.seg[0] : mp.seg[1]);
        const int end = sg == 0 ? (mp.seg[0] > 0 ? mp.seg[0] : N) : (sg == 1 && mp.seg[1] > 0 ? mp.seg[1] : N);
        wd[t] = sg == 0 ? mp.data[0] : (sg == 1 ? mp.data[1] : mp.data[2]);
        sp[t] = reinterpret_cast<const uint16_t *>(sg == 0 ? mp.scales[0] : (sg == 1 ? mp.scales[1] : mp.scales[2]));
        zp[t] = reinterpret_cast<const uint16_t *>(sg == 0 ? mp.zeros[0] : (sg == 1 ? mp.zeros[1] : mp.zeros[2]));
        rowc[t] = min(r0 + n_l, end - 1) - base;
    }
    const int ar = (n_l & 7) < B ? (n_l & 7) : 0;
    const _Float16 *arow = ((n_l >> 3) ? (img2 ? in.lo2 : in.lo) : (img2 ? in.hi2 : in.hi)) + (size_t)ar * K + kq * 8;

    uint16_t sv[NG][NT], zv[NG][NT];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = g0 + min(i, max(ng - 1, 0));
#pragma unroll
        for (int t = 0; t < NT; t++) {
            sv[i][t] = sp[t][(size_t)rowc[t] * G + g];
            zv[i][t] = zp[t][(size_t)rowc[t] * G + g];
        }
    }
    u32x4_t wq[NG][NT];
    half8_t av[NG][4];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const int g = g0 + min(i, max(ng - 1, 0));
#pragma unroll
        for (int j = 0; j < 4; j++) av[i][j] = *reinterpret_cast<const half8_t *>(arow + (size_t)g * kGS + j * 32);
#pragma unroll
        for (int t = 0; t < NT; t++)
            wq[i][t] = *reinterpret_cast<const u32x4_t *>(wd[t] + (size_t)rowc[t] * (K / 2) + (size_t)g * 64 + kq * 16);
    }
    const half8_t ones = __builtin_bit_cast(half8_t, (u32x4_t){0x00110011u, 0x00110011u, 0x00100010u, 0x00100010u});
    float4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NG; i++) {
        if (i < ng) {
            float4_t ds = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) ds = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i][j], ones, ds, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                float4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t w = wq[i][t][j];
                    const uint32_t q0 = __builtin_amdgcn_perm(w, 0u, 0x0C050C04u);
                    const uint32_t q1 = __builtin_amdgcn_perm(w, 0u, 0x0C070C06u);
                    const u32x4_t bq = {q0, q1, q0 & 0x00F000F0u, q1 & 0x00F000F0u};
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i][j], __builtin_bit_cast(half8_t, bq), d, 0, 0, 0);
                }
                const float s24 = (float)__builtin_bit_cast(_Float16, sv[i][t]) * kTwo24;
                const float z = (float)__builtin_bit_cast(_Float16, zv[i][t]);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[t][r] = __builtin_fmaf(s24, __builtin_fmaf(-z, ds[r], d[r]), acc[t][r]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) red[(t * waves + part_w) * 64 + lane] = acc[t];
    __syncthreads();
    // thread (t, lane < 32): tile t, D rows 4 (lane >> 4) + r (hi) and + 8 (lo),
    // parts in part order
    for (int o = tid; o < NT * 32; o += blockDim.x) {
        const int t = o >> 5, l = o & 31;
        if (tile0 + t >= tile_end) continue;
        const float4_t *rp = red + t * waves * 64;
        float4_t sum = rp[l] + rp[l + 32];
        for (int p = 1; p < waves; p++) sum += rp[p * 64 + l] + rp[p * 64 + l + 32];
        const int row = (tile0 + t) * 16 + (l & 15);
        if (row >= N) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 4 * (l >> 4) + r;
            if (m < B) part[((size_t)slice * B + m) * N + row] = sum[r];
        }
    }
}

// y = f16(sum over slices of part[s][m][row], slices in order, times
// row_scale[m] for rows below scale_rows) into the row's segment.  Every
// slice's load is issued before the first add (S <= kMaxSlices), so the
// thread waits one memory latency rather than S.
constexpr int kMaxSlices = 8;
__global__ void __launch_bounds__(256) int4_splitk_combine_kernel(const float *__restrict__ part, int S, int B, int N,
                                                                  MatPtrs mp, const float *__restrict__ row_scale,
                                                                  int scale_rows) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int count = B * N;
    if (i >= count) return;
    float v[kMaxSlices];
#pragma unroll
    for (int k = 0; k < kMaxSlices; k++) v[k] = k < S ? part[(size_t)k * count + i] : 0.0f;
    float s = v[0];
#pragma unroll
    for (int k = 1; k < kMaxSlices; k++)
        if (k < S) s += v[k];
    const int m = i / N, row = i - m * N;
    if (row_scale && row < scale_rows) s *= row_scale[m];
    const int sg = (mp.seg[0] > 0 && row >= mp.seg[0]) ? ((mp.seg[1] > 0 && row >= mp.seg[1]) ? 2 : 1) : 0;
    const int base = sg == 0 ? 0 : (sg == 1 ? mp.seg[0] : mp.seg[1]);
    const int end = sg == 0 ? (mp.seg[0] > 0 ? mp.seg[0] : N) : (sg == 1 && mp.seg[1] > 0 ? mp.seg[1] : N);
    __half *o = sg == 0 ? mp.out[0] : (sg == 1 ? mp.out[1] : mp.out[2]);
    o[(size_t)m * (end - base) + (row - base)] = __float2half(s);
}

}  // namespace

// Split-K over an image: one matrix (row segments allowed), 3-8 rows, >= 16
// groups, up to two tiles per CU -- where the per-tile kernels would read the
// whole operand image once per 16 rows.  split_rows: the rows from there on
// read the second image (mixed rounding), N otherwise.
namespace {
constexpr int kSplitNT = 5;   // 16-row tiles per band
constexpr int kSplitNG = 2;   // groups per wave at most (one up to 16 groups per slice)
struct SplitBands {
    int gb, bands0, bands, S;
};
SplitBands splitk_bands(int N, int split_rows, int cus) {
    const int tiles = (N + 15) / 16;
    SplitBands b;
    b.gb = split_rows >= N ? tiles : std::min(tiles, split_rows / 16);
    b.bands0 = (b.gb + kSplitNT - 1) / kSplitNT;
    b.bands = b.bands0 + (tiles - b.gb + kSplitNT - 1) / kSplitNT;
    b.S = std::max(2, std::min(kMaxSlices, cus / std::max(1, b.bands)));
    return b;
}
}  // namespace

bool splitk_applies(int nmat, int B, int N, int K, int split_rows, int cus) {
    const int G = K / kGS, tiles = (N + 15) / 16;
    if (nmat != 1 || B < 3 || B > 8 || G < 16 || tiles > 2 * cus) return false;
    const SplitBands b = splitk_bands(N, split_rows, cus);
    return (G + b.S - 1) / b.S <= 16 * kSplitNG;   // 16 waves of kSplitNG groups
}

size_t splitk_workspace_bytes(int B, int N, int split_rows, int cus) {
    return (size_t)splitk_bands(N, split_rows, cus).S * B * N * sizeof(float);
}

int launch_splitk(hipStream_t st, int cus, int N, int K, int B, const MatPtrs &mp, const ActIn &in, int split_rows,
                  void *ws) {
    const int G = K / kGS;
    const SplitBands b = splitk_bands(N, split_rows, cus);
    const int gper = (G + b.S - 1) / b.S;
    // one group per wave while a slice holds at most 16 (down at 3-8 rows:
    // 10 waves of 1 -- B=4 / 8 12.19 / 12.76 -> 11.46 / 12.03 us, decode step
    // B=8 3.26 -> 3.21 ms, against 5 waves of 2), else two
    const int ng = gper <= 16 ? 1 : kSplitNG;
    const int waves = std::min(16, (gper + ng - 1) / ng);
    if (waves * ng < gper) return imh::fail(IMH_EINVAL, "int4 split-K: too many groups per slice");
    const size_t lds = (size_t)kSplitNT * waves * 64 * sizeof(float4_t);
    float *part = static_cast<float *>(ws);
    if (ng == 1)
        hipLaunchKernelGGL((int4_splitk_kernel<kSplitNT, 1>), dim3(b.bands, b.S), dim3(64 * waves), lds, st, mp, in, N,
                           K, B, b.S, b.gb, b.bands0, part);
    else
        hipLaunchKernelGGL((int4_splitk_kernel<kSplitNT, kSplitNG>), dim3(b.bands, b.S), dim3(64 * waves), lds, st, mp,
                           in, N, K, B, b.S, b.gb, b.bands0, part);
    IMH_HIP(hipGetLastError());
    const int count = B * N;
    hipLaunchKernelGGL(int4_splitk_combine_kernel, dim3((count + 255) / 256), dim3(256), 0, st, part, b.S, B, N, mp,
                       in.row_scale, split_rows);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

bool image_da_applies(int nmat, int B, int K) {
    const int G = K / kGS;
    const int parts = std::min(kMaxWaves / nmat, G);
    return B >= 1 && B <= 8 && (G + parts - 1) / parts <= 5;
}

int launch_image_da(hipStream_t st, int nmat, int epi, int N, int K, int B, const MatPtrs &mp, const ActIn &in) {
    const int G = K / kGS;
    // waves per matrix: enough that each holds at most 5 groups of loads,
    // at least 4 (2 for a pair) so a tile's loads spread over the SIMDs
    const int parts = std::min(kMaxWaves / nmat, std::max((G + 4) / 5, std::min(4 / nmat, G)));
    const int ng = (G + parts - 1) / parts;
    const int waves = nmat * parts;
    const dim3 grid((N + 15) / 16), block(64 * waves);
    const size_t lds = (size_t)waves * 64 * sizeof(float4_t);
    if (nmat == 1)
        launch_ng_da<1, EPI_STORE>(ng, grid, block, lds, st, mp, in, N, K, B, parts);
    else if (epi == EPI_SILU)
        launch_ng_da<2, EPI_SILU>(ng, grid, block, lds, st, mp, in, N, K, B, parts);
    else if (epi == EPI_GELU)
        launch_ng_da<2, EPI_GELU>(ng, grid, block, lds, st, mp, in, N, K, B, parts);
    else
        launch_ng_da<2, EPI_STORE>(ng, grid, block, lds, st, mp, in, N, K, B, parts);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

}  // namespace imh_int4
