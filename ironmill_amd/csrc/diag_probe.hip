// diag_probe.hip -- a streaming probe: the weight reads of the INT4 matvec
// with no compute, as a ceiling for what one launch of a given grid and
// access pattern can move.
//
// TILE mode reads INT4 weights [N][K/2] the way a matvec workgroup does: each
// workgroup owns `tiles` consecutive tiles of `rows` rows (of each of `nmat`
// matrices stored back to back), `waves` waves per matrix split the tiles'
// load units, and every load is issued before any is consumed.  A load unit
// is one wave-wide 16-byte-per-lane load:
//   rows 16 -- 16 rows x 64 bytes (one group of each row; lane & 15 the row,
//              lane >> 4 the 16-byte quarter), the layout int4_matvec_kernel
//              reads;
//   rows 8  -- 8 rows x 128 bytes (two adjacent groups of each row; lane & 7
//              the row, bit 3 the group, lane >> 4 the quarter).
// FLAT mode splits the same bytes into `grid` contiguous runs read by
// `threads`-thread workgroups, 16 bytes per lane per load, 16 loads in
// flight.  Both fold what they load into one word and store it to sink[0]
// only if it equals `key` (the store keeps the loads live; a chance match
// writes one word, harmlessly).
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/ironmill_diag.h"
#include "imh_internal.h"

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kFlatLoads = 16;

__device__ __forceinline__ uint32_t fold(u32x4_t v) { return v.x ^ v.y ^ v.z ^ v.w; }

template <int NL, int NMAT, int R>
__global__ void __launch_bounds__(1024) probe_tile_kernel(const uint8_t *__restrict__ w, int N, int K, int T,
                                                         uint32_t key, uint32_t *__restrict__ sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = (blockDim.x >> 6) / NMAT;
    const int mat = wave / waves, part = wave - mat * waves;
    const int G = K / 128;
    const int per_tile = R == 16 ? G : G / 2;      // load units of one tile
    const int units = T * per_tile;
    const int u0 = (part * units) / waves, nu = ((part + 1) * units) / waves - u0;
    const uint8_t *wm = w + (size_t)mat * N * (K / 2);
    u32x4_t v[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int u = min(max(u0 + min(i, nu - 1), 0), units - 1);
        const int t = u / per_tile, gu = u - t * per_tile;
        const int r0 = ((int)blockIdx.x * T + t) * R;
        size_t off;
        if (R == 16)
            off = (size_t)min(r0 + (lane & 15), N - 1) * (K / 2) + gu * 64 + (lane >> 4) * 16;
        else
            off = (size_t)min(r0 + (lane & 7), N - 1) * (K / 2) + gu * 128 + ((lane >> 3) & 1) * 64 + (lane >> 4) * 16;
        v[i] = *reinterpret_cast<const u32x4_t *>(wm + off);
    }
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < NL; i++) x ^= fold(v[i]);
    if (x == key) sink[0] = x;
}

// BAND: the row-band matvec's launch -- workgroup b of gridDim.x reads rows
// [N b / NWG, N (b+1) / NWG) of each of NMAT weights, in tiles of 8 rows x
// 128 bytes per wave-load, `waves` waves per weight splitting the group
// pairs; loads past the band read nothing (buffer-resource bounds).
template <int TM, int NP, int NMAT>
__global__ void __launch_bounds__(1024) probe_band_kernel(const uint8_t *__restrict__ w, int N, int K, uint32_t key,
                                                         uint32_t *__restrict__ sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = (blockDim.x >> 6) / NMAT;
    const int mat = wave / waves, part = wave - mat * waves;
    const int P = K / 256;
    const int p0 = (part * P) / waves, np = ((part + 1) * P) / waves - p0;
    const int rb = (int)(((uint32_t)N * blockIdx.x) / gridDim.x);
    const int re = (int)(((uint32_t)N * (blockIdx.x + 1)) / gridDim.x);
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(w + (size_t)mat * N * (K / 2) + (size_t)rb * (K / 2)), 0, (re - rb) * (K / 2), 0x00020000u);
    const int off = (lane & 7) * (K / 2) + ((lane >> 3) & 1) * 64 + (lane >> 4) * 16;
    u32x4_t v[TM][NP];
#pragma unroll
    for (int i = 0; i < NP; i++)
#pragma unroll
        for (int t = 0; t < TM; t++)
            v[t][i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                      r, off + t * 8 * (K / 2) + (p0 + min(i, np - 1)) * 128, 0, 0));
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < NP; i++)
#pragma unroll
        for (int t = 0; t < TM; t++) x ^= fold(v[t][i]);
    if (x == key) sink[0] = x;
}

__global__ void __launch_bounds__(1024) probe_flat_kernel(const u32x4_t *__restrict__ src, size_t n16,
                                                          uint32_t key, uint32_t *__restrict__ sink) {
    const size_t per_wg = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t base = (size_t)blockIdx.x * per_wg;
    const size_t end = min(base + per_wg, n16);
    uint32_t x = 0;
    for (size_t i0 = base + threadIdx.x; i0 < end; i0 += (size_t)kFlatLoads * blockDim.x) {
        u32x4_t v[kFlatLoads];
#pragma unroll
        for (int i = 0; i < kFlatLoads; i++) {
            const size_t idx = min(i0 + (size_t)i * blockDim.x, end - 1);
            v[i] = src[idx];
        }
#pragma unroll
        for (int i = 0; i < kFlatLoads; i++) x ^= fold(v[i]);
    }
    if (x == key) sink[0] = x;
}

template <int NL, int NMAT>
void launch_tile(int rows, dim3 grid, dim3 block, hipStream_t s, const uint8_t *w, int N, int K, int T,
                 uint32_t *sink) {
    if (rows == 16)
        hipLaunchKernelGGL((probe_tile_kernel<NL, NMAT, 16>), grid, block, 0, s, w, N, K, T, 0x9E3779B9u, sink);
    else
        hipLaunchKernelGGL((probe_tile_kernel<NL, NMAT, 8>), grid, block, 0, s, w, N, K, T, 0x9E3779B9u, sink);
}

template <int TM, int NP>
void launch_band(int nmat, dim3 grid, dim3 block, hipStream_t s, const uint8_t *w, int N, int K, uint32_t *sink) {
    if (nmat == 2)
        hipLaunchKernelGGL((probe_band_kernel<TM, NP, 2>), grid, block, 0, s, w, N, K, 0x9E3779B9u, sink);
    else
        hipLaunchKernelGGL((probe_band_kernel<TM, NP, 1>), grid, block, 0, s, w, N, K, 0x9E3779B9u, sink);
}

template <int NMAT>
int launch_tile_nl(int nl, int rows, dim3 grid, dim3 block, hipStream_t s, const uint8_t *w, int N, int K, int T,
                   uint32_t *sink) {
    if (nl <= 2) launch_tile<2, NMAT>(rows, grid, block, s, w, N, K, T, sink);
    else if (nl <= 4) launch_tile<4, NMAT>(rows, grid, block, s, w, N, K, T, sink);
    else if (nl <= 6) launch_tile<6, NMAT>(rows, grid, block, s, w, N, K, T, sink);
    else if (nl <= 8) launch_tile<8, NMAT>(rows, grid, block, s, w, N, K, T, sink);
    else if (nl <= 12) launch_tile<12, NMAT>(rows, grid, block, s, w, N, K, T, sink);
    else if (nl <= 16) launch_tile<16, NMAT>(rows, grid, block, s, w, N, K, T, sink);
    else if (nl <= 24) launch_tile<24, NMAT>(rows, grid, block, s, w, N, K, T, sink);
    else if (nl <= 32) launch_tile<32, NMAT>(rows, grid, block, s, w, N, K, T, sink);
    else return 1;
    return 0;
}

}  // namespace

extern "C" {

int imh_diag_stream_read(imh_stream *stream, const void *src, uint32_t n, uint32_t k, const imh_probe_shape *sh,
                         uint32_t *sink) {
    const char *who = "imh_diag_stream_read";
    if (!stream || !src || !sink || !sh) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    if (n == 0 || k == 0 || k % 128) return imh::fail(IMH_EINVAL, std::string(who) + ": k must be a multiple of 128");
    if (reinterpret_cast<uintptr_t>(src) & 15) return imh::fail(IMH_EINVAL, std::string(who) + ": src not 16-byte aligned");
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    if (sh->mode == IMH_PROBE_TILE) {
        const int G = (int)k / 128;
        if (sh->nmat < 1 || sh->nmat > 2 || (sh->rows != 8 && sh->rows != 16) || sh->tiles < 1 || sh->tiles > 8 ||
            sh->waves < 1 || sh->waves * sh->nmat > 16 || (sh->rows == 8 && G % 2))
            return imh::fail(IMH_EINVAL, std::string(who) + ": nmat 1-2, rows 8 or 16 (8: k / 128 even), tiles 1-8, "
                                                            "waves * nmat <= 16");
        const int units = (int)sh->tiles * (sh->rows == 16 ? G : G / 2);
        const int nl = (units + (int)sh->waves - 1) / (int)sh->waves;
        const int rows_per_wg = (int)(sh->rows * sh->tiles);
        const dim3 grid((n + rows_per_wg - 1) / rows_per_wg), block(64 * sh->waves * sh->nmat);
        const uint8_t *w = static_cast<const uint8_t *>(src);
        const int bad = sh->nmat == 2
                            ? launch_tile_nl<2>(nl, (int)sh->rows, grid, block, stream->stream, w, (int)n, (int)k,
                                                (int)sh->tiles, sink)
                            : launch_tile_nl<1>(nl, (int)sh->rows, grid, block, stream->stream, w, (int)n, (int)k,
                                                (int)sh->tiles, sink);
        if (bad) return imh::fail(IMH_EINVAL, std::string(who) + ": more than 32 loads per lane");
    } else if (sh->mode == IMH_PROBE_BAND) {
        const int G = (int)k / 128;
        if (sh->nmat < 1 || sh->nmat > 2 || sh->waves < 1 || sh->waves * sh->nmat > 16 || sh->grid == 0 ||
            sh->grid > n || G % 2 || (uint64_t)n * sh->grid >= (1ull << 32))
            return imh::fail(IMH_EINVAL, std::string(who) + ": nmat 1-2, waves * nmat <= 16, 0 < grid <= n, "
                                                            "k / 128 even");
        const int rows = (int)((n + sh->grid - 1) / sh->grid), tm = (rows + 7) / 8;
        const int np = (G / 2 + (int)sh->waves - 1) / (int)sh->waves;
        const dim3 grid(sh->grid), block(64 * sh->waves * sh->nmat);
        const uint8_t *w = static_cast<const uint8_t *>(src);
        hipStream_t st = stream->stream;
        if (tm <= 2 && np <= 5) launch_band<2, 5>(sh->nmat, grid, block, st, w, (int)n, (int)k, sink);
        else if (tm <= 3 && np <= 5) launch_band<3, 5>(sh->nmat, grid, block, st, w, (int)n, (int)k, sink);
        else if (tm <= 5 && np <= 3) launch_band<5, 3>(sh->nmat, grid, block, st, w, (int)n, (int)k, sink);
        else return imh::fail(IMH_EINVAL, std::string(who) + ": band shape beyond (tiles, pairs) (2,5) (3,5) (5,3)");
    } else if (sh->mode == IMH_PROBE_FLAT) {
        if (sh->grid == 0 || sh->threads == 0 || sh->threads > 1024 || sh->threads % 64)
            return imh::fail(IMH_EINVAL, std::string(who) + ": grid > 0 and threads a multiple of 64 up to 1024");
        const size_t n16 = (size_t)n * (k / 2) / 16;   // k % 128 == 0: whole 16-byte units
        hipLaunchKernelGGL(probe_flat_kernel, dim3(sh->grid), dim3(sh->threads), 0, stream->stream,
                           static_cast<const u32x4_t *>(src), n16, 0x9E3779B9u, sink);
    } else {
        return imh::fail(IMH_EINVAL, std::string(who) + ": unknown mode");
    }
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

}  // extern "C"
