/* ironmill_diag.h -- measurement aids of libironmill_hip.  No counterpart in
 * the reference: they put a ceiling beside the kernels' timings.
 */
#ifndef IRONMILL_DIAG_H
#define IRONMILL_DIAG_H

#include "ironmill_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define IMH_PROBE_TILE 0
#define IMH_PROBE_FLAT 1
#define IMH_PROBE_BAND 2

/* Launch shape of the streaming probe.  TILE: ceil(n / (rows * tiles))
 * workgroups of 64 * waves * nmat threads; each owns `tiles` tiles of `rows`
 * rows (8 or 16) of each of `nmat` (1 or 2) n x k INT4 weights stored back to
 * back, `waves` waves per weight splitting the tiles' loads (16 rows: one
 * 64-byte group run per row per wave-load, the INT4 matvec's pattern; 8 rows:
 * two adjacent groups, 128 bytes per row).  FLAT: `grid` workgroups of
 * `threads` threads, each reading one contiguous run of the bytes.  BAND:
 * the row-band matvec's launch -- `grid` workgroups of 64 * waves * nmat
 * threads, workgroup b reading rows [n b / grid, n (b+1) / grid) of each
 * weight in 8-row tiles, 128 bytes per row per wave-load (k / 128 even). */
typedef struct {
    uint32_t mode;
    uint32_t nmat;
    uint32_t rows;
    uint32_t tiles;
    uint32_t waves;
    uint32_t grid;
    uint32_t threads;
} imh_probe_shape;

/* Streaming probe: reads nmat * n * k / 2 weight bytes at src (16-byte
 * aligned; FLAT reads n * k / 2) with no compute, in the given launch shape.
 * sink: one device word, written only on a chance match. */
int imh_diag_stream_read(imh_stream *stream, const void *src, uint32_t n, uint32_t k, const imh_probe_shape *shape,
                         uint32_t *sink);

/* VALU-dot INT4 matvec, for a counter A/B against the MFMA decode kernels:
 * y [batch][n] = the affine INT4 projection of x [batch][k] (the semantics of
 * imh_encode_affine_projection_int4: x / awq, (q - z) * s per group of 128,
 * f32 accumulation, f16 out) computed as a wavefront-reduction matvec -- 16
 * lanes per row reading 16-byte code chunks, nibble pairs dequantized in
 * registers into v_dot2_f32_f16 against the f16 hi and lo halves of x / awq,
 * a DPP row sum per row, one band of rows per compute unit.  k of 2560 or
 * 4096; batch <= 8 with batch x k x 4.125 bytes within the device's LDS per
 * workgroup. */
int imh_diag_valu_matvec(imh_stream *stream, const uint16_t *x, uint32_t batch, const imh_affine_int4_weight *w,
                         uint16_t *y);

#ifdef __cplusplus
}
#endif

#endif
