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

#ifdef __cplusplus
}
#endif

#endif
