// int4_matvec_mt2.hip -- instantiations of the INT4 matvec kernel for
// workgroups of 9..16 batch rows (two MFMA tiles) over a prebuilt image.
#include "int4_matvec_kernel.h"

namespace imh_int4 {

void launch_image_mt2(int nmat, int epi, const Launch &L, const MatPtrs &mp, const ActIn &in) {
    if (nmat == 1) return launch_ng<1, EPI_STORE, 2, SRC_IMAGE>(L, mp, in);
    if (epi == EPI_SILU) return launch_ng<2, EPI_SILU, 2, SRC_IMAGE>(L, mp, in);
    if (epi == EPI_GELU) return launch_ng<2, EPI_GELU, 2, SRC_IMAGE>(L, mp, in);
    return launch_ng<2, EPI_STORE, 2, SRC_IMAGE>(L, mp, in);
}

}  // namespace imh_int4
