// int4_matvec_raw.hip -- instantiations of the INT4 matvec kernel whose
// activation image is built in the workgroup (RAW, RAW_RN sources).
#include "int4_matvec_kernel.h"

namespace imh_int4 {

void launch_raw(int nmat, int epi, bool rn, const Launch &L, const MatPtrs &mp, const ActIn &in) {
    if (rn && nmat == 2 && epi == EPI_GELU) return launch_ng<2, EPI_GELU, 1, SRC_RAW_RN>(L, mp, in);
    if (rn && nmat == 2) return launch_ng<2, EPI_SILU, 1, SRC_RAW_RN>(L, mp, in);
    if (rn) return launch_ng<1, EPI_STORE, 1, SRC_RAW_RN>(L, mp, in);
    if (nmat == 1) return launch_ng<1, EPI_STORE, 1, SRC_RAW>(L, mp, in);
    if (epi == EPI_SILU) return launch_ng<2, EPI_SILU, 1, SRC_RAW>(L, mp, in);
    if (epi == EPI_GELU) return launch_ng<2, EPI_GELU, 1, SRC_RAW>(L, mp, in);
    return launch_ng<2, EPI_STORE, 1, SRC_RAW>(L, mp, in);
}

}  // namespace imh_int4
