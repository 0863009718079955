// matvec_f16.hip -- instantiates the dequant-fused matvec for LK_F16 weights.
#include "matvec_impl.h"

hipError_t lk_matvec_launch_f16(const LkMvArgs& a, int mode, int R, int nch, unsigned blocks, hipStream_t st) {
    return lk::launch_type<LK_F16>(a, mode, R, nch, blocks, st);
}
