// matvec_q8_0.hip -- instantiates the dequant-fused matvec for LK_Q8_0 weights.
#include "matvec_impl.h"

hipError_t lk_matvec_launch_q8_0(const LkMvArgs& a, int mode, int R, int nch, unsigned blocks, hipStream_t st) {
    return lk::launch_type<LK_Q8_0>(a, mode, R, nch, blocks, st);
}
