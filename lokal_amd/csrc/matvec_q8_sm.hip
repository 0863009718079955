// matvec_q8_sm.hip -- instantiates the dequant-fused matvec for LK_Q8_SM weights
// (the device form of Q5_K and Q6_K).
#include "matvec_impl.h"

hipError_t lk_matvec_launch_q8_sm(const LkMvArgs& a, int mode, int R, int nch, unsigned blocks, hipStream_t st) {
    return lk::launch_type<LK_Q8_SM>(a, mode, R, nch, blocks, st);
}
