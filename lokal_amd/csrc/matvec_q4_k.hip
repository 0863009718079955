// matvec_q4_k.hip -- instantiates the dequant-fused matvec for LK_Q4_K weights.
#include "matvec_impl.h"

hipError_t lk_matvec_launch_q4_k(const LkMvArgs& a, int mode, int R, int nch, unsigned blocks, hipStream_t st) {
    return lk::launch_type<LK_Q4_K>(a, mode, R, nch, blocks, st);
}
