// matvec.hip -- launch planning for the dequant-fused matvec, and the
// dequant / embedding-gather kernel (dequant_row_ref on the device).
#include "lkhip_common.h"
#include "matvec_impl.h"

#ifndef LK_MV_MAX_BLOCKS
#define LK_MV_MAX_BLOCKS 4096u
#endif

static uint32_t chunk_elems(uint32_t type) {
    switch (type) {
    case LK_Q8_0: case LK_Q8_SM: return 16;
    case LK_F16: return 8;
    case LK_Q4_K: return 32;
    default: return 0;
    }
}

// Rows per wave: the largest R that still leaves >= 2048 waves (8 per CU on
// 256 CUs) so small matrices spread over the whole chip and large ones keep
// more bytes in flight per lane.
LkMvPlan lk_matvec_plan(uint32_t type, uint32_t total_rows, uint32_t cols, int mode) {
    LkMvPlan p{};
    const uint32_t ce = chunk_elems(type);
    const uint32_t nchunk = ce ? cols / ce : 0;
    uint32_t nch = (nchunk + 63) / 64;
    if (nch > 6) nch = 8;
    if (nch == 0) nch = 1;
    int R = 1;
    if (mode == LK_MV_ARGMAX) {
        R = 4;
    } else {
        const int maxR = (mode == LK_MV_SWIGLU) ? 2 : 4;
        for (int r = maxR; r >= 1; r >>= 1) {
            if ((total_rows + r - 1) / r >= 2048u || r == 1) {
                R = r;
                break;
            }
        }
    }
    p.rows_per_wave = R;
    p.nch = (int)nch;
    const uint32_t waves = (total_rows + R - 1) / R;
    p.blocks = (waves + 3) / 4;
    // the kernel strides over row groups, so a large matrix needs no more
    // than 16 blocks per CU (lm_head shape, 151936 rows: 48.8 us at 2048
    // blocks, 40.7 at 4096, 41.7 uncapped at 9496)
    if (p.blocks > LK_MV_MAX_BLOCKS) p.blocks = LK_MV_MAX_BLOCKS;
    return p;
}

hipError_t lk_matvec_launch(const LkMvArgs& a, int mode, hipStream_t st, LkMvPlan* plan_out) {
    const uint32_t type = a.seg[0].w.type;
    LkMvPlan p = lk_matvec_plan(type, a.total_rows, a.cols, mode);
    if (plan_out) *plan_out = p;
    if (p.blocks == 0) return hipSuccess;
    switch (type) {
    case LK_Q8_0: return lk_matvec_launch_q8_0(a, mode, p.rows_per_wave, p.nch, p.blocks, st);
    case LK_F16: return lk_matvec_launch_f16(a, mode, p.rows_per_wave, p.nch, p.blocks, st);
    case LK_Q4_K: return lk_matvec_launch_q4_k(a, mode, p.rows_per_wave, p.nch, p.blocks, st);
    case LK_Q8_SM: return lk_matvec_launch_q8_sm(a, mode, p.rows_per_wave, p.nch, p.blocks, st);
    default: return hipErrorInvalidValue;
    }
}

// out[i, :] = dequant(row(i)); row(i) = ids[i] when ids is given, else row0 + i.
__global__ __launch_bounds__(256) void dequant_rows_kernel(const LkDevW w, const uint32_t* __restrict__ ids,
                                                           uint32_t row0, uint32_t nrows, float* __restrict__ out) {
    const uint32_t i = blockIdx.y;
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (i >= nrows || j >= w.cols) return;
    const uint32_t r = ids ? ids[i] : row0 + i;
    if (r >= w.rows) return;
    out[(size_t)i * w.cols + j] = lk_embed_elem(w, r, j);
}

hipError_t lk_dequant_launch(const LkDevW& w, uint32_t row0, uint32_t nrows, float* out, hipStream_t st) {
    if (nrows == 0) return hipSuccess;
    dim3 grid((w.cols + 255) / 256, nrows);
    hipLaunchKernelGGL(dequant_rows_kernel, grid, dim3(256), 0, st, w, (const uint32_t*)nullptr, row0, nrows, out);
    return hipGetLastError();
}

hipError_t lk_gather_launch(const LkDevW& table, const uint32_t* ids, uint32_t n_ids, float* out, hipStream_t st) {
    if (n_ids == 0) return hipSuccess;
    dim3 grid((table.cols + 255) / 256, n_ids);
    hipLaunchKernelGGL(dequant_rows_kernel, grid, dim3(256), 0, st, table, ids, 0u, n_ids, out);
    return hipGetLastError();
}

// Decode-step embedding: the token id lives in device memory (LkStepState),
// so a captured graph replays without host writes.
__global__ __launch_bounds__(256) void embed_step_kernel(const LkDevW w, const LkStepState* __restrict__ st,
                                                         float* __restrict__ x) {
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    const uint32_t r = st->token;
    if (j >= w.cols || r >= w.rows) return;
    x[j] = lk_embed_elem(w, r, j);
}

hipError_t lk_embed_step_launch(const LkDevW& table, const LkStepState* st_dev, float* x, hipStream_t st) {
    hipLaunchKernelGGL(embed_step_kernel, dim3((table.cols + 255) / 256), dim3(256), 0, st, table, st_dev, x);
    return hipGetLastError();
}
