// lmhead.hip -- the end of a decode step as one launch: the final RMSNorm
// (src/model.rs:254-255), the lm_head matvec (src/model.rs:256-261), the
// greedy argmax (src/sampler.rs:67-75, first maximum wins) and the step-state
// advance of the greedy loop (src/generate.rs:101-118).
//
// The lm_head is the largest matrix of a step (Qwen2.5-0.5B: 151936 x 896
// Q8_0, 145 MB) and one launch of it is a pure HBM stream, so it runs at the
// occupancy a stream needs: 8 waves per block, 4 blocks per CU, each wave
// walking rows (wave-strided, R rows in flight per lane) with its slice of
// the normalised x held in registers.  Every block normalises x itself (h
// floats, into h*4 bytes of LDS: small, so four blocks fit a CU), so no extra
// launch or grid barrier precedes the rows, and nothing of the norm is on the
// stream's critical path:
//   - x and the gains are loaded first, then the wave's first rows are
//     issued, then the norm runs while the rows are in flight (vector loads
//     return in issue order: loads issued after the rows would wait for them);
//   - the norm's block barriers wait for LDS operations only (__syncthreads
//     would also wait for the rows in flight).
// Each block publishes its best (value, index) key tagged with the launch's
// epoch.  Then either block 0 collects them (bounded wait) and advances the
// step state, or (defer) the launch ends there and the next one-kernel
// decode step folds the keys at its start (or lk_head_finish does): the
// collection's last round trips then overlap the next launch's start instead
// of ending this one.
#include "lkhip_common.h"
#include "matvec_impl.h"

#define HW 8
#define HT (HW * 64)
// widest hidden size the kernel takes (x is held in registers, h / HT per thread)
#define LK_HEAD_MAX_H 4096u

namespace lkh {

using namespace lk;

// Block barrier for data exchanged through LDS only: waits for this wave's
// LDS operations, not for its vector memory operations in flight.
__device__ __forceinline__ void lds_only_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt not waited
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <int WT, int NCH, int R>
__global__ __launch_bounds__(HT) void lm_head_kernel(const LkHeadArgs a) {
    extern __shared__ __align__(16) float xn[];  // h floats; 16-byte aligned after the static LDS
    __shared__ float red[HW];
    __shared__ uint64_t bk[HW];
    __shared__ int to_any;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar row loop
    const uint32_t h = a.h;
    const uint32_t ep = *a.epoch + 1;  // this launch's key epoch
    const uint32_t V = a.vocab;
    const uint32_t gw = blockIdx.x * HW + (uint32_t)wave, nw = gridDim.x * HW;
    const bool collector = !a.defer && blockIdx.x == 0;

    constexpr int XPT = (int)(LK_HEAD_MAX_H / HT);  // x values per thread
    float xv[XPT], gv[XPT];                          // x and the final norm's gains
#pragma unroll
    for (int k = 0; k < XPT; k++) {
        const uint32_t i = threadIdx.x + (uint32_t)k * HT;
        xv[k] = i < h ? a.x[(size_t)i * a.x_stride] : 0.f;
        gv[k] = i < h ? a.norm[i] : 0.f;
    }
    // the collecting block advances the step state at the end: read it now,
    // before the rows (as plain registers: a struct copy would go through
    // scratch, and its store would wait for this load)
    uint4 st0 = make_uint4(0, 0, 0, 0);  // token, pos, n_out, n_feed
    uint32_t st_fed = 0;
    if (collector && threadIdx.x == 0) {
        st0 = *(const uint4*)lk_g((const uint32_t*)a.st);
        st_fed = lk_g((const uint32_t*)a.st)[4];
    }
    Row<WT, NCH> rr[R];
    uint32_t r0 = gw * R;
#pragma unroll
    for (int k = 0; k < R; k++) row_issue(rr[k], a.w, r0 + k < V ? r0 + k : V - 1, lane);

    // math::rmsnorm (src/math.rs:45-49): x * (1/sqrt(mean(x^2) + eps)) * w
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < XPT; k++) ss = fmaf(xv[k], xv[k], ss);
    ss = lk_wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    lds_only_barrier();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < HW; i++) tot += red[i];
    const float scale = 1.0f / sqrtf(tot / (float)h + a.eps);
#pragma unroll
    for (int k = 0; k < XPT; k++) {
        const uint32_t i = threadIdx.x + (uint32_t)k * HT;
        if (i < h) xn[i] = __fmul_rn(__fmul_rn(xv[k], scale), gv[k]);
    }
    lds_only_barrier();

    // this lane's slice of x for every row (Q4_K: 16 low-, then 16 high-nibble values)
    constexpr uint32_t CE = ChunkTraits<WT>::elems;
    float xr[NCH][CE];
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const uint32_t ch = (uint32_t)lane + 64u * i;
        const bool ok = ch < h / CE;
        if constexpr (WT == LK_Q4_K) {
            const uint32_t sb = ch >> 3, k = ch & 7;
            const float* xl = xn + (ok ? sb * 256 + (k >> 1) * 64 + (k & 1) * 16 : 0);
#pragma unroll
            for (int e = 0; e < 16; e++) {
                xr[i][e] = ok ? xl[e] : 0.f;
                xr[i][16 + e] = ok ? xl[32 + e] : 0.f;
            }
        } else {
#pragma unroll
            for (int e = 0; e < (int)CE; e++) xr[i][e] = ok ? xn[ch * CE + e] : 0.f;
        }
    }

    uint64_t best = 0;
    const uint32_t step = nw * R;
    for (; r0 < V; r0 += step) {
        if (r0 != gw * R) {  // the first group was issued before the norm
#pragma unroll
            for (int k = 0; k < R; k++) row_issue(rr[k], a.w, r0 + k < V ? r0 + k : V - 1, lane);
        }
        // the R rows' dots, their wave sums interleaved (each result equals lk_wave_sum's)
        float d[R];
#pragma unroll
        for (int k = 0; k < R; k++) d[k] = row_dot_reg(rr[k], xr, h, lane);
#pragma unroll
        for (int k = 0; k < R; k++) d[k] += lk_dpp<0xB1, 0xF>(d[k], 0.f);
#pragma unroll
        for (int k = 0; k < R; k++) d[k] += lk_dpp<0x4E, 0xF>(d[k], 0.f);
#pragma unroll
        for (int k = 0; k < R; k++) d[k] += lk_dpp<0x124, 0xF>(d[k], 0.f);
#pragma unroll
        for (int k = 0; k < R; k++) d[k] += lk_dpp<0x128, 0xF>(d[k], 0.f);
#pragma unroll
        for (int k = 0; k < R; k++) d[k] += lk_dpp<0x142, 0xA>(d[k], 0.f);
#pragma unroll
        for (int k = 0; k < R; k++) d[k] += lk_dpp<0x143, 0xC>(d[k], 0.f);
#pragma unroll
        for (int k = 0; k < R; k++) {
            const float v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, d[k]), 63));
            if (r0 + k < V && lane == 0) {
                a.logits[r0 + k] = v;
                best = max_u64(best, lk_argmax_key(v, r0 + k));
            }
        }
    }
    // the block's key: its barrier need not wait for the logits stores
    if (lane == 0) bk[wave] = best;
    lds_only_barrier();
    if (threadIdx.x == 0) {
        uint64_t b = bk[0];
        for (int w2 = 1; w2 < HW; w2++) b = max_u64(b, bk[w2]);
        __hip_atomic_store(a.keys + 2 * blockIdx.x, ((uint64_t)ep << 32) | (b >> 32), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.keys + 2 * blockIdx.x + 1, ((uint64_t)ep << 32) | (b & 0xFFFFFFFFu), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!collector) return;
    // block 0: collect every block's key (bounded wait), then advance the
    // step.  Every thread polls its KPT blocks' key words, all in flight at
    // once, re-polling only the words still missing.
    static_assert(LK_HEAD_MAX_BLOCKS <= 2 * HT, "two blocks' keys per thread");
    constexpr int KPT = 2;
    const uint64_t none = (uint64_t)ep << 32;  // a block past the grid: a zero key, ready
    uint64_t kw[2 * KPT];
#pragma unroll
    for (int k = 0; k < 2 * KPT; k++) {
        const uint32_t i = threadIdx.x + (uint32_t)(k >> 1) * HT;
        kw[k] = i < gridDim.x ? __hip_atomic_load(a.keys + 2 * i + (k & 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : none;
    }
    bool timed_out = false;
    for (uint32_t n = 0;; n++) {
        bool done = true;
#pragma unroll
        for (int k = 0; k < 2 * KPT; k++) done &= (uint32_t)(kw[k] >> 32) == ep;
        if (done) break;
        if (n > (1u << 20)) {
            timed_out = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < 2 * KPT; k++) {
            const uint32_t i = threadIdx.x + (uint32_t)(k >> 1) * HT;
            if ((uint32_t)(kw[k] >> 32) != ep)
                kw[k] = __hip_atomic_load(a.keys + 2 * i + (k & 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    uint64_t b = 0;
#pragma unroll
    for (int k = 0; k < KPT; k++) b = max_u64(b, (kw[2 * k] << 32) | (kw[2 * k + 1] & 0xFFFFFFFFu));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) b = max_u64(b, __shfl_xor(b, m, 64));
    if (threadIdx.x == 0) to_any = 0;
    lds_only_barrier();
    if (timed_out) to_any = 1;
    if (lane == 0) bk[wave] = b;
    lds_only_barrier();
    if (wave != 0) return;
    b = lane < HW ? bk[lane] : 0;
#pragma unroll
    for (int m = 4; m >= 1; m >>= 1) b = max_u64(b, __shfl_xor(b, m, 64));
    if (to_any) {
        if (lane == 0) (void)__hip_atomic_fetch_or(a.err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // keeps bit 0 (one-kernel step) if set
        return;
    }
    if (lane == 0) {
        uint32_t token = st0.x, pos = st0.y, n_out = st0.z, n_feed = st0.w, fed = st_fed;
        lk_step_advance(token, pos, n_out, n_feed, fed, lk_argmax_idx(b), a.feed, a.ids_out, true);
        uint32_t* sp = (uint32_t*)a.st;
        *(uint4*)sp = make_uint4(token, pos, n_out, n_feed);
        sp[4] = fed;
        sp[5] = 0;  // not pending
        *a.epoch = ep;
    }
}

// The fold of a deferred launch's keys, when nothing else consumes them: one
// block, after that launch (every key word carries its epoch).
__global__ __launch_bounds__(1024) void head_finish_kernel(const LkHeadArgs a, uint32_t blocks) {
    __shared__ uint64_t bk[16];
    __shared__ uint32_t pend;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (threadIdx.x == 0) pend = a.st->pending;
    __syncthreads();
    if (!pend) return;
    const uint32_t ep = *a.epoch + 1;
    bool ok = true;
    uint64_t b = lk_head_keys_fold(a.keys, blocks, ep, threadIdx.x, blockDim.x, ok);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) b = max_u64(b, __shfl_xor(b, m, 64));
    if (lane == 0) bk[wave] = b;
    if (!ok) (void)__hip_atomic_fetch_or(a.err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int w = 1; w < (int)(blockDim.x / 64); w++) b = max_u64(b, bk[w]);
    b = max_u64(b, bk[0]);
    LkStepState s = *a.st;
    lk_step_advance(s.token, s.pos, s.n_out, s.n_feed, s.fed, lk_argmax_idx(b), a.feed, a.ids_out, true);
    s.pending = 0;
    *a.st = s;
    *a.epoch = ep;
}

// The final norm and lm_head of NB activation rows at once (the Batcher's
// 2-row steps): rows x + b*h of a.x (b < nrows) normalised into LDS by every
// block, each weight row read once and dotted with all NB rows, logits row b at
// a.logits + b*vocab (the GEMM's layout, read by the greedy launch that
// follows).  Rows b >= nrows are computed from row nrows-1 and not stored.
// Same norm arithmetic as lm_head_kernel; no argmax here.
template <int WT, int NCH, int R, int NB>
__global__ __launch_bounds__(HT) void lm_head_rows_kernel(const LkHeadArgs a, uint32_t nrows) {
    extern __shared__ __align__(16) float xn[];  // NB * h floats
    __shared__ float red[NB][HW];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t h = a.h, V = a.vocab;
    const uint32_t gw = blockIdx.x * HW + (uint32_t)wave, nw = gridDim.x * HW;

    constexpr int XPT = (int)(LK_HEAD_MAX_H / HT);
    float xv[NB][XPT], gv[XPT];
#pragma unroll
    for (int k = 0; k < XPT; k++) {
        const uint32_t i = threadIdx.x + (uint32_t)k * HT;
        gv[k] = i < h ? a.norm[i] : 0.f;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const uint32_t rb = (uint32_t)b < nrows ? (uint32_t)b : nrows - 1;
            xv[b][k] = i < h ? a.x[(size_t)rb * h + i] : 0.f;
        }
    }
    Row<WT, NCH> rr[R];
    uint32_t r0 = gw * R;
#pragma unroll
    for (int k = 0; k < R; k++) row_issue(rr[k], a.w, r0 + k < V ? r0 + k : V - 1, lane);

    // math::rmsnorm (src/math.rs:45-49) per row, as in lm_head_kernel
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < XPT; k++) ss = fmaf(xv[b][k], xv[b][k], ss);
        ss = lk_wave_sum(ss);
        if (lane == 0) red[b][wave] = ss;
    }
    lds_only_barrier();
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < HW; i++) tot += red[b][i];
        const float scale = 1.0f / sqrtf(tot / (float)h + a.eps);
#pragma unroll
        for (int k = 0; k < XPT; k++) {
            const uint32_t i = threadIdx.x + (uint32_t)k * HT;
            if (i < h) xn[(size_t)b * h + i] = __fmul_rn(__fmul_rn(xv[b][k], scale), gv[k]);
        }
    }
    lds_only_barrier();

    constexpr uint32_t CE = ChunkTraits<WT>::elems;
    float xr[NB][NCH][CE];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const float* xb = xn + (size_t)b * h;
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const uint32_t ch = (uint32_t)lane + 64u * i;
            const bool ok = ch < h / CE;
            if constexpr (WT == LK_Q4_K) {
                const uint32_t sb = ch >> 3, k = ch & 7;
                const float* xl = xb + (ok ? sb * 256 + (k >> 1) * 64 + (k & 1) * 16 : 0);
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    xr[b][i][e] = ok ? xl[e] : 0.f;
                    xr[b][i][16 + e] = ok ? xl[32 + e] : 0.f;
                }
            } else {
#pragma unroll
                for (int e = 0; e < (int)CE; e++) xr[b][i][e] = ok ? xb[ch * CE + e] : 0.f;
            }
        }
    }

    const uint32_t step = nw * R;
    for (; r0 < V; r0 += step) {
        if (r0 != gw * R) {
#pragma unroll
            for (int k = 0; k < R; k++) row_issue(rr[k], a.w, r0 + k < V ? r0 + k : V - 1, lane);
        }
        float d[R][NB];
#pragma unroll
        for (int k = 0; k < R; k++)
#pragma unroll
            for (int b = 0; b < NB; b++) d[k][b] = row_dot_reg(rr[k], xr[b], h, lane);
        // wave sums (each equals lk_wave_sum's), then lane b*R + k stores (k, b)
        float out = 0.f;
#pragma unroll
        for (int k = 0; k < R; k++)
#pragma unroll
            for (int b = 0; b < NB; b++) {
                float v = d[k][b];
                v += lk_dpp<0xB1, 0xF>(v, 0.f);
                v += lk_dpp<0x4E, 0xF>(v, 0.f);
                v += lk_dpp<0x124, 0xF>(v, 0.f);
                v += lk_dpp<0x128, 0xF>(v, 0.f);
                v += lk_dpp<0x142, 0xA>(v, 0.f);
                v += lk_dpp<0x143, 0xC>(v, 0.f);
                v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
                out = lane == b * R + k ? v : out;
            }
        const uint32_t ob = (uint32_t)lane / R, ok_ = (uint32_t)lane % R;
        if ((uint32_t)lane < (uint32_t)(R * NB) && ob < nrows && r0 + ok_ < V) a.logits[(size_t)ob * V + r0 + ok_] = out;
    }
}

template <int WT, int NCH, int R>
hipError_t launch(const LkHeadArgs& a, unsigned blocks, hipStream_t st) {
    hipLaunchKernelGGL((lm_head_kernel<WT, NCH, R>), dim3(blocks), dim3(HT), a.h * sizeof(float), st, a);
    return hipGetLastError();
}

}  // namespace lkh

uint32_t lk_lm_head_blocks(uint32_t vocab, uint32_t type, uint32_t h) {
    const uint32_t R = lk_lm_head_rows(type, h);
    const uint32_t need = (vocab + HW * R - 1) / (HW * R);
    return need < LK_HEAD_MAX_BLOCKS ? (need ? need : 1) : LK_HEAD_MAX_BLOCKS;
}

static uint32_t head_chunk_elems(uint32_t type) {
    return (type == LK_Q8_0 || type == LK_Q8_SM) ? 16 : (type == LK_F16 ? 8 : 32);
}

uint32_t lk_lm_head_rows(uint32_t type, uint32_t h) {
    const uint32_t elems = head_chunk_elems(type);
    const uint32_t nch = (h / elems + 63) / 64;
    return nch > 1 ? 2 : 4;
}

bool lk_lm_head_fits(uint32_t type, uint32_t h) {
    if (type != LK_Q8_0 && type != LK_F16 && type != LK_Q4_K && type != LK_Q8_SM) return false;
    if (h > LK_HEAD_MAX_H) return false;
    const uint32_t elems = head_chunk_elems(type);
    return h > 0 && h % elems == 0 && (h / elems + 63) / 64 <= 4;
}

hipError_t lk_lm_head_launch(const LkHeadArgs& a, uint32_t blocks, hipStream_t st) {
    if (!lk_lm_head_fits(a.w.type, a.h) || blocks == 0 || blocks > LK_HEAD_MAX_BLOCKS) return hipErrorInvalidValue;
    const uint32_t t = a.w.type;
    const uint32_t elems = head_chunk_elems(t);
    const uint32_t nch = (a.h / elems + 63) / 64;
#define LKH_NCH(T)                                                    \
    switch (nch) {                                                    \
    case 1: return lkh::launch<T, 1, 4>(a, blocks, st);               \
    case 2: return lkh::launch<T, 2, 2>(a, blocks, st);               \
    case 3: return lkh::launch<T, 3, 2>(a, blocks, st);               \
    case 4: return lkh::launch<T, 4, 2>(a, blocks, st);               \
    default: return hipErrorInvalidValue;                             \
    }
    if (t == LK_Q8_0) { LKH_NCH(LK_Q8_0) }
    if (t == LK_F16) { LKH_NCH(LK_F16) }
    if (t == LK_Q4_K) { LKH_NCH(LK_Q4_K) }
    if (t == LK_Q8_SM) { LKH_NCH(LK_Q8_SM) }
#undef LKH_NCH
    return hipErrorInvalidValue;
}

// Two activation rows at most: a third and fourth make the kernel VALU-bound
// (each 16-weight chunk then costs 64 FMAs and four wave reductions per lane;
// Qwen2.5-0.5B shape, 3 / 4 rows: 0.744 / 0.754 ms per step against 0.728 /
// 0.738 with the norm launch + MFMA GEMM, measured), and NCH <= 2 keeps both
// rows' x slices in registers.  Not Q4_K: its dequant makes even two rows
// VALU-bound (TinyLlama shape, 2 rows: 0.899 against 0.890 ms per step).
bool lk_lm_head_rows_fits(uint32_t type, uint32_t h, uint32_t nrows) {
    if (type == LK_Q4_K || !lk_lm_head_fits(type, h) || nrows == 0 || nrows > LK_HEAD_ROWS_MAX) return false;
    const uint32_t nch = (h / head_chunk_elems(type) + 63) / 64;
    return nch <= 2;
}

namespace lkh {
template <int T>
hipError_t launch_rows(const LkHeadArgs& a, uint32_t nrows, uint32_t nch, uint32_t blocks, hipStream_t st) {
    const size_t lds = 2 * (size_t)a.h * sizeof(float);
    if (nch == 1)
        hipLaunchKernelGGL((lm_head_rows_kernel<T, 1, 4, 2>), dim3(blocks), dim3(HT), lds, st, a, nrows);
    else
        hipLaunchKernelGGL((lm_head_rows_kernel<T, 2, 2, 2>), dim3(blocks), dim3(HT), lds, st, a, nrows);
    return hipGetLastError();
}
}  // namespace lkh

hipError_t lk_lm_head_rows_launch(const LkHeadArgs& a, uint32_t nrows, uint32_t blocks, hipStream_t st) {
    if (!lk_lm_head_rows_fits(a.w.type, a.h, nrows) || blocks == 0 || blocks > LK_HEAD_MAX_BLOCKS)
        return hipErrorInvalidValue;
    const uint32_t t = a.w.type;
    const uint32_t nch = (a.h / head_chunk_elems(t) + 63) / 64;
    if (t == LK_Q8_0) return lkh::launch_rows<LK_Q8_0>(a, nrows, nch, blocks, st);
    if (t == LK_F16) return lkh::launch_rows<LK_F16>(a, nrows, nch, blocks, st);
    if (t == LK_Q8_SM) return lkh::launch_rows<LK_Q8_SM>(a, nrows, nch, blocks, st);
    return hipErrorInvalidValue;
}

hipError_t lk_head_finish_launch(const LkHeadArgs& a, uint32_t blocks, hipStream_t st) {
    if (blocks == 0 || blocks > LK_HEAD_MAX_BLOCKS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(lkh::head_finish_kernel, dim3(1), dim3(1024), 0, st, a, blocks);
    return hipGetLastError();
}
