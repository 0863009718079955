// lmhead.hip -- the end of a decode step as one launch: the final RMSNorm
// (src/model.rs:254-255), the lm_head matvec (src/model.rs:256-261), the
// greedy argmax (src/sampler.rs:67-75, first maximum wins) and the step-state
// advance of the greedy loop (src/generate.rs:101-118).
//
// The lm_head is the largest matrix of a step (Qwen2.5-0.5B: 151936 x 896
// Q8_0, 145 MB) and one launch of it is a pure HBM stream, so it runs at the
// occupancy a stream needs: 8 waves per block, up to 4 blocks per CU, each
// wave walking rows (wave-strided, R rows in flight per lane) with its slice
// of the normalised x held in registers.  Every block normalises x itself
// (h floats from L2, into h*4 bytes of LDS: small, so four blocks fit a CU),
// so no extra launch or grid barrier precedes the rows.
// Each block publishes its best (value, index) key tagged with the launch's
// epoch; block 0 waits for all of them (bounded), folds them and advances the
// step.  No fences or counters: the tag is the completion flag.
#include "lkhip_common.h"
#include "matvec_impl.h"

#define HW 8
#define HT (HW * 64)

namespace lkh {

using namespace lk;

template <int WT, int NCH, int R>
__global__ __launch_bounds__(HT) void lm_head_kernel(const LkHeadArgs a) {
    extern __shared__ float xn[];  // h floats
    __shared__ float red[HW];
    __shared__ uint64_t bk[HW];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar row loop
    const uint32_t h = a.h;
    const uint32_t ep = *a.epoch + 1;  // this launch's key epoch

    // math::rmsnorm (src/math.rs:45-49): x * (1/sqrt(mean(x^2) + eps)) * w
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < h; i += HT) {
        const float v = a.x[(size_t)i * a.x_stride];
        xn[i] = v;
        ss = fmaf(v, v, ss);
    }
    ss = lk_wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < HW; i++) tot += red[i];
    const float scale = 1.0f / sqrtf(tot / (float)h + a.eps);
    for (uint32_t i = threadIdx.x; i < h; i += HT) xn[i] = __fmul_rn(__fmul_rn(xn[i], scale), a.norm[i]);
    __syncthreads();

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

    const uint32_t V = a.vocab;
    const uint32_t gw = blockIdx.x * HW + (uint32_t)wave, nw = gridDim.x * HW;
    uint64_t best = 0;
    for (uint32_t r0 = gw * R; r0 < V; r0 += nw * R) {
        Row<WT, NCH> rr[R];
#pragma unroll
        for (int k = 0; k < R; k++) row_issue(rr[k], a.w, r0 + k < V ? r0 + k : V - 1, lane);
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
                const uint64_t kk = lk_argmax_key(v, r0 + k);
                best = kk > best ? kk : best;
            }
        }
    }
    if (lane == 0) bk[wave] = best;
    __syncthreads();
    if (wave != 0) return;
    uint64_t b = lane < HW ? bk[lane] : 0;
    if (threadIdx.x == 0) {
        for (int w2 = 1; w2 < HW; w2++) b = bk[w2] > b ? bk[w2] : b;
        // (epoch | high half), (epoch | low half): a word carrying this
        // launch's epoch is this launch's key, so nothing needs clearing
        __hip_atomic_store(a.keys + 2 * blockIdx.x, ((uint64_t)ep << 32) | (b >> 32), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.keys + 2 * blockIdx.x + 1, ((uint64_t)ep << 32) | (b & 0xFFFFFFFFu), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (blockIdx.x != 0) return;
    // block 0, wave 0: collect every block's key (bounded wait), then advance the step
    b = 0;
    bool timed_out = false;
    for (uint32_t i = (uint32_t)lane; i < gridDim.x; i += 64) {
        uint64_t hi = 0, lo = 0;
        for (uint32_t n = 0;; n++) {
            hi = __hip_atomic_load(a.keys + 2 * i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lo = __hip_atomic_load(a.keys + 2 * i + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((uint32_t)(hi >> 32) == ep && (uint32_t)(lo >> 32) == ep) break;
            if (n > (1u << 20)) {
                timed_out = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        const uint64_t kk = (hi << 32) | (lo & 0xFFFFFFFFu);
        b = kk > b ? kk : b;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = __shfl_xor(b, m, 64);
        b = o > b ? o : b;
    }
    if (__any(timed_out)) {
        if (lane == 0) (void)__hip_atomic_fetch_or(a.err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // keeps bit 0 (one-kernel step) if set
        return;
    }
    if (lane == 0) {
        const uint32_t tok = lk_argmax_idx(b);
        LkStepState s = *a.st;
        if (s.n_feed > 0) {  // prefill: the next prompt id is fed
            s.token = a.feed[s.fed];
            s.fed += 1;
            s.n_feed -= 1;
        } else {             // greedy decode: the argmax is the next token
            if (a.ids_out) a.ids_out[s.n_out] = tok;
            s.n_out += 1;
            s.token = tok;
        }
        s.pos += 1;
        *a.st = s;
        *a.epoch = ep;
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
