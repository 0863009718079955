// attention.hip -- GQA flash-decoding over the KV cache (model::attention,
// src/model.rs:286-318, computed split-K over positions and merged).
//
// One block = one (sequence, kv head, chunk of 64*A*T positions).  The G
// query heads that share the kv head are staged in LDS (or registers), so
// every K and V byte of the chunk is read from HBM exactly once for the whole
// group.  Each of the block's A active waves (A = 8, 4, 2 or 1 of its 8)
// takes the 64-position tiles w, w+A, ... of the chunk with an online softmax
// across them:
//   scores : lane = position, the K row (128 B) is converted once and dotted
//            against all G query rows (LDS broadcast reads);
//   softmax: per-tile max / exp / sum by wave reductions;
//   P.V    : lane = (position group lane & 7, 8 dims), one 16-byte V load per
//            lane covers 8 positions x 64 dims per instruction; the 8 lanes that
//            share a dim slice are combined by DPP.
// Loads are straight-line (positions past ctx re-read the last live row and
// are masked), issued before the dependent arithmetic.
// The waves merge in LDS into one (m, l, acc[64]) partial per query head,
// written with coherent stores; the block then counts itself in on its
// (sequence, kv head) counter, and the block that arrives last folds every
// chunk's partials (max-rescaled sums) into the output and clears the
// counter -- one launch per layer, no separate merge kernel.  The host picks
// A and T per launch (attn_plan): at most 32 chunks per (sequence, kv head),
// so the fold reads each head's partials in one round trip, and, where the
// cache is short, smaller chunks (A < 8) so the grid still has >= 128 blocks.
// Few large chunks beat many small ones: each chunk costs a partial write,
// an atomic on its counter and a share of the fold, and those counters sit
// 256 bytes apart so the atomics of different (sequence, kv head) do not
// contend for one cache line.
// fp32 throughout; scale 1/sqrt(64) = 0.125 is exact.
#include "lkhip_common.h"

#include <cstdlib>
#include <cstring>
#include <mutex>

#define LK_HD 64
#ifndef LK_ACHUNK
#define LK_ACHUNK 512
#endif
#define LK_AW (LK_ACHUNK / 64)  // waves per block: one 64-position tile each per round
#ifndef LK_MAXCH
#define LK_MAXCH 32  // chunks per (sequence, kv head) at most: the fold's loads per lane
#endif
#ifndef LK_ATTN_MINBLOCKS
#define LK_ATTN_MINBLOCKS 128  // grid size below which the plan shrinks the chunk
#endif

// Partial slots per (sequence, head): every plan's chunk holds >= 64 positions.
static inline uint32_t attn_chunk_cap(uint32_t max_seq) {
    const uint32_t t = (max_seq + 63) / 64;
    return t < LK_MAXCH ? t : LK_MAXCH;
}
struct AttnPlan {
    uint32_t waves, tiles, chunks;  // active waves per block, tiles per wave, chunks per (seq, kvh)
};
// The largest A in 8, 4, 2, 1 whose grid has >= LK_ATTN_MINBLOCKS blocks,
// else the one with the most blocks (the larger A on a tie), with T the
// fewest tiles per wave that keep the chunks per (seq, kvh) <= LK_MAXCH.
static AttnPlan attn_plan(uint32_t n_seq, uint32_t n_kv, uint32_t max_seq) {
    AttnPlan best{};
    for (uint32_t A = LK_AW; A >= 1; A /= 2) {
        AttnPlan p{};
        // Many (sequence, kv head) pairs -- prefill rows, large batches -- fill
        // the chip with 4-wave chunks already, and those idle fewer waves on
        // short causal rows than 8-wave ones (a 512-token prefill of the
        // Qwen2.5-0.5B shape: 6.70 -> 6.47 ms)
        if (A > 4) {
            const uint32_t t4 = (max_seq + 64 * 4 * LK_MAXCH - 1) / (64 * 4 * LK_MAXCH);
            const uint32_t c4 = (max_seq + 64 * 4 * t4 - 1) / (64 * 4 * t4);
            if ((uint64_t)c4 * n_kv * n_seq >= 1024) continue;
        }
        const uint32_t per = 64 * A * LK_MAXCH;
        p.waves = A;
        p.tiles = (max_seq + per - 1) / per;
        if (!p.tiles) p.tiles = 1;
        p.chunks = (max_seq + 64 * A * p.tiles - 1) / (64 * A * p.tiles);
        if (!best.waves || p.chunks > best.chunks) best = p;
        if ((uint64_t)p.chunks * n_kv * n_seq >= LK_ATTN_MINBLOCKS) return p;
    }
    return best;
}
uint32_t lk_attn_chunk(uint32_t max_seq) {
    const AttnPlan p = attn_plan(1, 1, max_seq);
    return 64 * p.waves * p.tiles;
}

// Fixed partial buffer of lkhip_attn_decode_noalloc, for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops).  Each
// device holds its own copy for the life of the process.  In host code the
// array's name is only a stand-in: its device address comes from
// hipGetSymbolAddress, once per device (lk_attn_scratch below), and only that
// address is ever passed to a kernel.  Every call on a device shares it, so
// calls that overlap on one device race.  Its arrival counters start at zero
// (static storage) and every launch leaves them zero again.
static __device__ __align__(256) float scratch[LK_ATTN_SCRATCH_FLOATS];

hipError_t lk_attn_scratch(float** out) {
    static std::mutex mu;
    static float* addr[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[dev] = (float*)p;
    }
    *out = addr[dev];
    return hipSuccess;
}

size_t lk_attn_part_floats(uint32_t n_seq, uint32_t n_heads, uint32_t max_seq) {
    return (size_t)n_seq * n_heads * attn_chunk_cap(max_seq) * (2 + LK_HD);
}

__device__ __forceinline__ uint32_t attn_ctx(const LkAttnArgs& a, uint32_t seq) {
    const uint32_t c = a.ctx_len ? a.ctx_len[seq] : a.st->pos + 1;
    return c < a.max_seq ? c : a.max_seq;  // never read past the cache
}

// 8 consecutive cache elements as f32: f16 cache (one 16-byte load) or f32
// cache (two 16-byte loads).
__device__ __forceinline__ void load8(const uint16_t* p, float* o) {
    const uint4 v = *(const uint4*)p;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int h = 0; h < 4; h++) {
        o[2 * h] = lk_h2f((uint16_t)(w[h] & 0xFFFF));
        o[2 * h + 1] = lk_h2f((uint16_t)(w[h] >> 16));
    }
}
__device__ __forceinline__ void load8(const float* p, float* o) {
    const float4 a = ((const float4*)p)[0], b = ((const float4*)p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}


__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store((uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
    return __uint_as_float(__hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// After a block has written its chunk partials (coherent stores): wait until
// they are acknowledged, count the block in, and if it is the last of the
// nch chunks of (seq, kvh), fold all of them into the output.  The partial
// stores are write-through and complete before the count (s_waitcnt
// vmcnt(0) + the barrier), and the folding block reads them with coherent
// loads after seeing the count, so it sees every chunk's words; no cache
// writeback is needed.  Wave w folds heads w, w+4: lane k holds chunk k's
// (m, l), and every lane its dim of all chunks' acc -- one round trip for
// the lot (nch <= LK_MAXCH = 64).
// Memory order of the arrival count.  Acquire-release at agent scope makes the
// fold's visibility a guarantee of the memory model rather than of the
// write-through partial stores; LK_ATTN_FOLD_ORDER=__ATOMIC_RELAXED builds the
// variant that relies on the stores alone (kept for measurement).
#ifndef LK_ATTN_FOLD_ORDER
#define LK_ATTN_FOLD_ORDER __ATOMIC_ACQ_REL
#endif

template <int G>
__device__ __forceinline__ void count_in_and_fold(const LkAttnArgs& a, uint32_t seq, uint32_t kvh, uint32_t nch) {
    __shared__ uint32_t last;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are complete
    __syncthreads();
    if (tid == 0) {
        uint32_t* cnt = a.cnt + ((size_t)seq * a.n_kv + kvh) * LK_ATTN_CNT_STRIDE;
        last = __hip_atomic_fetch_add(cnt, 1u, LK_ATTN_FOLD_ORDER, __HIP_MEMORY_SCOPE_AGENT) == nch - 1;
    }
    __syncthreads();
    if (!last) return;
#pragma unroll
    for (int r = 0; r < (8 + LK_AW - 1) / LK_AW; r++) {
        const uint32_t g = (uint32_t)w + LK_AW * r;
        if (g >= (uint32_t)G) break;
        const uint32_t h = kvh * G + g;
        const float* ph = a.part + ((size_t)seq * a.n_heads + h) * a.cstride * (2 + LK_HD);
        const bool live = (uint32_t)lane < nch;
        const float* pk = ph + (size_t)(live ? lane : 0) * (2 + LK_HD);
        const float mk = ld_coherent(pk), lk = ld_coherent(pk + 1);
        float av[LK_MAXCH];
#pragma unroll
        for (int k = 0; k < LK_MAXCH; k++) {
            const uint32_t c = (uint32_t)k < nch ? (uint32_t)k : 0u;  // in-range reload, weighted 0 below
            av[k] = ld_coherent(ph + (size_t)c * (2 + LK_HD) + 2 + lane);
        }
        const float M = lk_wave_max(live ? mk : -INFINITY);  // finite: chunk 0 is live
        const float sck = live ? expf(mk - M) : 0.f;          // chunk k's weight, held by lane k
        const float L = lk_wave_sum(sck * lk);
        float A = 0.f;
#pragma unroll
        for (int k = 0; k < LK_MAXCH; k++) {
            const float sk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sck), k));
            A = fmaf(sk, av[k], A);
        }
        a.out[((size_t)seq * a.n_heads + h) * LK_HD + lane] = A / L;
    }
    if (tid == 0)
        __hip_atomic_store(a.cnt + ((size_t)seq * a.n_kv + kvh) * LK_ATTN_CNT_STRIDE, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// The 4 waves' (m, l, acc) of each head (red_m[w][g] etc.) -> the chunk's
// partial per head, with coherent stores.
template <int G, typename RM, typename RA>
__device__ __forceinline__ void write_chunk_partial(const LkAttnArgs& a, uint32_t seq, uint32_t kvh, uint32_t chunk,
                                                    const RM& red_m, const RM& red_l, const RA& red_acc) {
    float* part = a.part + (((size_t)seq * a.n_heads + (size_t)kvh * G) * a.cstride + chunk) * (2 + LK_HD);
    for (int t = threadIdx.x; t < G * LK_HD; t += LK_AW * 64) {
        const int g = t / LK_HD, d = t % LK_HD;
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < LK_AW; ww++) M = fmaxf(M, red_m[ww][g]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int ww = 0; ww < LK_AW; ww++) {
            if (red_m[ww][g] != -INFINITY) {
                const float sc = expf(red_m[ww][g] - M);
                L = fmaf(sc, red_l[ww][g], L);
                A = fmaf(sc, red_acc[ww][g][d], A);
            }
        }
        float* ph = part + (size_t)g * a.cstride * (2 + LK_HD);
        if (d == 0) {
            st_coherent(ph, M);
            st_coherent(ph + 1, L);
        }
        st_coherent(ph + 2 + d, A);
    }
}

template <int G, typename KV>
__global__ __launch_bounds__(LK_AW * 64) void attn_partial_kernel(const LkAttnArgs a) {
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const uint32_t ctx = attn_ctx(a, seq);
    const uint32_t A = a.waves, T = a.tiles, CH = 64 * A * T;
    const uint32_t c0 = chunk * CH;
    if (c0 >= ctx) return;  // uniform over the block
    const uint32_t nch = (ctx + CH - 1) / CH;
    const uint32_t slot = a.slots ? a.slots[seq] : seq;
    const size_t kv_base = (size_t)slot * a.seq_stride + (size_t)kvh * a.max_seq * LK_HD;
    const KV* __restrict__ K = (const KV*)a.k + kv_base;
    const KV* __restrict__ V = (const KV*)a.v + kv_base;

    __shared__ float qs[G][LK_HD];
    __shared__ float ps[LK_AW][G][64];      // [wave][head][group * 8 + jj]
    __shared__ float red_m[LK_AW][G], red_l[LK_AW][G];
    __shared__ float red_acc[LK_AW][G][LK_HD];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t plast = ctx - 1;
    const float* qsrc = a.q + (size_t)seq * a.q_stride + (size_t)kvh * G * LK_HD;
    for (int i = tid; i < G * LK_HD; i += LK_AW * 64) qs[i / LK_HD][i % LK_HD] = qsrc[i];
    __syncthreads();

    // P.V lane map: position group sub = lane & 7, dims dq..dq+7 (dq = 8 * (lane >> 3))
    const uint32_t sub = (uint32_t)lane & 7, dq = ((uint32_t)lane >> 3) * 8;
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.f;
    }
    for (uint32_t t = 0; t < T && (uint32_t)w < A; t++) {
        const uint32_t p0 = c0 + ((uint32_t)w + A * t) * 64;
        if (p0 >= ctx) break;  // wave-uniform
        // Straight-line loads: positions past ctx re-read the last live row (in
        // bounds) and are masked below.  K: lane = position, its whole 64-dim row.
        const uint32_t p = p0 + (uint32_t)lane;
        const KV* krow = K + (size_t)(p < ctx ? p : plast) * LK_HD;
        float kf[LK_HD];
#pragma unroll
        for (int i = 0; i < 8; i++) load8(krow + 8 * i, kf + 8 * i);
        // V for the P.V pass, issued before the scores so it is in flight meanwhile
        float vf[8][8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const uint32_t pj = p0 + (uint32_t)jj * 8 + sub;
            load8(V + (size_t)(pj < ctx ? pj : plast) * LK_HD + dq, vf[jj]);
        }
        // ---- scores: lane = position, q rows by LDS broadcast
        const bool valid = p < ctx;
        float s[G];
#pragma unroll
        for (int g = 0; g < G; g++) s[g] = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float4 qv = *(const float4*)&qs[g][4 * i];
                float u = s[g];
                u = fmaf(kf[4 * i], qv.x, u);
                u = fmaf(kf[4 * i + 1], qv.y, u);
                u = fmaf(kf[4 * i + 2], qv.z, u);
                u = fmaf(kf[4 * i + 3], qv.w, u);
                s[g] = u;
            }
        }
        // online softmax across this wave's tiles
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float sg = valid ? s[g] * 0.125f : -INFINITY;
            const float mn = fmaxf(m[g], lk_wave_max(sg));  // finite: the tile holds a live position
            const float sc = expf(m[g] - mn);                // 0 on the wave's first tile
            const float pg = valid ? expf(sg - mn) : 0.f;
            l[g] = fmaf(l[g], sc, lk_wave_sum(pg));
            m[g] = mn;
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] *= sc;
            ps[w][g][(lane & 7) * 8 + (lane >> 3)] = pg;  // position lane -> [group][jj]
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's P is in LDS
        __builtin_amdgcn_wave_barrier();
        // ---- P.V (weights of masked positions are 0 and their V rows are finite)
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float pw = ps[w][g][sub * 8 + jj];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] = fmaf(pw, vf[jj][e], acc[g][e]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // the P reads are done before the next tile rewrites ps
        __builtin_amdgcn_wave_barrier();
    }
    // sum the 8 position groups of each dims chunk (8 adjacent lanes) by
    // DPP: quad pairs, quad halves, row_ror 4 -> lanes 4..7 of each 8 hold it
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = acc[g][e];
            v += lk_dpp<0xB1, 0xF>(v, 0.f);
            v += lk_dpp<0x4E, 0xF>(v, 0.f);
            v += lk_dpp<0x124, 0xF>(v, 0.f);
            acc[g][e] = v;
        }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            red_m[w][g] = m[g];  // -inf for a wave with no live tile
            red_l[w][g] = l[g];
        }
    }
    if ((lane & 7) == 4) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) red_acc[w][g][dq + e] = acc[g][e];
    }
    __syncthreads();
    write_chunk_partial<G>(a, seq, kvh, chunk, red_m, red_l, red_acc);
    count_in_and_fold<G>(a, seq, kvh, nch);
}

// The f16-cache partial on the matrix cores.  Same block/tile split as
// attn_partial_kernel (a chunk of 256*T positions per block, 64-position
// tiles w, w+4, ... per wave), with both products of a tile on
// v_mfma_f32_16x16x16f16:
//   scores : S[pos][head] = K . q, 16 positions x 16 heads (G used) per MFMA,
//            K rows exact in f16, q split into f16 hi + lo (22 significant
//            bits), f32 accumulation.  MFMA row m of sub-tile t is position
//            16t + 4(m & 3) + (m >> 2) (a fixed permutation, shared by P.V);
//            lane l holds that row of K for m = l & 15, dims 16*(l >> 4) ..
//            +15 -- the same dims for q -- so a wave's K load is 16 whole
//            128-byte rows;
//   softmax: per head (lane & 15) over the tile's 64 positions, folded into
//            the wave's running (max, sum, O) across its tiles;
//   P.V    : O[head][dim] = P . V with P straight from the score registers
//            (lane l holds P[head l & 15][positions 4*(l >> 4) .. +3], exactly
//            the A-operand layout), split hi + lo like q, and V read back from
//            LDS in the B-operand layout: the tile is staged there by
//            coalesced 16-byte loads, and a lane reads 4 dims of each of its
//            4 positions with one 8-byte LDS read (MFMA d of a sub-tile takes
//            dim 4n + d for column n).  With the row permutation the two
//            16-lane groups of a half-wave read rows of opposite parity, i.e.
//            disjoint LDS banks.
// At GQA 7 this is ~1/5 of the vector-ALU work of the scalar kernel, whose
// FMA rate per HBM byte is close to the ALU's.
typedef _Float16 lk_h4 __attribute__((ext_vector_type(4)));
typedef float lk_f4 __attribute__((ext_vector_type(4)));
typedef unsigned int lk_u4 __attribute__((ext_vector_type(4)));
#define LK_VS 64  // LDS row stride of a staged V tile (halves)

__device__ __forceinline__ lk_h4 h4_bits(uint32_t lo, uint32_t hi) {
    const uint2 u = make_uint2(lo, hi);
    return __builtin_bit_cast(lk_h4, u);
}

template <int G>
__global__ __launch_bounds__(LK_AW * 64) void attn_mfma_kernel(const LkAttnArgs a) {
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const uint32_t ctx = attn_ctx(a, seq);
    const uint32_t A = a.waves, T = a.tiles, CH = 64 * A * T;
    const uint32_t c0 = chunk * CH;
    if (c0 >= ctx) return;  // uniform over the block
    const uint32_t nch = (ctx + CH - 1) / CH;
    const uint32_t slot = a.slots ? a.slots[seq] : seq;
    const size_t kv_base = (size_t)slot * a.seq_stride + (size_t)kvh * a.max_seq * LK_HD;
    const uint16_t* __restrict__ K = (const uint16_t*)a.k + kv_base;
    const uint16_t* __restrict__ V = (const uint16_t*)a.v + kv_base;

    // the staged V tiles, reused for the waves' O tiles once all P.V are done
    __shared__ __align__(16) uint16_t vs[LK_AW][64 * LK_VS];
    __shared__ float red_m[LK_AW][16], red_l[LK_AW][16];
    float(*red_acc)[16][LK_HD] = (float(*)[16][LK_HD])&vs[0][0];
    static_assert(sizeof(vs) >= LK_AW * 16 * LK_HD * sizeof(float), "O tiles fit the V staging area");

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t j = (uint32_t)lane >> 4, c16 = (uint32_t)lane & 15;
    const uint32_t plast = ctx - 1;

    // q of head c16 (zero past G), dims 16j + 4s .. +3 for step s, as f16 hi + lo
    lk_h4 qh[4], ql[4];
    {
        const float* qrow = a.q + (size_t)seq * a.q_stride + ((size_t)kvh * G + (c16 < (uint32_t)G ? c16 : 0)) * LK_HD;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const float4 v = *(const float4*)(qrow + 16 * j + 4 * st);
            const float x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float xv = c16 < (uint32_t)G ? x[e] : 0.f;
                const _Float16 hi = (_Float16)xv;
                qh[st][e] = hi;
                ql[st][e] = (_Float16)(xv - (float)hi);
            }
        }
    }
    // running (max, sum) of head c16 and O (lane: heads 4j + i, dim 4 c16 + d)
    float mt = -INFINITY, lt = 0.f;
    lk_f4 o[4];
#pragma unroll
    for (int d = 0; d < 4; d++) o[d] = lk_f4{0.f, 0.f, 0.f, 0.f};
    uint16_t* vw = vs[w];
    for (uint32_t tt = 0; tt < T && (uint32_t)w < A; tt++) {
        const uint32_t p0 = c0 + ((uint32_t)w + A * tt) * 64;
        if (p0 >= ctx) break;  // wave-uniform
        // K: sub-tile t rows p0 + 16t + c16, this lane's 32 bytes (dims 16j..16j+15);
        // V: rows p0 + 8it + (lane >> 3), bytes 16*(lane & 7) -- 1 KiB per instruction
        uint4 kr[4][2];
        lk_u4 vr[8];  // a vector type (not the uint4 struct): held in registers, not in scratch
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t p = p0 + 16u * t + 4u * (c16 & 3) + (c16 >> 2);  // MFMA row c16
            const uint4* src = (const uint4*)(K + (size_t)(p < ctx ? p : plast) * LK_HD + 16 * j);
            kr[t][0] = src[0];
            kr[t][1] = src[1];
        }
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const uint32_t p = p0 + 8u * it + ((uint32_t)lane >> 3);
            vr[it] = *(const lk_u4*)(V + (size_t)(p < ctx ? p : plast) * LK_HD + 8 * (lane & 7));
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the previous tile's V reads are done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int it = 0; it < 8; it++)
            *(lk_u4*)&vw[(8 * it + (lane >> 3)) * LK_VS + 8 * (lane & 7)] = vr[it];
        // ---- scores
        lk_f4 sc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            lk_f4 acc = lk_f4{0.f, 0.f, 0.f, 0.f};
            const uint32_t kw[8] = {kr[t][0].x, kr[t][0].y, kr[t][0].z, kr[t][0].w,
                                    kr[t][1].x, kr[t][1].y, kr[t][1].z, kr[t][1].w};
#pragma unroll
            for (int st = 0; st < 4; st++) {
                const lk_h4 kk = h4_bits(kw[2 * st], kw[2 * st + 1]);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kk, qh[st], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kk, ql[st], acc, 0, 0, 0);
            }
            sc[t] = acc;  // lane: positions p0 + 16t + 4j + i, head c16
        }
        // ---- softmax over the tile's 64 positions, per head (lanes c16, +16, +32, +48)
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t p = p0 + 16u * t + 4u * (uint32_t)i + j;  // MFMA row 4j + i
                const float v = p < ctx ? sc[t][i] * 0.125f : -INFINITY;
                sc[t][i] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mn = fmaxf(mt, mx);    // finite: the tile holds a live position
        const float fo = expf(mt - mn);    // the running sums' factor (0 on the first tile)
        float sum = 0.f;
        lk_h4 ph[4], pl[4];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pe = expf(sc[t][i] - mn);  // 0 for masked positions
                sum += pe;
                const _Float16 hi = (_Float16)pe;
                ph[t][i] = hi;
                pl[t][i] = (_Float16)(pe - (float)hi);
            }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        lt = fmaf(lt, fo, sum);
        mt = mn;
        // O's heads are 4j + i: their factors live on lanes 4j + i
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float f = __shfl(fo, (int)(4 * j + i), 64);
#pragma unroll
            for (int d = 0; d < 4; d++) o[d][i] *= f;
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the V tile is in LDS
        __builtin_amdgcn_wave_barrier();
        // ---- P.V: k = 4j + i <-> position 16t + 4i + j, n = c16 <-> dim 4 c16 + d
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint2 r[4];  // dims 4 c16 .. +3 of positions 16t + 4i + j
#pragma unroll
            for (int i = 0; i < 4; i++) r[i] = *(const uint2*)&vw[(16 * t + 4 * i + j) * LK_VS + 4 * c16];
#pragma unroll
            for (int d = 0; d < 4; d++) {
                // halves d of the four rows, paired into two dwords
                const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u;
                const uint32_t v01 = __builtin_amdgcn_perm(d < 2 ? r[1].x : r[1].y, d < 2 ? r[0].x : r[0].y, sel);
                const uint32_t v23 = __builtin_amdgcn_perm(d < 2 ? r[3].x : r[3].y, d < 2 ? r[2].x : r[2].y, sel);
                const lk_h4 vb = h4_bits(v01, v23);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph[t], vb, o[d], 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl[t], vb, o[d], 0, 0, 0);
            }
        }
    }
    // o[d] lane: heads 4j + i, dim 4 c16 + d (relative to this wave's max)
    __syncthreads();  // every wave is done with its V tile
    if (j == 0) {
        red_m[w][c16] = mt;  // -inf for a wave with no live tile
        red_l[w][c16] = lt;
    }
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int i = 0; i < 4; i++) red_acc[w][4 * j + i][4 * c16 + d] = o[d][i];
    __syncthreads();
    write_chunk_partial<G>(a, seq, kvh, chunk, red_m, red_l, red_acc);
    count_in_and_fold<G>(a, seq, kvh, nch);
}

hipError_t lk_attn_launch(const LkAttnArgs& args, hipStream_t st) {
    if (args.n_kv == 0 || args.n_heads % args.n_kv || !args.cnt || !args.max_seq) return hipErrorInvalidValue;
    LkAttnArgs a = args;
    const AttnPlan p = attn_plan(a.n_seq, a.n_kv, a.max_seq);
    a.waves = p.waves;
    a.tiles = p.tiles;
    a.cstride = attn_chunk_cap(a.max_seq);
    const uint32_t G = a.n_heads / a.n_kv;
    dim3 grid(p.chunks, a.n_kv, a.n_seq);
    // The matrix-core kernel is the faster one at every context measured (4
    // sequences x 24 layers: 268 vs 327 us per step at ctx 4096, 562 vs 690
    // at 32768); LKHIP_ATTN=valu selects the vector-ALU kernel.
    const char* fe = getenv("LKHIP_ATTN");
    const bool mfma = !(fe && strcmp(fe, "valu") == 0);
#define LK_ATTN_CASE(g)                                                                         \
    case g:                                                                                     \
        if (a.kv_f32) hipLaunchKernelGGL((attn_partial_kernel<g, float>), grid, dim3(LK_AW * 64), 0, st, a); \
        else if (mfma) hipLaunchKernelGGL((attn_mfma_kernel<g>), grid, dim3(LK_AW * 64), 0, st, a);     \
        else hipLaunchKernelGGL((attn_partial_kernel<g, uint16_t>), grid, dim3(LK_AW * 64), 0, st, a);  \
        break;
    switch (G) {
        LK_ATTN_CASE(1)
        LK_ATTN_CASE(2)
        LK_ATTN_CASE(3)
        LK_ATTN_CASE(4)
        LK_ATTN_CASE(5)
        LK_ATTN_CASE(6)
        LK_ATTN_CASE(7)
        LK_ATTN_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef LK_ATTN_CASE
    return hipGetLastError();
}
