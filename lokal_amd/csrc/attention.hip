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
// cache is short, smaller chunks (A < 8) so the grid still has >= 128 blocks,
// unless there are >= 64 (sequence, kv head) pairs: then one chunk each,
// which writes the output itself (no partial, count or fold).
// Few large chunks beat many small ones: each chunk costs a partial write,
// an atomic on its counter and a share of the fold, and those counters sit
// 256 bytes apart so the atomics of different (sequence, kv head) do not
// contend for one cache line.
// fp32 throughout; scale 1/sqrt(64) = 0.125 is exact.
#include "lkhip_common.h"

#include <cstdlib>
#include <cstring>
#include <mutex>

#include "attention_impl.h"


// Partial slots per (sequence, head): every plan's chunk holds >= 64 positions.
static inline uint32_t attn_chunk_cap(uint32_t max_seq) {
    const uint32_t t = (max_seq + 63) / 64;
    return t < LK_MAXCH ? t : LK_MAXCH;
}
struct AttnPlan {
    uint32_t waves, tiles, chunks;  // active waves per block, tiles per wave, chunks per (seq, kvh)
};
#ifndef LK_ATTN_ONE_PAIRS
#define LK_ATTN_ONE_PAIRS 64
#endif
// The largest A in 8, 4, 2, 1 whose grid has >= LK_ATTN_MINBLOCKS blocks,
// else the one with the most blocks (the larger A on a tie), with T the
// fewest tiles per wave that keep the chunks per (seq, kvh) <= LK_MAXCH.
static AttnPlan attn_plan(uint32_t n_seq, uint32_t n_kv, uint32_t max_seq) {
    AttnPlan best{};
    // Many (sequence, kv head) pairs over a short cache: one chunk each (all
    // 8 waves, at most 2 tiles per wave), whose block writes the output
    // directly -- no partial, count or fold.  Batcher steps of 32 / 64 rows
    // 1.78 / 2.03 -> 1.745 / 1.99 ms, 512-token prefill 4.73 -> 4.45 ms; at
    // 32 pairs (16 rows) the chunked plan's parallelism wins (1.455 against
    // 1.487 ms).
    if ((uint64_t)n_seq * n_kv >= LK_ATTN_ONE_PAIRS && max_seq <= 2 * 64 * LK_AW) {
        best.waves = LK_AW;
        best.tiles = (max_seq + 64 * LK_AW - 1) / (64 * LK_AW);
        best.chunks = 1;
        return best;
    }
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
uint32_t lk_attn_set_plan(LkAttnArgs& a) {
    const AttnPlan p = attn_plan(a.n_seq, a.n_kv, a.max_seq);
    a.waves = p.waves;
    a.tiles = p.tiles;
    a.cstride = attn_chunk_cap(a.max_seq);
    return p.chunks;
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
    write_chunk_partial<G>(a, seq, kvh, chunk, nch, red_m, red_l, red_acc);
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
template <int G, int PR, bool ROPE = false>
__global__ __launch_bounds__(LK_AW * 64) void attn_mfma_kernel(const LkAttnArgs a) {
    attn_mfma_item<G, PR, ROPE>(a, blockIdx.x, blockIdx.y, blockIdx.z * PR);
}
// Rows per item of a grouped (prefill) launch: as many as fill the 16 MFMA columns.
static constexpr uint32_t attn_rows_per_item(uint32_t G) { return 16 / G; }

hipError_t lk_attn_launch(const LkAttnArgs& args, hipStream_t st) {
    if (args.n_kv == 0 || args.n_heads % args.n_kv || !args.cnt || !args.max_seq) return hipErrorInvalidValue;
    LkAttnArgs a = args;
    const uint32_t G = a.n_heads / a.n_kv;
    // The matrix-core kernel is the faster one at every context measured (4
    // sequences x 24 layers: 268 vs 327 us per step at ctx 4096, 562 vs 690
    // at 32768); LKHIP_ATTN=valu selects the vector-ALU kernel.
    const char* fe = getenv("LKHIP_ATTN");
    const bool mfma = !(fe && strcmp(fe, "valu") == 0);
    // a prefill chunk on the matrix-core kernel: several rows per item, so a
    // K/V tile is read once for all of them
    const bool group = a.grouped && !a.kv_f32 && mfma && G <= 8;
    if (a.rope && (a.kv_f32 || group || !mfma)) {
        // the RoPE + KV append as its own launch first: only the one-row f16
        // matrix-core kernel does it in the attention launch
        const hipError_t e = lk_rows_rope_kv_launch((float*)a.q, a.rope_part, a.rope_ks, a.bq, a.bk, a.bv, a.n_heads,
                                                    a.n_kv, a.freq, a.pos_rows, a.n_seq, (void*)a.k, (void*)a.v,
                                                    (int)a.kv_f32, a.max_seq, a.seq_stride, a.slots, st);
        if (e != hipSuccess) return e;
        a.rope = 0;
    }
    const uint32_t pr = group ? attn_rows_per_item(G) : 1;
    const uint32_t items = (a.n_seq + pr - 1) / pr;
    const AttnPlan p = attn_plan(items, a.n_kv, a.max_seq);
    a.waves = p.waves;
    a.tiles = p.tiles;
    a.cstride = attn_chunk_cap(a.max_seq);
    dim3 grid(p.chunks, a.n_kv, items);
#define LK_ATTN_CASE(g)                                                                         \
    case g:                                                                                     \
        if (a.kv_f32) hipLaunchKernelGGL((attn_partial_kernel<g, float>), grid, dim3(LK_AW * 64), 0, st, a); \
        else if (group) hipLaunchKernelGGL((attn_mfma_kernel<g, attn_rows_per_item(g)>), grid, dim3(LK_AW * 64), 0, st, a); \
        else if (mfma && a.rope) hipLaunchKernelGGL((attn_mfma_kernel<g, 1, true>), grid, dim3(LK_AW * 64), 0, st, a); \
        else if (mfma) hipLaunchKernelGGL((attn_mfma_kernel<g, 1>), grid, dim3(LK_AW * 64), 0, st, a);     \
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
