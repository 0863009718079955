// attention_impl.h -- device code of the GQA flash-decoding attention
// (attention.hip), shared with the Batcher's persistent step (batch_step.hip):
// the chunk item on the matrix cores, the chunk partials, and the
// last-arriving block's fold.  See attention.hip for the algorithm.
#pragma once
#include "lkhip_common.h"

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
// The attention output: write-through (COH) where a later phase of the same
// launch reads it on another XCD (the persistent Batcher step), else a plain
// store -- agent-scope atomic loads and stores cost 8-16% per standalone
// launch (4 sequences x 24 layers at 4096-32768 positions, measured).
template <bool COH>
__device__ __forceinline__ void st_out(float* p, float v) {
    if constexpr (COH) st_coherent(p, v);
    else *p = v;
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
// Memory order of the arrival count: relaxed.  The partials are agent-scope
// atomic stores, which on this target write through to the memory-side
// cache, and s_waitcnt vmcnt(0) + the block barrier complete them before the
// count is incremented; the folding block reads them with agent-scope loads,
// which bypass the non-coherent caches.  So the fold sees every chunk's words
// by the hardware's ordering of write-through stores and the count; the HIP
// memory model alone would need release/acquire on the count.  Built with
// LK_ATTN_FOLD_ORDER=__ATOMIC_ACQ_REL the release writes back and the acquire
// invalidates the L2 on every block: measured on MI355X (4 sequences x 24
// layers) 256 against 228 us per step at 4096 positions, 405 against 352 at
// 16384, 533 against 496 at 32768.
#ifndef LK_ATTN_FOLD_ORDER
#define LK_ATTN_FOLD_ORDER __ATOMIC_RELAXED
#endif

// PR > 1: the item covers rows seq .. seq + PR - 1 (consecutive positions of
// one sequence, a prefill chunk), column c = (row c / G, head c % G); the
// count is the first row's.
template <int G, int PR = 1, bool COH = false>
__device__ __forceinline__ void count_in_and_fold(const LkAttnArgs& a, uint32_t seq, uint32_t kvh, uint32_t nch) {
    if (nch == 1) return;  // write_chunk_partial wrote the output itself
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
    for (int r = 0; r < (G * PR + LK_AW - 1) / LK_AW; r++) {
        const uint32_t cg = (uint32_t)w + LK_AW * r;
        if (cg >= (uint32_t)(G * PR)) break;
        const uint32_t rs = PR == 1 ? seq : seq + cg / G, g = PR == 1 ? cg : cg % G;
        if (PR > 1 && rs >= a.n_seq) break;  // a ragged last group
        const uint32_t h = kvh * G + g;
        const float* ph = a.part + ((size_t)rs * a.n_heads + h) * a.cstride * (2 + LK_HD);
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
        // write-through: read by another XCD later in the same launch (the
        // persistent Batcher step's o_proj phase)
        st_out<COH>(a.out + ((size_t)rs * a.n_heads + h) * LK_HD + lane, A / L);
    }
    if (tid == 0)
        __hip_atomic_store(a.cnt + ((size_t)seq * a.n_kv + kvh) * LK_ATTN_CNT_STRIDE, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// The 4 waves' (m, l, acc) of each head (red_m[w][g] etc.) -> the chunk's
// partial per head, with coherent stores.  The only chunk of its (sequence,
// kv head) (nch == 1) writes the output acc / l instead: the fold would
// weight that one partial by exp(0) = 1 and return the same quotient, so the
// partial store, the count and the fold's reads are skipped.
// PR > 1: columns c = (row seq + c / G, head c % G), as in count_in_and_fold.
template <int G, int PR = 1, bool COH = false, typename RM, typename RA>
__device__ __forceinline__ void write_chunk_partial(const LkAttnArgs& a, uint32_t seq, uint32_t kvh, uint32_t chunk,
                                                    uint32_t nch, const RM& red_m, const RM& red_l,
                                                    const RA& red_acc) {
    float* const part1 = a.part + (((size_t)seq * a.n_heads + (size_t)kvh * G) * a.cstride + chunk) * (2 + LK_HD);
    for (int t = threadIdx.x; t < G * PR * LK_HD; t += LK_AW * 64) {
        const int g = t / LK_HD, d = t % LK_HD;  // g: the column
        float* part;
        if constexpr (PR == 1) {
            part = part1 + (size_t)g * a.cstride * (2 + LK_HD);
        } else {
            const uint32_t rs = seq + (uint32_t)g / G;
            if (rs >= a.n_seq) break;  // a ragged last group (t only grows)
            part = a.part + (((size_t)rs * a.n_heads + (size_t)kvh * G + (uint32_t)g % G) * a.cstride + chunk) *
                                (2 + LK_HD);
        }
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
        if (nch == 1) {
            // write-through, as the fold's output: read by another XCD later
            // in the same launch (the persistent Batcher step's o_proj phase)
            const uint32_t rs = PR == 1 ? seq : seq + (uint32_t)g / G, hg = PR == 1 ? (uint32_t)g : (uint32_t)g % G;
            st_out<COH>(a.out + ((size_t)rs * a.n_heads + kvh * G + hg) * LK_HD + d, A / L);
            continue;
        }
        float* ph = part;
        if (d == 0) {
            st_coherent(ph, M);
            st_coherent(ph + 1, L);
        }
        st_coherent(ph + 2 + d, A);
    }
}


typedef _Float16 lk_h4 __attribute__((ext_vector_type(4)));
typedef float lk_f4 __attribute__((ext_vector_type(4)));
typedef unsigned int lk_u4 __attribute__((ext_vector_type(4)));
#define LK_VS 64  // LDS row stride of a staged V tile (halves)

__device__ __forceinline__ lk_h4 h4_bits(uint32_t lo, uint32_t hi) {
    const uint2 u = make_uint2(lo, hi);
    return __builtin_bit_cast(lk_h4, u);
}

// One (chunk, kv head, sequence) item of the f16-cache partial on the matrix
// cores, by a block of LK_AW waves: attn_mfma_kernel runs one item per block;
// the Batcher's persistent step (batch_step.hip) runs them in its attention
// phase.  PR > 1 (a prefill chunk: rows seq .. seq + PR - 1 are consecutive
// positions of one sequence, so they share its K/V): the item takes the PR
// rows' G heads as the MFMA's G * PR <= 16 columns, column c = (row c / G,
// head c % G), and each K/V tile is read once for all of them; a column's
// positions past its own row's are masked (causal).
template <int G, int PR = 1, bool ROPE = false, bool COH = false>
__device__ __forceinline__ void attn_mfma_item(const LkAttnArgs& a, uint32_t chunk, uint32_t kvh, uint32_t seq) {
    static_assert(!ROPE || PR == 1, "RoPE in the attention launch is for one-row items");
    static_assert(G * PR <= 16, "the item's columns fit one 16-column MFMA tile");
    // the item's context: its last row's (positions grow along the rows)
    const uint32_t rlast = PR == 1 ? seq : (seq + PR - 1 < a.n_seq ? seq + PR - 1 : a.n_seq - 1);
    const uint32_t ctx = attn_ctx(a, rlast);
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
    // this lane's column: row seq + crow, head cg; live columns c16 < G * PR
    // of rows inside the call
    const uint32_t crow = PR == 1 ? 0 : (c16 / G < (uint32_t)PR ? c16 / G : 0);
    const uint32_t cg = PR == 1 ? (c16 < (uint32_t)G ? c16 : 0) : c16 % G;
    const bool clive = PR == 1 ? c16 < (uint32_t)G : (c16 < (uint32_t)(G * PR) && seq + crow < a.n_seq);
    const uint32_t cctx = PR > 1 ? attn_ctx(a, clive ? seq + crow : seq) : ctx;  // the column's causal bound

    // LkAttnArgs::rope: this row's q heads of kv head kvh rotated into rq, and,
    // in the block whose chunk holds position plast, the row's k / v (rounded
    // to f16) into rkh / rvh and the cache
    __shared__ float rq[ROPE ? G * LK_HD : 1];
    __shared__ __align__(16) uint16_t rkh[ROPE ? LK_HD : 8], rvh[ROPE ? LK_HD : 8];
    constexpr bool rope = ROPE;
    const bool own_pos = ROPE && plast < c0 + CH;  // c0 <= plast: c0 < ctx
    if constexpr (ROPE) {
        const uint32_t qd = a.n_heads * LK_HD, kvd = a.n_kv * LK_HD;
        const float fpos = (float)plast;
        // element idx of the row's q | k | v: split-K partials summed in
        // split order, then the bias (rows_rope_kv_kernel's order)
        auto val = [&](uint32_t idx, const float* bias, uint32_t bi) -> float {
            if (!a.rope_ks) return a.q[(size_t)seq * a.q_stride + idx];
            const float sum = lk_sum_splits(a.rope_part + (size_t)seq * a.q_stride + idx,
                                             (size_t)a.n_seq * a.q_stride, a.rope_ks);
            return bias ? sum + bias[bi] : sum;
        };
        const uint32_t nq = G * 32, nt = nq + (own_pos ? 32 + LK_HD : 0);
        for (uint32_t t = (uint32_t)tid; t < nt; t += LK_AW * 64) {
            if (t < nq) {
                const uint32_t g = t / 32, i = t % 32, o = (kvh * G + g) * LK_HD + i;
                float x0 = val(o, a.bq, o), x1 = val(o + 32, a.bq, o + 32);
                lk_rot_pair(x0, x1, __fmul_rn(fpos, a.freq.f[i]));
                rq[g * LK_HD + i] = x0;
                rq[g * LK_HD + i + 32] = x1;
            } else if (t < nq + 32) {
                const uint32_t i = t - nq, o = kvh * LK_HD + i;
                float x0 = val(qd + o, a.bk, o), x1 = val(qd + o + 32, a.bk, o + 32);
                lk_rot_pair(x0, x1, __fmul_rn(fpos, a.freq.f[i]));
                const uint16_t h0 = __half_as_ushort(__float2half_rn(x0)), h1 = __half_as_ushort(__float2half_rn(x1));
                rkh[i] = h0;
                rkh[i + 32] = h1;
                uint16_t* Kw = (uint16_t*)a.k + kv_base + (size_t)plast * LK_HD;
                Kw[i] = h0;
                Kw[i + 32] = h1;
            } else {
                const uint32_t d = t - nq - 32, o = kvh * LK_HD + d;
                const uint16_t hv = __half_as_ushort(__float2half_rn(val(qd + kvd + o, a.bv, o)));
                rvh[d] = hv;
                ((uint16_t*)a.v)[kv_base + (size_t)plast * LK_HD + d] = hv;
            }
        }
        __syncthreads();
    }

    // q of column c16 (zero for a dead column), dims 16j + 4s .. +3 for step s, as f16 hi + lo
    lk_h4 qh[4], ql[4];
    {
        const float* qrow = a.q + (size_t)(seq + (clive ? crow : 0u)) * a.q_stride + ((size_t)kvh * G + cg) * LK_HD;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            float x[4];
            if constexpr (rope) {
                const float4 r4 = *(const float4*)&rq[cg * LK_HD + 16 * j + 4 * st];
                x[0] = r4.x, x[1] = r4.y, x[2] = r4.z, x[3] = r4.w;
            } else if constexpr (!COH) {
                const float4 r4 = *(const float4*)(qrow + 16 * j + 4 * st);
                x[0] = r4.x, x[1] = r4.y, x[2] = r4.z, x[3] = r4.w;
            } else {
                // q written earlier in the same launch by another XCD
                x[0] = ld_coherent(qrow + 16 * j + 4 * st);
                x[1] = ld_coherent(qrow + 16 * j + 4 * st + 1);
                x[2] = ld_coherent(qrow + 16 * j + 4 * st + 2);
                x[3] = ld_coherent(qrow + 16 * j + 4 * st + 3);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float xv = clive ? x[e] : 0.f;
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
        if (ROPE && own_pos && plast < p0 + 64) {
            // this tile holds position plast: its K / V row (and the clamped
            // rows past it, masked below) from rkh / rvh, not the cache row
            // this launch is writing
            const uint4 k0 = *(const uint4*)&rkh[16 * j], k1 = *(const uint4*)&rkh[16 * j + 8];
            const lk_u4 vv = *(const lk_u4*)&rvh[8 * (lane & 7)];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t p = p0 + 16u * t + 4u * (c16 & 3) + (c16 >> 2);
                if (p >= plast) {
                    kr[t][0] = k0;
                    kr[t][1] = k1;
                }
            }
#pragma unroll
            for (int it = 0; it < 8; it++)
                if (p0 + 8u * it + ((uint32_t)lane >> 3) >= plast) vr[it] = vv;
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
                const float v = p < cctx ? sc[t][i] * 0.125f : -INFINITY;
                sc[t][i] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // finite for PR == 1: the tile holds a live position.  PR > 1: a
        // column may have none yet (its row ends before the tile); it keeps
        // (-inf, 0, 0) with any finite reference for the exponentials
        const float mn0 = fmaxf(mt, mx);
        const float mn = (PR > 1 && mn0 == -INFINITY) ? 0.f : mn0;
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
        mt = mn0;
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
    write_chunk_partial<G, PR, COH>(a, seq, kvh, chunk, nch, red_m, red_l, red_acc);
    count_in_and_fold<G, PR, COH>(a, seq, kvh, nch);
}
