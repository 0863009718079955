// attention.hip -- GQA flash-decoding over the f16 KV cache (model::attention,
// src/model.rs:286-318, computed split-K over positions and merged).
//
// One block = one (sequence, kv head, 256-position chunk).  The G query heads
// that share the kv head are staged in LDS, so every K and V byte of the chunk
// is read from HBM exactly once for the whole group.  Each of the 4 waves owns
// a 64-position tile:
//   scores : lane = position, the K row (128 B) is converted once and dotted
//            against all G query rows (LDS broadcast reads);
//   softmax: per-tile max / exp / sum by wave reductions;
//   P.V    : lane = (position group lane & 7, 8 dims), one 16-byte V load per
//            lane covers 8 positions x 64 dims per instruction; the 8 lanes that
//            share a dim slice are combined by DPP.
// Loads are straight-line (positions past ctx re-read the last live row and
// are masked), issued before the dependent arithmetic.
// The 4 tiles merge in LDS into one (m, l, acc[64]) partial per query head;
// attn_merge_kernel folds the partials of all chunks with the usual
// max-rescaled sums.  fp32 throughout; scale 1/sqrt(64) = 0.125 is exact.
#include "lkhip_common.h"

#include <cstdlib>
#include <cstring>
#include <mutex>

#define LK_HD 64
#ifndef LK_ACHUNK
#define LK_ACHUNK 256
#endif
#define LK_AW (LK_ACHUNK / 64)  // waves per partial block: one 64-position tile each
#define LK_MB 32  // chunks per merge wave and round

uint32_t lk_attn_chunk(uint32_t) { return LK_ACHUNK; }

// Fixed partial buffer of lkhip_attn_decode_noalloc, for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops).  Each
// device holds its own copy for the life of the process.  In host code the
// array's name is only a stand-in: its device address comes from
// hipGetSymbolAddress, once per device (lk_attn_scratch below), and only that
// address is ever passed to a kernel.  Every call on a device shares it, so
// calls that overlap on one device race.
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
    const size_t nch = (max_seq + LK_ACHUNK - 1) / LK_ACHUNK;
    return (size_t)n_seq * n_heads * nch * (2 + LK_HD);
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

template <int G, typename KV>
__global__ __launch_bounds__(LK_AW * 64) void attn_partial_kernel(const LkAttnArgs a) {
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const uint32_t ctx = attn_ctx(a, seq);
    const uint32_t c0 = chunk * LK_ACHUNK;
    if (c0 >= ctx) return;  // uniform over the block
    const uint32_t max_chunks = (a.max_seq + LK_ACHUNK - 1) / LK_ACHUNK;
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
    const uint32_t p0 = c0 + (uint32_t)w * 64;
    const bool tile_live = p0 < ctx;  // wave-uniform
    const uint32_t plast = ctx - 1;
    // Straight-line loads: positions past ctx re-read the last live row (in
    // bounds) and are masked below.  K: lane = position, its whole 64-dim row.
    const uint32_t p = p0 + (uint32_t)lane;
    const KV* krow = K + (size_t)(p < ctx ? p : plast) * LK_HD;
    float kf[LK_HD];
    if (tile_live) {
#pragma unroll
        for (int i = 0; i < 8; i++) load8(krow + 8 * i, kf + 8 * i);
    }
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
    if (tile_live) {
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
                float t = s[g];
                t = fmaf(kf[4 * i], qv.x, t);
                t = fmaf(kf[4 * i + 1], qv.y, t);
                t = fmaf(kf[4 * i + 2], qv.z, t);
                t = fmaf(kf[4 * i + 3], qv.w, t);
                s[g] = t;
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float sg = valid ? s[g] * 0.125f : -INFINITY;
            m[g] = lk_wave_max(sg);
            const float pg = valid ? expf(sg - m[g]) : 0.f;
            l[g] = lk_wave_sum(pg);
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
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            red_m[w][g] = m[g];
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

    // ---- merge the 4 tiles into one partial per query head
    float* part = a.part + (((size_t)seq * a.n_heads + (size_t)kvh * G) * max_chunks + chunk) * (2 + LK_HD);
    for (int t = tid; t < G * LK_HD; t += LK_AW * 64) {
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
        float* ph = part + (size_t)g * max_chunks * (2 + LK_HD);
        if (d == 0) {
            ph[0] = M;
            ph[1] = L;
        }
        ph[2 + d] = A;
    }
}

// The f16-cache partial on the matrix cores.  Same block/tile split as
// attn_partial_kernel (a 256-position chunk per block, a 64-position tile per
// wave), with both products on v_mfma_f32_16x16x16f16:
//   scores : S[pos][head] = K . q, 16 positions x 16 heads (G used) per MFMA,
//            K rows exact in f16, q split into f16 hi + lo (22 significant
//            bits), f32 accumulation.  MFMA row m of sub-tile t is position
//            16t + 4(m & 3) + (m >> 2) (a fixed permutation, shared by P.V);
//            lane l holds that row of K for m = l & 15, dims 16*(l >> 4) ..
//            +15 -- the same dims for q -- so a wave's K load is 16 whole
//            128-byte rows;
//   softmax: per head (lane & 15) over the wave's 64 positions;
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
    const uint32_t c0 = chunk * LK_ACHUNK;
    if (c0 >= ctx) return;  // uniform over the block
    const uint32_t max_chunks = (a.max_seq + LK_ACHUNK - 1) / LK_ACHUNK;
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
    const uint32_t p0 = c0 + (uint32_t)w * 64;
    const bool tile_live = p0 < ctx;  // wave-uniform
    const uint32_t plast = ctx - 1;

    // K: sub-tile t rows p0 + 16t + c16, this lane's 32 bytes (dims 16j..16j+15);
    // V: rows p0 + 8it + (lane >> 3), bytes 16*(lane & 7) -- 1 KiB per instruction
    uint4 kr[4][2];
    lk_u4 vr[8];  // a vector type (not the uint4 struct): held in registers, not in scratch
    if (tile_live) {
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
    }
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
    float mt = -INFINITY, lt = 0.f;
    lk_f4 o[4];
#pragma unroll
    for (int d = 0; d < 4; d++) o[d] = lk_f4{0.f, 0.f, 0.f, 0.f};
    if (tile_live) {
        uint16_t* vw = vs[w];
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
        // ---- softmax over the wave's 64 positions, per head (lanes c16, +16, +32, +48)
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
        float sum = 0.f;
        lk_h4 ph[4], pl[4];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pe = expf(sc[t][i] - mx);  // 0 for masked positions
                sum += pe;
                const _Float16 hi = (_Float16)pe;
                ph[t][i] = hi;
                pl[t][i] = (_Float16)(pe - (float)hi);
            }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        mt = mx;
        lt = sum;
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

    // ---- merge the 4 tiles into one partial per query head
    float* part = a.part + (((size_t)seq * a.n_heads + (size_t)kvh * G) * max_chunks + chunk) * (2 + LK_HD);
    for (int t = tid; t < G * LK_HD; t += LK_AW * 64) {
        const int g = t / LK_HD, dd = t % LK_HD;
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < LK_AW; ww++) M = fmaxf(M, red_m[ww][g]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int ww = 0; ww < LK_AW; ww++) {
            if (red_m[ww][g] != -INFINITY) {
                const float scl = expf(red_m[ww][g] - M);
                L = fmaf(scl, red_l[ww][g], L);
                A = fmaf(scl, red_acc[ww][g][dd], A);
            }
        }
        float* ph = part + (size_t)g * max_chunks * (2 + LK_HD);
        if (dd == 0) {
            ph[0] = M;
            ph[1] = L;
        }
        ph[2 + dd] = A;
    }
}

// Fold the chunk partials of one query head: out = sum_c e^{m_c-M} acc_c /
// sum_c e^{m_c-M} l_c.  Four waves take interleaved quarters of the chunks
// (lane = dim; 32 chunks' words in flight per lane, so contexts up to 32768
// positions take one memory round trip), each folding online against its own
// running max, and combine their (m, l, acc) in LDS.
__global__ __launch_bounds__(256) void attn_merge_kernel(const LkAttnArgs a) {
    const uint32_t h = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ctx = attn_ctx(a, seq);
    const uint32_t max_chunks = (a.max_seq + LK_ACHUNK - 1) / LK_ACHUNK;
    const uint32_t nch = (ctx + LK_ACHUNK - 1) / LK_ACHUNK;
    const float* part = a.part + ((size_t)seq * a.n_heads + h) * max_chunks * (2 + LK_HD);
    __shared__ float wm[4], wl[4], wa[4][LK_HD];
    float M = -INFINITY, L = 0.f, A = 0.f;
    for (uint32_t c0 = w * LK_MB; c0 < nch; c0 += 4 * LK_MB) {  // this wave's next LK_MB chunks
        // (m, l) by vector loads: lane k < 32 holds chunk c0+k's m, lane
        // 32+k its l (uniform-address scalar loads would queue behind the
        // scalar unit's few outstanding requests)
        const uint32_t kk = lane & 31;
        const bool live = c0 + kk < nch;
        const float ml = live ? part[(size_t)(c0 + kk) * (2 + LK_HD) + (lane >> 5)] : (lane < 32 ? -INFINITY : 0.f);
        float av[LK_MB];
#pragma unroll
        for (int k = 0; k < LK_MB; k++) {
            const uint32_t c = c0 + k < nch ? c0 + k : c0;  // in-range reload, dropped below
            av[k] = part[(size_t)c * (2 + LK_HD) + 2 + lane];
        }
        float mx = lane < 32 ? ml : -INFINITY;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        const float Mn = fmaxf(M, __shfl(mx, 0, 64));
        const float rs = expf(M - Mn);  // 0 while M is still -inf
        // lane k < 32: chunk k's weight e^{m_k - Mn} (0 for dead chunks)
        const float sck = lane < 32 && live ? expf(ml - Mn) : 0.f;
        const float lk = __shfl(ml, (int)kk + 32, 64);  // chunk kk's l
        float ls = lane < 32 ? sck * lk : 0.f;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) ls += __shfl_xor(ls, o, 64);
        L = fmaf(L, rs, __shfl(ls, 0, 64));
        A *= rs;
#pragma unroll
        for (int k = 0; k < LK_MB; k++) {
            const float sk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sck), k));
            A = fmaf(sk, av[k], A);
        }
        M = Mn;
    }
    if (lane == 0) {
        wm[w] = M;
        wl[w] = L;
    }
    wa[w][lane] = A;
    __syncthreads();
    if (w != 0) return;
    float Mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; i++) Mt = fmaxf(Mt, wm[i]);
    float Lt = 0.f, At = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (wm[i] != -INFINITY) {  // a wave with no chunks holds nothing
            const float sc = expf(wm[i] - Mt);
            Lt = fmaf(sc, wl[i], Lt);
            At = fmaf(sc, wa[i][lane], At);
        }
    }
    a.out[((size_t)seq * a.n_heads + h) * LK_HD + lane] = At / Lt;
}

hipError_t lk_attn_launch(const LkAttnArgs& a, hipStream_t st) {
    if (a.n_kv == 0 || a.n_heads % a.n_kv) return hipErrorInvalidValue;
    const uint32_t G = a.n_heads / a.n_kv;
    const uint32_t max_chunks = (a.max_seq + LK_ACHUNK - 1) / LK_ACHUNK;
    dim3 grid(max_chunks, a.n_kv, a.n_seq);
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
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(a.n_heads, a.n_seq), dim3(256), 0, st, a);
    return hipGetLastError();
}
