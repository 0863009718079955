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
//   P.V    : lane = (position j%8 group, 8 dims), one 16-byte V load per lane
//            covers 8 positions x 64 dims per instruction; the 8 lanes that share
//            a dim slice are combined by xor-shuffles.
// The 4 tiles merge in LDS into one (m, l, acc[64]) partial per query head;
// attn_merge_kernel folds the partials of all chunks with the usual
// max-rescaled sums.  fp32 throughout; scale 1/sqrt(64) = 0.125 is exact.
#include "lkhip_common.h"

#define LK_HD 64
#define LK_ACHUNK 256

uint32_t lk_attn_chunk(uint32_t) { return LK_ACHUNK; }

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
__global__ __launch_bounds__(256) void attn_partial_kernel(const LkAttnArgs a) {
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
    __shared__ float ps[4][G][64];
    __shared__ float red_m[4][G], red_l[4][G];
    __shared__ float red_acc[4][G][LK_HD];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* qsrc = a.q + (size_t)seq * a.q_stride + (size_t)kvh * G * LK_HD;
    for (int i = tid; i < G * LK_HD; i += 256) qs[i / LK_HD][i % LK_HD] = qsrc[i];
    __syncthreads();

    const uint32_t p0 = c0 + (uint32_t)w * 64;
    const bool tile_live = p0 < ctx;
    float m[G], l[G];
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.f;
    }

    if (tile_live) {
        // ---- scores: lane = position
        const uint32_t p = p0 + (uint32_t)lane;
        const bool valid = p < ctx;
        float s[G];
#pragma unroll
        for (int g = 0; g < G; g++) s[g] = 0.f;
        if (valid) {
            const KV* krow = K + (size_t)p * LK_HD;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float k8[8];
                load8(krow + 8 * i, k8);
#pragma unroll
                for (int e = 0; e < 8; e++) {
#pragma unroll
                    for (int g = 0; g < G; g++) s[g] = fmaf(k8[e], qs[g][8 * i + e], s[g]);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float sg = valid ? s[g] * 0.125f : -INFINITY;
            m[g] = lk_wave_max(sg);
            const float pg = valid ? expf(sg - m[g]) : 0.f;
            l[g] = lk_wave_sum(pg);
            ps[w][g][lane] = pg;
        }
    }
    __syncthreads();  // P of every tile is in LDS

    if (tile_live) {
        // ---- P.V: lane = (position group, 8-dim slice)
        const uint32_t sub = (uint32_t)lane >> 3, dq = ((uint32_t)lane & 7) * 8;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t pj = p0 + (uint32_t)j * 8 + sub;
            if (pj < ctx) {
                float vf[8];
                load8(V + (size_t)pj * LK_HD + dq, vf);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float pw = ps[w][g][j * 8 + sub];
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[g][e] = fmaf(pw, vf[e], acc[g][e]);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float v = acc[g][e];
                v += __shfl_xor(v, 8, 64);
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
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
    if (lane < 8) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) red_acc[w][g][lane * 8 + e] = acc[g][e];
    }
    __syncthreads();

    // ---- merge the 4 tiles into one partial per query head
    float* part = a.part + (((size_t)seq * a.n_heads + (size_t)kvh * G) * max_chunks + chunk) * (2 + LK_HD);
    for (int t = tid; t < G * LK_HD; t += 256) {
        const int g = t / LK_HD, d = t % LK_HD;
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) M = fmaxf(M, red_m[ww][g]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
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

// Fold the chunk partials of one query head: out = sum_c e^{m_c-M} acc_c / sum_c e^{m_c-M} l_c.
__global__ __launch_bounds__(64) void attn_merge_kernel(const LkAttnArgs a) {
    const uint32_t h = blockIdx.x, seq = blockIdx.y, d = threadIdx.x;
    const uint32_t ctx = attn_ctx(a, seq);
    const uint32_t max_chunks = (a.max_seq + LK_ACHUNK - 1) / LK_ACHUNK;
    const uint32_t nch = (ctx + LK_ACHUNK - 1) / LK_ACHUNK;
    const float* part = a.part + ((size_t)seq * a.n_heads + h) * max_chunks * (2 + LK_HD);
    float M = -INFINITY;
    for (uint32_t c = 0; c < nch; c++) M = fmaxf(M, part[(size_t)c * (2 + LK_HD)]);
    float L = 0.f, A = 0.f;
    for (uint32_t c = 0; c < nch; c++) {
        const float* pc = part + (size_t)c * (2 + LK_HD);
        const float sc = expf(pc[0] - M);
        L = fmaf(sc, pc[1], L);
        A = fmaf(sc, pc[2 + d], A);
    }
    a.out[((size_t)seq * a.n_heads + h) * LK_HD + d] = A / L;
}

hipError_t lk_attn_launch(const LkAttnArgs& a, hipStream_t st) {
    if (a.n_kv == 0 || a.n_heads % a.n_kv) return hipErrorInvalidValue;
    const uint32_t G = a.n_heads / a.n_kv;
    const uint32_t max_chunks = (a.max_seq + LK_ACHUNK - 1) / LK_ACHUNK;
    dim3 grid(max_chunks, a.n_kv, a.n_seq);
#define LK_ATTN_CASE(g)                                                                         \
    case g:                                                                                     \
        if (a.kv_f32) hipLaunchKernelGGL((attn_partial_kernel<g, float>), grid, dim3(256), 0, st, a); \
        else hipLaunchKernelGGL((attn_partial_kernel<g, uint16_t>), grid, dim3(256), 0, st, a);  \
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
    hipLaunchKernelGGL(attn_merge_kernel, dim3(a.n_heads, a.n_seq), dim3(64), 0, st, a);
    return hipGetLastError();
}
