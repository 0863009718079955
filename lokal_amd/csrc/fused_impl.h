// fused_impl.h -- device helpers shared by the one-kernel decode steps
// (fused.hip: one sequence; fused_rows.hip: a few Batcher rows at once):
// the (f32 | epoch) exchange words, bounded waits, block reductions, RMSNorm
// in LDS, RoPE and KV-cache element helpers.
#pragma once
#include "lkhip_common.h"
#include "matvec_impl.h"
#include "fused.h"

#define FW ((int)LK_FUSED_WAVES)
#define FT (FW * 64)

namespace lkf {


using namespace lk;

struct Ctx {
    const LkFusedArgs* a;
    uint32_t* err;
    int lane, wave, gw, nw;
};

// Block barrier for data exchanged through LDS only.  __syncthreads() is
// also a workgroup-scope release/acquire fence, and on this target that
// waits for every global store still in flight (vmcnt(0)): after a stage
// publishes its (value | epoch) words that is a full memory round trip per
// barrier, paid by every wave.  The exchange words need no such ordering
// (the epoch in each word is the completion flag), so the barrier waits for
// this wave's LDS operations only; the empty asm statements keep the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt not waited
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint64_t word(float v, uint32_t ep) {
    return ((uint64_t)ep << 32) | (uint64_t)__float_as_uint(v);
}
__device__ __forceinline__ void publish(uint64_t* p, float v, uint32_t ep) {
    __hip_atomic_store(p, word(v, ep), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Spin until word p carries epoch ep; returns its value.  Bounded: after
// ~2^21 polls (tens of ms) the error flag is raised and every later wait
// returns at once, so the grid always drains.
__device__ __forceinline__ float await(const Ctx& c, const uint64_t* p, uint32_t ep) {
    uint64_t w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((uint32_t)(w >> 32) == ep) return __uint_as_float((uint32_t)w);
    for (uint32_t n = 0;; n++) {
        __builtin_amdgcn_s_sleep(1);
        w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((uint32_t)(w >> 32) == ep) break;
        if ((n & 255) == 255) {
            if (__hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
            if (n > (1u << 21)) {
                __hip_atomic_store(c.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    return __uint_as_float((uint32_t)w);
}

__device__ __forceinline__ uint64_t ld_word(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Words src[i0 + k*step], k < N, i < n, into dst[...]: all N loads are in
// flight together, and every round re-polls all the words still missing
// together, so a late vector costs one round trip per round rather than one
// per missing word.  Bounded like await().
template <int N>
__device__ __forceinline__ void awaitN(const Ctx& c, const uint64_t* src, uint32_t i0, uint32_t step, uint32_t n,
                                       uint32_t ep, float* dst) {
    uint64_t w[N];
#pragma unroll
    for (int k = 0; k < N; k++) {
        const uint32_t i = i0 + k * step;
        w[k] = i < n ? ld_word(src + i) : ((uint64_t)ep << 32);
    }
    for (uint32_t r = 0;; r++) {
        bool done = true;
#pragma unroll
        for (int k = 0; k < N; k++) done &= (uint32_t)(w[k] >> 32) == ep;
        if (done) break;
        if ((r & 255) == 255) {
            if (__hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
            if (r > (1u << 21)) {
                __hip_atomic_store(c.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < N; k++)
            if ((uint32_t)(w[k] >> 32) != ep) w[k] = ld_word(src + i0 + k * step);
    }
#pragma unroll
    for (int k = 0; k < N; k++) {
        const uint32_t i = i0 + k * step;
        if (i < n) dst[i] = __uint_as_float((uint32_t)w[k]);
    }
}

// Block-cooperative: wait for n published words into LDS.  half < 0: every
// wave polls; otherwise only the waves of one half (half 0: waves 0..FW/2-1,
// half 1: the rest) do: a wave's loads retire in issue order, so the polling
// half is the one with no weight rows of its own still streaming in.
// N: words in flight per thread (sized so one batch covers the vector).
template <int N>
__device__ __forceinline__ void stage_in(const Ctx& c, const uint64_t* src, uint32_t n, uint32_t ep, float* dst,
                                         int half) {
    lds_barrier();  // every wave is done reading dst from the previous stage
    if (half < 0) {
        for (uint32_t i = threadIdx.x; i < n; i += N * FT) awaitN<N>(c, src, i, FT, n, ep, dst);
    } else {
        const uint32_t t = threadIdx.x - (uint32_t)half * (FT / 2);
        if ((int)(threadIdx.x >= FT / 2) == half)
            for (uint32_t i = t; i < n; i += N * (FT / 2)) awaitN<N>(c, src, i, FT / 2, n, ep, dst);
    }
    lds_barrier();
}

// Totals of NB block-wide sums whose per-wave partials sit at red[b*FW + w]:
// lane 8b + w reads partial (b, w) -- one LDS read for all of them, instead
// of NB * FW dependent reads -- and the 8 lanes of each row add up by DPP
// (quad pairs, quad halves, row_ror 4: lane 8b + 4 then holds row b's total).
static_assert(FW == 8, "the partials of one sum fill 8 adjacent lanes");
template <int NB>
__device__ __forceinline__ void block_partials_sum(const float* red, float (&tot)[NB]) {
    static_assert(NB * FW <= 64, "one lane per partial");
    const int lane = threadIdx.x & 63;
    float v = lane < NB * FW ? red[lane] : 0.f;
    v += lk_dpp<0xB1, 0xF>(v, 0.f);
    v += lk_dpp<0x4E, 0xF>(v, 0.f);
    v += lk_dpp<0x124, 0xF>(v, 0.f);
#pragma unroll
    for (int b = 0; b < NB; b++)
        tot[b] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 8 * b + 4));
}

__device__ __forceinline__ float block_sum(float v, float* red) {
    v = lk_wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    float t[1];
    block_partials_sum<1>(red, t);
    lds_barrier();
    return t[0];
}

// math::rmsnorm (src/math.rs:45-49) of the LDS vector xr into xo (gains g in LDS).
__device__ __forceinline__ void rmsnorm_lds(const float* xr, const float* g, uint32_t n, float eps,
                                            float* xo, float* red) {
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += FT) ss = fmaf(xr[i], xr[i], ss);
    const float tot = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += FT) xo[i] = __fmul_rn(__fmul_rn(xr[i], scale), g[i]);
    lds_barrier();
}

// math::rmsnorm (src/math.rs:45-49) of NB rows of n in LDS (row b at xr + b*n)
// into xo; red holds NB * FW partial sums.  A thread's elements of every row
// are read once into registers (one LDS round trip), squared and summed in
// index order, then scaled from the same registers.
template <int NB>
__device__ __forceinline__ void rmsnorm_rows(const float* xr, const float* g, uint32_t n, float eps, float* xo,
                                             float* red) {
    constexpr int EPT = ((int)LK_FUSED_MAX_H + FT - 1) / FT;
    float v[NB][EPT], ss[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        ss[b] = 0.f;
#pragma unroll
        for (int e = 0; e < EPT; e++) {
            const uint32_t i = threadIdx.x + (uint32_t)e * FT;
            v[b][e] = i < n ? xr[b * n + i] : 0.f;
            ss[b] = fmaf(v[b][e], v[b][e], ss[b]);
        }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) ss[b] = lk_wave_sum(ss[b]);
    if ((threadIdx.x & 63) == 0)
#pragma unroll
        for (int b = 0; b < NB; b++) red[b * FW + (threadIdx.x >> 6)] = ss[b];
    lds_barrier();
    float tot[NB], scale[NB];
    block_partials_sum<NB>(red, tot);
#pragma unroll
    for (int b = 0; b < NB; b++) scale[b] = 1.0f / sqrtf(tot[b] / (float)n + eps);
#pragma unroll
    for (int e = 0; e < EPT; e++) {
        const uint32_t i = threadIdx.x + (uint32_t)e * FT;
        if (i < n) {
            const float gv = g[i];
#pragma unroll
            for (int b = 0; b < NB; b++) xo[b * n + i] = __fmul_rn(__fmul_rn(v[b][e], scale[b]), gv);
        }
    }
    lds_barrier();
}

__device__ __forceinline__ float kv_round(float v, bool f32) {
    return f32 ? v : __half2float(__float2half_rn(v));
}
__device__ __forceinline__ void kv_put(uint16_t* p, float v) { *p = __half_as_ushort(__float2half_rn(v)); }
__device__ __forceinline__ void kv_put(float* p, float v) { *p = v; }
__device__ __forceinline__ void kv8(const uint16_t* p, float* o) {
    const uint4 v = *(const uint4*)p;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int h = 0; h < 4; h++) {
        o[2 * h] = lk_h2f((uint16_t)(w[h] & 0xFFFF));
        o[2 * h + 1] = lk_h2f((uint16_t)(w[h] >> 16));
    }
}
__device__ __forceinline__ void kv8(const float* p, float* o) {
    const float4 a = ((const float4*)p)[0], b = ((const float4*)p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

// RoPE pair rotation (src/model.rs:268-279) by the angle with cosine c, sine s.
__device__ __forceinline__ void rot(float& x0, float& x1, float c, float s) {
    const float n0 = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
    const float n1 = __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
    x0 = n0;
    x1 = n1;
}

// Cache-chunk packing of values held as f32: 4 floats (f32 cache) or 8
// f16-representable floats (f16 cache: exact) into one 16-byte chunk.
__device__ __forceinline__ uint32_t h2bits(float a, float b) {
    return (uint32_t)__half_as_ushort(__float2half_rn(a)) | ((uint32_t)__half_as_ushort(__float2half_rn(b)) << 16);
}
__device__ __forceinline__ uint4 pack4(const float* v, bool f32) {
    if (f32) return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
    return make_uint4(h2bits(v[0], v[1]), h2bits(v[2], v[3]), h2bits(v[4], v[5]), h2bits(v[6], v[7]));
}
// Elements 8q..8q+7 of a raw cache row as f32.
template <typename U4, int N>
__device__ __forceinline__ void unpack8(const U4 (&raw)[N], int q, bool f32, float* o) {
    if (f32) {
        const U4 a0 = raw[2 * q], a1 = raw[(2 * q + 1) < N ? 2 * q + 1 : 0];
        o[0] = __uint_as_float(a0.x); o[1] = __uint_as_float(a0.y);
        o[2] = __uint_as_float(a0.z); o[3] = __uint_as_float(a0.w);
        o[4] = __uint_as_float(a1.x); o[5] = __uint_as_float(a1.y);
        o[6] = __uint_as_float(a1.z); o[7] = __uint_as_float(a1.w);
    } else {
        const U4 a = raw[q];
        const uint32_t w4[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            o[2 * e] = lk_h2f((uint16_t)(w4[e] & 0xFFFF));
            o[2 * e + 1] = lk_h2f((uint16_t)(w4[e] >> 16));
        }
    }
}

// N wave sums at once: each DPP step is applied to all N values before the
// next, so the N dependent chains overlap (lk_wave_sum's order of additions:
// each result is bit-identical to it).
template <int N>
__device__ __forceinline__ void wave_sums(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += lk_dpp<0xB1, 0xF>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += lk_dpp<0x4E, 0xF>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += lk_dpp<0x124, 0xF>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += lk_dpp<0x128, 0xF>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += lk_dpp<0x142, 0xA>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += lk_dpp<0x143, 0xC>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; i++)
        v[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[i]), 63));
}

// This lane's slice of an LDS vector for rows of NCH 16-byte chunks (lane l
// takes chunks l + 64 i), read once and reused by every row: chunk
// elements are contiguous (Q8_0, F16, Q8_SM); Q4_K's 16 low-nibble then 16
// high-nibble elements of its chunk (sub-block pair k >> 1, half k & 1 of
// super-block ch >> 3).
template <int WT, int NCH>
__device__ __forceinline__ void x_slice(const float* x, uint32_t cols, int lane,
                                        float (&xr)[NCH][ChunkTraits<WT>::elems]) {
    constexpr uint32_t CE = ChunkTraits<WT>::elems;
    const uint32_t nchunk = cols / CE;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const uint32_t ch0 = (uint32_t)lane + 64u * i;
        const uint32_t ch = ch0 < nchunk ? ch0 : 0u;
        if constexpr (WT == LK_Q4_K) {
            const uint32_t sb = ch >> 3, k = ch & 7;
            const float* xl = x + sb * 256 + (k >> 1) * 64 + (k & 1) * 16;
#pragma unroll
            for (uint32_t e = 0; e < 16; e += 4) {
                const float4 lo = *(const float4*)(xl + e), hi = *(const float4*)(xl + 32 + e);
                xr[i][e] = lo.x; xr[i][e + 1] = lo.y; xr[i][e + 2] = lo.z; xr[i][e + 3] = lo.w;
                xr[i][16 + e] = hi.x; xr[i][16 + e + 1] = hi.y; xr[i][16 + e + 2] = hi.z; xr[i][16 + e + 3] = hi.w;
            }
        } else {
            const float* xc = x + (size_t)ch * CE;
#pragma unroll
            for (uint32_t e = 0; e < CE; e += 4) {
                const float4 v = *(const float4*)(xc + e);
                xr[i][e] = v.x; xr[i][e + 1] = v.y; xr[i][e + 2] = v.z; xr[i][e + 3] = v.w;
            }
        }
    }
}

// math::rmsnorm (src/math.rs:45-49) of an LDS vector, by each wave for its
// own lanes' slice: the sum of squares over the wave (no block barrier),
// then (x * scale) * g per element, both products rounded as the CPU path
// rounds them.
template <int WT, int NCH>
__device__ __forceinline__ void norm_slice(const float* x, const float* g, uint32_t n, float eps, int lane,
                                           float (&xr)[NCH][ChunkTraits<WT>::elems]) {
    constexpr uint32_t CE = ChunkTraits<WT>::elems;
    const uint32_t nchunk = n / CE;
    x_slice<WT, NCH>(x, n, lane, xr);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const bool ok = (uint32_t)lane + 64u * i < nchunk;
#pragma unroll
        for (uint32_t e = 0; e < CE; e++) ss = ok ? fmaf(xr[i][e], xr[i][e], ss) : ss;
    }
    ss = lk_wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    float gr[NCH][CE];
    x_slice<WT, NCH>(g, n, lane, gr);
#pragma unroll
    for (int i = 0; i < NCH; i++)
#pragma unroll
        for (uint32_t e = 0; e < CE; e++) xr[i][e] = __fmul_rn(__fmul_rn(xr[i][e], scale), gr[i][e]);
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}


}  // namespace lkf
