// batch_step.hip -- one decode step of up to 64 Batcher rows (src/engine.rs:
// 42-47: one token of each of B sequences, each at its own position and KV
// slot) as ONE persistent launch.
//
// Why: a Batcher step of B rows is Model::forward (src/model.rs:196-262) for B
// tokens: per layer five linear layers that read each weight once for all B
// rows, plus each row's attention.  As one launch per linear layer or row
// kernel (the per-layer path, ~220 launches a step) every step pays the
// launches' ramps and drains, not bytes or flops.  Here the grid (one
// workgroup of 8 waves per CU, all resident) walks the phases of every layer
// and meets at a grid barrier between phases:
//   QKV      X = RMSNorm(x) (applied as X is staged), Y = X W^T on the matrix
//            cores; the last split of each output tile adds bias, rotates q/k
//            pairs (RoPE at each row's position) and writes q to `qkv`, k and
//            v (rounded to f16) to the row's cache slot;
//   attn     (row, kv head, chunk) items of the f16-cache flash-decoding
//            partial on the matrix cores (attention_impl.h), the last chunk
//            of each (row, kv head) folding them into `att`;
//   o_proj   x += att W^T; the tile's squares summed for the next RMSNorm;
//   gate/up  X = RMSNorm(x), inner = silu(X Wg^T) * (X Wu^T);
//   down     x += inner Wd^T (+ the squares).
// Five barriers per layer.  The final norm, lm_head and argmax run after the
// launch on the multi-row kernels (one GEMM over all rows).
//
// Linear layers: an item is 128 output columns (8 waves x 16) x 32 rows x a
// run of 128-column K chunks, with v_mfma_f32_16x16x4f32 tiles, weights
// dequantized exactly as they are loaded and X staged through LDS (the tile
// code of gemm.hip).  Layers too small to give every CU an item split K; each
// split stores its partial tile, and the split that arrives last (an arrival
// counter per tile) sums them in split order and runs the epilogue.
//
// Memory: every activation written in a phase and read in a later one is
// stored write-through and loaded L2-bypassing at agent scope (sc1), and a
// block's stores are acknowledged (s_waitcnt vmcnt(0)) before it arrives at a
// barrier, so a phase sees the previous phase's data without cache flushes;
// the barrier is a monotonic arrival count polled at agent scope.  The
// current position's K/V row is written in the QKV phase and first read in
// the attention phase, a line no reader has cached before: rows past a
// sequence's position are never read.  Every wait is bounded: after a
// timeout the error flag is raised, later barriers stop waiting, and the
// host reports the failure and falls back to the per-layer launches.
#include "batch_step.h"

#include "attention_impl.h"
#include "gemm_impl.h"

#define BW 8
#define BTH (BW * 64)
#define BR 32      // batch rows an item holds at most (MB = 2 16-row MFMA column blocks)
#define NTILE 128  // output columns of an item (8 waves x 16)

namespace lkb {

using namespace lk;
using lkg::KC;
using lkg::Raw;
using lkg::XS;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

// Buffer resources over a uniform base: 16-byte loads and stores with the
// agent-scope coherence bit (sc1 = cache policy 16).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float4 ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16);
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ void st4(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 f) {
    const u4 v = {__float_as_uint(f.x), __float_as_uint(f.y), __float_as_uint(f.z), __float_as_uint(f.w)};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, 16);
}
__device__ __forceinline__ float ld1(const float* p) {
    return __uint_as_float(__hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st1(float* p, float v) {
    __hip_atomic_store((uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Grid barrier without read-modify-write: block b stores the barrier's tag
// (launch epoch * 256 + barrier index) into its own word bar[b], and every
// block polls all the words (wave 0, every lane a few) until each carries
// this tag or a later one.  Stores to distinct words proceed in parallel,
// where increments of one counter would serialise at the memory side (~40 ns
// each: 256 arrivals made a 10 us barrier).  Bounded: after ~2^22 polls the
// error flag is raised and from then on no barrier waits.
__device__ __forceinline__ void grid_sync(const LkBatchStepArgs& a, uint64_t tag, uint32_t mark) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are acknowledged
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(a.bar + blockIdx.x, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x < 64 && !__hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        const uint32_t nb = gridDim.x;
        for (uint32_t n = 0;; n++) {
            bool done = true;
            for (uint32_t i = threadIdx.x; i < nb; i += 64)
                done &= __hip_atomic_load(a.bar + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= tag;
            if (__all(done)) break;
            if ((n & 63) == 63) {
                if (__hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
                if (n > (1u << 20)) {
                    __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (a.trace && blockIdx.x == 0 && threadIdx.x == 0) a.trace[mark] = __builtin_amdgcn_s_memrealtime();
    }
    __syncthreads();
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// One linear layer of the step.
struct Lin {
    // segments, consecutive in the layer descriptor in global memory (QKV: q,
    // k, v and their biases; gate/up: gate, up; else one): read through these
    // pointers (scalar loads), never copied into a private array, which a
    // runtime segment index would put in scratch memory
    const LkDevW* w;
    const float* const* bias;
    uint32_t nseg, N, K;
    const float* x;       // X rows [B][ldx]
    uint32_t ldx;
    const float* gain;    // non-null: X = RMSNorm(x) with these gains (scales from a.ss)
    uint32_t ks, per;     // K splits, chunks per split
    uint32_t* cnt;        // this layer's arrival counters
};

// LDS of a linear-layer item: the double-buffered X tile, reused after the K
// loop as the output tile(s) [2][BR][NTILE + 4], plus the rows' norm scales.
struct LinLds {
    float xs[2][BR * XS];
    float scale[BR];
    uint32_t last;
};
static_assert(2 * BR * XS >= 2 * BR * (NTILE + 4), "output tiles fit the X staging area");
#define OT(t, r, c) xs_flat[((t) * BR + (r)) * (NTILE + 4) + (c)]

template <int WT, int KIND, int MB>
__device__ __forceinline__ void lin_item(const LkBatchStepArgs& a, const Lin& g, LinLds& S, uint32_t item, uint32_t L) {
    constexpr bool SW = KIND == LK_BS_GATEUP;
    const uint32_t B = a.nrows, N = g.N, K = g.K;
    constexpr uint32_t RB = 16 * MB;  // batch rows of this item
    const uint32_t NT = (N + NTILE - 1) / NTILE, BT = (B + RB - 1) / RB;
    const uint32_t z = item / (NT * BT), tile = item % (NT * BT);
    const uint32_t nt = tile / BT, bt = tile % BT;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nbase = nt * NTILE, n0 = nbase + 16 * wave;
    const bool live = n0 < N;  // wave-uniform
    const uint32_t b0 = bt * RB;
    const uint32_t nck = (K + KC - 1) / KC;
    const uint32_t c_begin = z * g.per, c_end = c_begin + g.per < nck ? c_begin + g.per : nck;
    const uint32_t j = (uint32_t)lane >> 4;
    float* xs_flat = &S.xs[0][0];

    // the rows' RMSNorm scales (src/math.rs:45-49) from the per-tile sums of squares
    if (g.gain && threadIdx.x < RB) {
        const uint32_t b = b0 + threadIdx.x < B ? b0 + threadIdx.x : B - 1;
        const uint32_t nts = (a.h + NTILE - 1) / NTILE;
        float s = 0.f;
        for (uint32_t t = 0; t < nts; t++) s += ld1(a.ss + (size_t)b * LK_BS_MAXT + t);
        S.scale[threadIdx.x] = 1.0f / sqrtf(s / (float)a.h + a.eps);
    }

    // segment of this wave's 16 rows (segments hold whole 16-row tiles)
    uint32_t si = 0, nb = 0;
    if constexpr (!SW) {
        while (si + 1 < g.nseg && n0 >= nb + g.w[si].rows) {
            nb += g.w[si].rows;
            si++;
        }
    }
    const LkDevW W0 = g.w[si];
    const LkDevW W1 = g.w[SW ? 1 : si];
    uint32_t r = live ? n0 - nb + ((uint32_t)lane & 15) : 0;
    r = r < W0.rows ? r : W0.rows - 1;

    const __amdgpu_buffer_rsrc_t xr = rsrc(g.x, B * g.ldx * 4);
    constexpr int XV = RB * KC / 4 / BTH;  // float4 per thread per chunk
    float4 xv[XV];
    auto x_fetch = [&](uint32_t c) {
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const uint32_t e = threadIdx.x + BTH * i;
            const uint32_t row = e / (KC / 4), col = (e % (KC / 4)) * 4;
            const uint32_t bb = b0 + row < B ? b0 + row : B - 1;
            const uint32_t k = c * KC + col;
            const float4 v = ld4(xr, (bb * g.ldx + (k < K ? k : 0)) * 4);  // unconditional, dropped past K
            xv[i] = k < K ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto x_store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const uint32_t e = threadIdx.x + BTH * i;
            const uint32_t row = e / (KC / 4), col = (e % (KC / 4)) * 4;
            *(float4*)&S.xs[buf][row * XS + col] = xv[i];
        }
    };
    // RMSNorm applied as the chunk is staged: (x * scale) * gain
    auto x_norm = [&](uint32_t c) {
        if (!g.gain) return;
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const uint32_t e = threadIdx.x + BTH * i;
            const uint32_t row = e / (KC / 4), col = (e % (KC / 4)) * 4;
            const uint32_t k = c * KC + col;
            // past K x is zero, so any in-range gain leaves it zero
            const float4 gv = *(const float4*)(g.gain + (k < K ? k : 0));
            const float s = S.scale[row];
            xv[i].x = __fmul_rn(__fmul_rn(xv[i].x, s), gv.x);
            xv[i].y = __fmul_rn(__fmul_rn(xv[i].y, s), gv.y);
            xv[i].z = __fmul_rn(__fmul_rn(xv[i].z, s), gv.z);
            xv[i].w = __fmul_rn(__fmul_rn(xv[i].w, s), gv.w);
        }
    };
    auto kb_of = [&](uint32_t c) -> uint32_t {
        const uint32_t kb = c * KC + 32 * j;
        return kb < K ? kb : K - 32;
    };

    f4 acc[MB], accu[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) {
        acc[m] = f4{0.f, 0.f, 0.f, 0.f};
        accu[m] = f4{0.f, 0.f, 0.f, 0.f};
    }
    // Loads are issued unconditionally (dead waves read in-range rows whose
    // values go unused) and the last chunk is peeled, so the wait before a
    // chunk's MFMAs leaves the next chunk's loads in flight; a load under a
    // branch would make the compiler wait for every load where paths meet.
    Raw<WT> cur, nxt, curu, nxtu;
    __syncthreads();  // the scales are in LDS; the previous item is done with xs
    if (c_begin < c_end) {
        x_fetch(c_begin);
        x_norm(c_begin);
        x_store(0);
        lkg::raw_load(cur, W0, r, kb_of(c_begin));
        if constexpr (SW) lkg::raw_load(curu, W1, r, kb_of(c_begin));
    }
    // one chunk's MFMAs on cur and X buffer buf
    auto chunk = [&](uint32_t c, int buf) {
        if (live) {
            const uint32_t kb = kb_of(c);
            const bool ok = c * KC + 32 * j < K;
            const float* xrow = &S.xs[buf][((uint32_t)lane & 15) * XS + 32 * j];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                float w[8], wu[8];
                lkg::dequant8<WT>(cur, s, kb, ok, w);
                if constexpr (SW) lkg::dequant8<WT>(curu, s, kb, ok, wu);
                float xb[MB][8];
#pragma unroll
                for (int m = 0; m < MB; m++) {
                    const float4 p = *(const float4*)(xrow + m * 16 * XS + 8 * s);
                    const float4 q = *(const float4*)(xrow + m * 16 * XS + 8 * s + 4);
                    xb[m][0] = p.x; xb[m][1] = p.y; xb[m][2] = p.z; xb[m][3] = p.w;
                    xb[m][4] = q.x; xb[m][5] = q.y; xb[m][6] = q.z; xb[m][7] = q.w;
                }
#pragma unroll
                for (int t = 0; t < 8; t++) {
#pragma unroll
                    for (int m = 0; m < MB; m++) {
                        acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[t], xb[m][t], acc[m], 0, 0, 0);
                        if constexpr (SW)
                            accu[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(wu[t], xb[m][t], accu[m], 0, 0, 0);
                    }
                }
            }
        }
    };
    uint32_t c = c_begin;
    for (; c + 1 < c_end; c++) {
        const int buf = (int)((c - c_begin) & 1);
        __syncthreads();  // X tile of chunk c is in xs[buf]
        x_fetch(c + 1);
        lkg::raw_load(nxt, W0, r, kb_of(c + 1));
        if constexpr (SW) lkg::raw_load(nxtu, W1, r, kb_of(c + 1));
        chunk(c, buf);
        x_norm(c + 1);
        x_store(buf ^ 1);  // last read in the previous chunk, before this chunk's barrier
        cur = nxt;
        if constexpr (SW) curu = nxtu;
    }
    if (c < c_end) {
        __syncthreads();  // X tile of chunk c is in xs[buf]
        chunk(c, (int)((c - c_begin) & 1));
    }
    __syncthreads();  // every wave is done with xs: it now holds the output tile(s)

    // D layout of a 16x16 tile: lane holds rows n0 + 4j + i (i = 0..3) of
    // batch column 16m + (lane & 15).  Output tile OT[t][b - b0][n - nbase].
    const uint32_t np = SW ? 2 * N : N;
    // the accumulators into the output tile(s) in LDS
    if (live) {
#pragma unroll
        for (int m = 0; m < MB; m++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t bl = 16u * m + ((uint32_t)lane & 15), nl = 16 * wave + 4 * j + i;
                OT(0, bl, nl) = acc[m][i];
                if constexpr (SW) OT(1, bl, nl) = accu[m][i];
            }
    }
    if (g.ks > 1) {
        // this split's partial tile (16-byte write-through stores), then the
        // arrival count; the split that arrives last sums them all in split
        // order, 8 splits' loads in flight at a time
        __syncthreads();
        const __amdgpu_buffer_rsrc_t pr = rsrc(a.part, g.ks * B * np * 4);
        constexpr uint32_t PC = RB * (NTILE / 4);  // float4 pieces of a tile
        constexpr int NO = SW ? 2 : 1;
        for (uint32_t e = threadIdx.x; e < PC; e += BTH) {
            const uint32_t bl = e / (NTILE / 4), cl = (e % (NTILE / 4)) * 4;
            const uint32_t b = b0 + bl, n = nbase + cl;
            if (b >= B || n >= N) continue;
#pragma unroll
            for (int t = 0; t < NO; t++)
                st4(pr, ((z * B + b) * np + t * N + n) * 4,
                    make_float4(OT(t, bl, cl), OT(t, bl, cl + 1), OT(t, bl, cl + 2), OT(t, bl, cl + 3)));
        }
        __builtin_amdgcn_s_waitcnt(0);  // the partial stores are acknowledged
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t* cn = g.cnt + (size_t)tile * LK_ATTN_CNT_STRIDE;
            const uint32_t arrived = __hip_atomic_fetch_add(cn, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            S.last = arrived == g.ks - 1;
            if (S.last) __hip_atomic_store(cn, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!S.last) return;
        for (uint32_t e = threadIdx.x; e < PC; e += BTH) {
            const uint32_t bl = e / (NTILE / 4), cl = (e % (NTILE / 4)) * 4;
            const uint32_t b = b0 + bl, n = nbase + cl;
            if (b >= B || n >= N) continue;
#pragma unroll
            for (int t = 0; t < NO; t++) {
                float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
                for (uint32_t z0 = 0; z0 < g.ks; z0 += 8) {
                    float4 v[8];
#pragma unroll
                    for (int q = 0; q < 8; q++)
                        v[q] = z0 + q < g.ks ? ld4(pr, (((z0 + q) * B + b) * np + t * N + n) * 4)
                                             : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        if (z0 + q < g.ks) {
                            sum.x += v[q].x;
                            sum.y += v[q].y;
                            sum.z += v[q].z;
                            sum.w += v[q].w;
                        }
                    }
                }
                OT(t, bl, cl) = sum.x;
                OT(t, bl, cl + 1) = sum.y;
                OT(t, bl, cl + 2) = sum.z;
                OT(t, bl, cl + 3) = sum.w;
            }
        }
    }
    __syncthreads();  // the output tile is complete

    if constexpr (KIND == LK_BS_QKV) {
        // bias, RoPE of q/k pairs (i, i + 32) at each row's position
        // (src/model.rs:268-279), k and v rounded to f16 into the row's slot
        const uint32_t qd = a.nh * 64, kvd = a.nkv * 64;
        const uint32_t* pos_rows = a.meta + a.meta_cap;
        const uint32_t* slots = a.meta + 2 * a.meta_cap;
        for (uint32_t e = threadIdx.x; e < RB * 2 * 32; e += BTH) {
            const uint32_t bl = e / 64, hb = (e / 32) & 1, u = e % 32;
            const uint32_t b = b0 + bl;
            const uint32_t nh0 = nbase + 64 * hb;  // the head block's first column
            if (b >= B || nh0 >= N) continue;
            const uint32_t seg = nh0 < qd ? 0 : (nh0 < qd + kvd ? 1 : 2);
            const uint32_t sb = seg == 0 ? 0 : (seg == 1 ? qd : qd + kvd);
            const float* bias = g.bias ? g.bias[seg] : nullptr;
            const uint32_t pos = pos_rows[b], slot = slots[b];
            if (seg < 2) {
                if (u >= 16) continue;
                const uint32_t i = 2 * u;  // dims i, i + 1 and their partners i + 32, i + 33
                const uint32_t cl = 64 * hb + i;
                float v0 = OT(0, bl, cl), v1 = OT(0, bl, cl + 1), w0 = OT(0, bl, cl + 32), w1 = OT(0, bl, cl + 33);
                if (bias) {
                    const uint32_t o = nh0 - sb + i;
                    v0 += bias[o];
                    v1 += bias[o + 1];
                    w0 += bias[o + 32];
                    w1 += bias[o + 33];
                }
                const float fpos = (float)pos;
                lk_rot_pair(v0, w0, __fmul_rn(fpos, a.freq.f[i]));
                lk_rot_pair(v1, w1, __fmul_rn(fpos, a.freq.f[i + 1]));
                if (seg == 0) {
                    float* q = a.qkv + (size_t)b * (qd + 2 * kvd) + nh0 + i;
                    st1(q, v0);
                    st1(q + 1, v1);
                    st1(q + 32, w0);
                    st1(q + 33, w1);
                } else {
                    const uint32_t kvh = (nh0 - qd) / 64;
                    uint16_t* dst = (uint16_t*)(a.kc + (size_t)L * a.layer_bytes) + (size_t)slot * a.slot_elems +
                                    ((size_t)kvh * a.kv_seq + pos) * 64 + i;
                    const uint32_t lo = (uint32_t)__half_as_ushort(__float2half_rn(v0)) |
                                        ((uint32_t)__half_as_ushort(__float2half_rn(v1)) << 16);
                    const uint32_t hi = (uint32_t)__half_as_ushort(__float2half_rn(w0)) |
                                        ((uint32_t)__half_as_ushort(__float2half_rn(w1)) << 16);
                    __hip_atomic_store((uint32_t*)dst, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store((uint32_t*)(dst + 32), hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else {
                const uint32_t d = 2 * u;
                const uint32_t cl = 64 * hb + d;
                float v0 = OT(0, bl, cl), v1 = OT(0, bl, cl + 1);
                if (bias) {
                    v0 += bias[nh0 - sb + d];
                    v1 += bias[nh0 - sb + d + 1];
                }
                const uint32_t kvh = (nh0 - qd - kvd) / 64;
                uint16_t* dst = (uint16_t*)(a.vc + (size_t)L * a.layer_bytes) + (size_t)slot * a.slot_elems +
                                ((size_t)kvh * a.kv_seq + pos) * 64 + d;
                const uint32_t pk = (uint32_t)__half_as_ushort(__float2half_rn(v0)) |
                                    ((uint32_t)__half_as_ushort(__float2half_rn(v1)) << 16);
                __hip_atomic_store((uint32_t*)dst, pk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    } else if constexpr (KIND == LK_BS_GATEUP) {
        // SwiGLU (src/model.rs:241-252): inner = silu(gate) * up
        const __amdgpu_buffer_rsrc_t ir = rsrc(a.inner, B * a.I * 4);
        for (uint32_t e = threadIdx.x; e < RB * (NTILE / 4); e += BTH) {
            const uint32_t bl = e / (NTILE / 4), cl = (e % (NTILE / 4)) * 4;
            const uint32_t b = b0 + bl, n = nbase + cl;
            if (b >= B || n >= N) continue;
            float4 o;
            o.x = silu_mul(OT(0, bl, cl), OT(1, bl, cl));
            o.y = silu_mul(OT(0, bl, cl + 1), OT(1, bl, cl + 1));
            o.z = silu_mul(OT(0, bl, cl + 2), OT(1, bl, cl + 2));
            o.w = silu_mul(OT(0, bl, cl + 3), OT(1, bl, cl + 3));
            st4(ir, (b * a.I + n) * 4, o);
        }
    } else {
        // residual (src/model.rs:235-237, :253-255) and the tile's sums of
        // squares for the next RMSNorm: 16 threads per row, 8 columns each
        const __amdgpu_buffer_rsrc_t xr2 = rsrc(a.x, B * a.h * 4);
        const uint32_t bl = threadIdx.x / 16, cl = (threadIdx.x % 16) * 8;
        const uint32_t b = b0 + bl, n = nbase + cl;
        float sq = 0.f;
        if (bl < RB && b < B && n < N) {
            const uint32_t off = (b * a.h + n) * 4;
            float4 x0 = ld4(xr2, off), x1 = ld4(xr2, off + 16);
            x0.x += OT(0, bl, cl);
            x0.y += OT(0, bl, cl + 1);
            x0.z += OT(0, bl, cl + 2);
            x0.w += OT(0, bl, cl + 3);
            x1.x += OT(0, bl, cl + 4);
            x1.y += OT(0, bl, cl + 5);
            x1.z += OT(0, bl, cl + 6);
            x1.w += OT(0, bl, cl + 7);
            st4(xr2, off, x0);
            st4(xr2, off + 16, x1);
            sq = x0.x * x0.x + x0.y * x0.y + x0.z * x0.z + x0.w * x0.w + x1.x * x1.x + x1.y * x1.y + x1.z * x1.z +
                 x1.w * x1.w;
        }
        // the 16 threads of a row are 16 adjacent lanes
        sq += __shfl_xor(sq, 1, 64);
        sq += __shfl_xor(sq, 2, 64);
        sq += __shfl_xor(sq, 4, 64);
        sq += __shfl_xor(sq, 8, 64);
        if (bl < RB && b < B && (threadIdx.x % 16) == 0) st1(a.ss + (size_t)b * LK_BS_MAXT + nt, sq);
    }
}

template <int WT, int KIND, int MB>
__device__ __forceinline__ void lin_phase(const LkBatchStepArgs& a, const Lin& g, LinLds& S, uint32_t L) {
    const uint32_t NT = (g.N + NTILE - 1) / NTILE, BT = (a.nrows + 16 * MB - 1) / (16 * MB);
    const uint32_t items = NT * BT * g.ks;
    for (uint32_t it = blockIdx.x; it < items; it += gridDim.x) lin_item<WT, KIND, MB>(a, g, S, it, L);
}

template <int WT, int G, int MB>
__global__ __launch_bounds__(BTH, 1) void batch_step_kernel(const LkBatchStepArgs a) {
    extern __shared__ __align__(16) float dyn[];  // 16-byte aligned after the static LDS
    LinLds& S = *(LinLds*)dyn;
    const uint32_t B = a.nrows, h = a.h, I = a.I;
    const uint32_t qd = a.nh * 64, kvd = a.nkv * 64, qkvd = qd + 2 * kvd;

    if (a.trace && blockIdx.x == 0 && threadIdx.x == 0) a.trace[0] = __builtin_amdgcn_s_memrealtime();
    // this launch's barrier tags: the epoch advances once per launch (block
    // 0, after the last barrier, when every block has read it)
    const uint64_t tag0 = (uint64_t)(*a.epoch) * 256;
    // the embedding rows (src/model.rs:200-202) and their tile sums of squares
    for (uint32_t b = blockIdx.x; b < B; b += gridDim.x) {
        const uint32_t tok = a.meta[b];
        float* row = &S.xs[0][0];
        for (uint32_t jj = threadIdx.x; jj < h; jj += BTH) {
            const float v = lk_embed_elem(a.embed, tok, jj);
            row[jj] = v;
            st1(a.x + (size_t)b * h + jj, v);
        }
        __syncthreads();
        // wave w sums tiles w, w + 8, ...: two elements per lane, then the wave sum
        const uint32_t nts = (h + NTILE - 1) / NTILE, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        for (uint32_t t = w; t < nts; t += BW) {
            const uint32_t j0 = t * NTILE + lane, j1 = j0 + 64;
            float sq = j0 < h ? row[j0] * row[j0] : 0.f;
            if (j1 < h) sq = fmaf(row[j1], row[j1], sq);
            sq = lk_wave_sum(sq);
            if (lane == 0) st1(a.ss + (size_t)b * LK_BS_MAXT + t, sq);
        }
        __syncthreads();
    }
    grid_sync(a, tag0 + 1, 1);

    for (uint32_t L = 0; L < a.n_layers; L++) {
        const LkFusedLayer& ly = a.layers[L];
        {  // q, k, v
            Lin g{};
            g.w = &ly.q;  // q, k, v
            g.bias = &ly.bq;  // bq, bk, bv
            g.nseg = 3;
            g.N = qkvd;
            g.K = h;
            g.x = a.x;
            g.ldx = h;
            g.gain = ly.in_norm;
            g.ks = a.ks[LK_BS_QKV];
            g.per = a.per[LK_BS_QKV];
            g.cnt = a.cnt + (size_t)LK_BS_QKV * LK_BS_CNT_PER_GEMM * LK_ATTN_CNT_STRIDE;
            lin_phase<WT, LK_BS_QKV, MB>(a, g, S, L);
        }
        grid_sync(a, tag0 + 2 + 5 * L + 0, 2 + 5 * L + 0);
        {  // attention: (chunk, kv head, row) items
            LkAttnArgs at = a.attn;
            at.q = a.qkv;
            at.k = a.kc + (size_t)L * a.layer_bytes;
            at.v = a.vc + (size_t)L * a.layer_bytes;
            at.out = a.att;
            const uint32_t nch = at.tiles ? (a.kv_seq + 64 * at.waves * at.tiles - 1) / (64 * at.waves * at.tiles) : 1;
            const uint32_t items = nch * a.nkv * B;
            for (uint32_t it = blockIdx.x; it < items; it += gridDim.x)
                attn_mfma_item<G, 1, false, true>(at, it % nch, (it / nch) % a.nkv, it / (nch * a.nkv));
        }
        grid_sync(a, tag0 + 2 + 5 * L + 1, 2 + 5 * L + 1);
        {  // o_proj + residual
            Lin g{};
            g.w = &ly.o;
            g.nseg = 1;
            g.N = h;
            g.K = qd;
            g.x = a.att;
            g.ldx = qd;
            g.ks = a.ks[LK_BS_O];
            g.per = a.per[LK_BS_O];
            g.cnt = a.cnt + (size_t)LK_BS_O * LK_BS_CNT_PER_GEMM * LK_ATTN_CNT_STRIDE;
            lin_phase<WT, LK_BS_O, MB>(a, g, S, L);
        }
        grid_sync(a, tag0 + 2 + 5 * L + 2, 2 + 5 * L + 2);
        {  // RMSNorm + gate/up + SwiGLU
            Lin g{};
            g.w = &ly.gate;  // gate, up
            g.nseg = 2;
            g.N = I;
            g.K = h;
            g.x = a.x;
            g.ldx = h;
            g.gain = ly.post_norm;
            g.ks = a.ks[LK_BS_GATEUP];
            g.per = a.per[LK_BS_GATEUP];
            g.cnt = a.cnt + (size_t)LK_BS_GATEUP * LK_BS_CNT_PER_GEMM * LK_ATTN_CNT_STRIDE;
            lin_phase<WT, LK_BS_GATEUP, MB>(a, g, S, L);
        }
        grid_sync(a, tag0 + 2 + 5 * L + 3, 2 + 5 * L + 3);
        {  // down + residual
            Lin g{};
            g.w = &ly.down;
            g.nseg = 1;
            g.N = h;
            g.K = I;
            g.x = a.inner;
            g.ldx = I;
            g.ks = a.ks[LK_BS_DOWN];
            g.per = a.per[LK_BS_DOWN];
            g.cnt = a.cnt + (size_t)LK_BS_DOWN * LK_BS_CNT_PER_GEMM * LK_ATTN_CNT_STRIDE;
            lin_phase<WT, LK_BS_DOWN, MB>(a, g, S, L);
        }
        grid_sync(a, tag0 + 2 + 5 * L + 4, 2 + 5 * L + 4);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *a.epoch = *a.epoch + 1;
}

template <int WT, int G, int MB>
static hipError_t launch_t(const LkBatchStepArgs& a, unsigned blocks, hipStream_t st, bool setup) {
    auto kfn = batch_step_kernel<WT, G, MB>;
    const size_t lds = lk_batch_step_lds_bytes();
    if (setup) {
        hipError_t e = hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        int nb = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, (const void*)kfn, BTH, lds);
        if (e != hipSuccess) return e;
        return nb >= 1 ? hipSuccess : hipErrorInvalidConfiguration;
    }
    hipLaunchKernelGGL(kfn, dim3(blocks), dim3(BTH), lds, st, a);
    return hipGetLastError();
}

}  // namespace lkb

size_t lk_batch_step_lds_bytes() { return sizeof(lkb::LinLds); }

template <int WT>
static hipError_t launch_g(const LkBatchStepArgs& a, int G, bool one, unsigned blocks, hipStream_t st, bool setup) {
    switch (G) {
    case 3: return one ? lkb::launch_t<WT, 3, 1>(a, blocks, st, setup) : lkb::launch_t<WT, 3, 2>(a, blocks, st, setup);
    case 4: return one ? lkb::launch_t<WT, 4, 1>(a, blocks, st, setup) : lkb::launch_t<WT, 4, 2>(a, blocks, st, setup);
    case 7: return one ? lkb::launch_t<WT, 7, 1>(a, blocks, st, setup) : lkb::launch_t<WT, 7, 2>(a, blocks, st, setup);
    case 8: return one ? lkb::launch_t<WT, 8, 1>(a, blocks, st, setup) : lkb::launch_t<WT, 8, 2>(a, blocks, st, setup);
    default: return hipErrorInvalidValue;
    }
}

static hipError_t launch_w(const LkBatchStepArgs& a, uint32_t wt, int G, bool one, unsigned blocks, hipStream_t st,
                           bool setup) {
    switch (wt) {
    case LK_Q8_0: return launch_g<LK_Q8_0>(a, G, one, blocks, st, setup);
    case LK_F16: return launch_g<LK_F16>(a, G, one, blocks, st, setup);
    case LK_Q4_K: return launch_g<LK_Q4_K>(a, G, one, blocks, st, setup);
    default: return hipErrorInvalidValue;
    }
}

hipError_t lk_batch_step_launch(const LkBatchStepArgs& a, uint32_t wt, int G, unsigned blocks, hipStream_t st,
                                bool setup) {
    if (setup) {  // both instances: up to 16 rows (one 16-row MFMA column block per item) and more (two)
        const hipError_t e = launch_w(a, wt, G, true, blocks, st, true);
        return e != hipSuccess ? e : launch_w(a, wt, G, false, blocks, st, true);
    }
    return launch_w(a, wt, G, lk_batch_step_mb(a.nrows) == 1, blocks, st, false);
}
