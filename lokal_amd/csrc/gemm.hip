// gemm.hip -- the multi-row dequant-fused linear layer on the matrix cores:
// Y[b][n] = sum_k X[b][k] * W[n][k] (+ bias[n]) for b < B rows of f32
// activations, W in its device type (F16, Q8_0, Q4_K, Q8_SM) dequantized as it is
// loaded.  This is Linear::forward (src/model.rs:27-35) applied to a batch of
// tokens: the Batcher's decode step (one row per sequence, src/engine.rs:42-47)
// and chunked prefill (rows = prompt positions of one sequence), the work
// lokal's Metal backend gives matmul_pg (src/gpu/kernels.metal:1749-1985).
//
// Arithmetic: v_mfma_f32_16x16x4f32 -- fp32 operands, fp32 accumulation.
// Dequantized weights are exact f32 values (int8 * f16 scale, 4-bit Q4_K with
// the reference's two roundings, f16), so the only difference from the CPU
// path's dot (src/math.rs:10-38) is the summation order.
//
// Work split:
//   wave   = 16 weight rows x 16*MB batch rows, over a range of K chunks
//            (segments of a multi-segment launch hold whole 16-row tiles);
//   block  = 4 waves on 64 consecutive weight rows sharing one X tile;
//   chunk  = 128 columns of K: lane l takes weight row (l & 15) and the 32
//            consecutive columns 32*(l >> 4) .. +31 of the chunk, so a row's
//            128 columns are one contiguous run fetched by 4 lanes, and a
//            Q8_0 lane holds exactly one 32-weight block (one scale);
//   MFMA t (t = 0..31) multiplies every lane's t-th weight with the X value of
//            the same column: the lane-group/column map is a permutation of
//            k shared by both operands, so the product is the plain dot.
// X chunks are staged in LDS (double-buffered, one barrier per chunk) and
// shared by the block's 4 waves; the next chunk's weights and X are loaded
// before the current chunk's MFMAs.  Small matrices split K over the grid
// (blockIdx.z); their partial tiles go to a workspace and gemm_reduce_kernel
// sums them in a fixed order and runs the epilogue.
#include "gemm_impl.h"

#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace lkg {

// Epilogue of one output element: segment n (global index over segments).
__device__ __forceinline__ void emit(const LkGemmArgs& a, int mode, uint32_t b, uint32_t n, float v, float u) {
    if (mode == LK_MV_SWIGLU) {
        a.seg[0].out[(size_t)b * a.ldy + n] = silu_mul(v, u);
        return;
    }
    uint32_t si = 0, nb = 0;
    while (si + 1 < a.nseg && n >= nb + a.seg[si].w.rows) {
        nb += a.seg[si].w.rows;
        si++;
    }
    const LkSeg& s = a.seg[si];
    const uint32_t nl = n - nb;
    if (s.bias) v += s.bias[nl];
    float* o = s.out + (size_t)b * a.ldy + nl;
    if (mode == LK_MV_ACC) *o += v;
    else *o = v;
}

template <int WT, int MB, int MODE>
__global__ __launch_bounds__(256) void gemm_kernel(const LkGemmArgs a) {
    constexpr bool SW = MODE == LK_MV_SWIGLU;
    constexpr int BR = 16 * MB;  // batch rows of the block tile
    __shared__ float xs[2][BR * XS];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t n0 = (blockIdx.x * 4 + wave) * 16;
    const bool live = n0 < a.N;  // wave-uniform; dead waves still stage X
    const uint32_t B = a.n_rows, K = a.K;
    const uint32_t b0 = blockIdx.y * BR;
    const uint32_t nck = (K + KC - 1) / KC;
    const uint32_t per = (nck + a.ks - 1) / a.ks;
    const uint32_t c_begin = blockIdx.z * per;
    const uint32_t c_end = c_begin + per < nck ? c_begin + per : nck;
    const uint32_t j = (uint32_t)lane >> 4;

    // weight row of this lane (segment lookup is wave-uniform: segments hold
    // whole 16-row tiles)
    uint32_t si = 0, nb = 0;
    if constexpr (!SW) {
        while (si + 1 < a.nseg && n0 >= nb + a.seg[si].w.rows) {
            nb += a.seg[si].w.rows;
            si++;
        }
    }
    const LkDevW W0 = a.seg[si].w;
    const LkDevW W1 = a.seg[SW ? 1 : si].w;
    // rows past the last (a ragged final tile) re-read the last row; their
    // outputs are not stored
    uint32_t r = live ? n0 - nb + ((uint32_t)lane & 15) : 0;
    r = r < W0.rows ? r : W0.rows - 1;

    // X staging: thread t loads float4 number t + 256*i of the BR x KC tile
    constexpr int XV = BR * KC / 4 / 256;  // float4 per thread per chunk
    float4 xv[XV];
    auto x_fetch = [&](uint32_t c) {
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const uint32_t e = threadIdx.x + 256u * i;  // float4 index in the tile
            const uint32_t row = e / (KC / 4), col = (e % (KC / 4)) * 4;
            uint32_t bb = b0 + row;
            bb = bb < B ? bb : B - 1;
            const uint32_t k = c * KC + col;
            // the load is unconditional (an in-range address), its value
            // dropped past K: a load under a branch makes the compiler wait
            // for every load in flight where the paths meet
            const float4 v = *(const float4*)(a.x + (size_t)bb * a.ldx + (k < K ? k : 0));
            xv[i] = k < K ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto x_store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const uint32_t e = threadIdx.x + 256u * i;
            const uint32_t row = e / (KC / 4), col = (e % (KC / 4)) * 4;
            *(float4*)&xs[buf][row * XS + col] = xv[i];
        }
    };
    auto kb_of = [&](uint32_t c) -> uint32_t {
        const uint32_t kb = c * KC + 32 * j;
        return kb < K ? kb : K - 32;
    };

    f4 acc[MB], accu[SW ? MB : 1];
#pragma unroll
    for (int m = 0; m < MB; m++) {
        acc[m] = f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (SW) accu[m] = f4{0.f, 0.f, 0.f, 0.f};
    }
    // Loads are issued unconditionally (dead waves read in-range addresses
    // whose values go unused), so the wait before a chunk's MFMAs counts only
    // the loads issued before the next chunk's; a load under a branch would
    // make the compiler wait for every load in flight where the paths meet.
    Raw<WT> cur, nxt, curu, nxtu;
    if (c_begin < c_end) {
        x_fetch(c_begin);
        x_store(0);
        raw_load(cur, W0, r, kb_of(c_begin));
        if constexpr (SW) raw_load(curu, W1, r, kb_of(c_begin));
    }
    // one chunk's MFMAs on cur and X buffer buf
    auto chunk = [&](uint32_t c, int buf) {
        if (live) {
            const uint32_t kb = kb_of(c);
            const bool ok = c * KC + 32 * j < K;
            const float* xrow = &xs[buf][((uint32_t)lane & 15) * XS + 32 * j];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                float w[8], wu[8];
                dequant8<WT>(cur, s, kb, ok, w);
                if constexpr (SW) dequant8<WT>(curu, s, kb, ok, wu);
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
    // every chunk but the last prefetches the next one's X and weights
    uint32_t c = c_begin;
    for (; c + 1 < c_end; c++) {
        const int buf = (int)((c - c_begin) & 1);
        __syncthreads();  // X tile of chunk c is in xs[buf]
        x_fetch(c + 1);
        raw_load(nxt, W0, r, kb_of(c + 1));
        if constexpr (SW) raw_load(nxtu, W1, r, kb_of(c + 1));
        chunk(c, buf);
        x_store(buf ^ 1);  // last read in the previous chunk, before this chunk's barrier
        cur = nxt;
        if constexpr (SW) curu = nxtu;
    }
    if (c < c_end) {
        __syncthreads();  // X tile of chunk c is in xs[buf]
        chunk(c, (int)((c - c_begin) & 1));
    }
    if (!live) return;

    // D layout of the 16x16 tile: lane holds rows n0 + 4j + i (i = 0..3) of
    // column b = lane & 15.
#pragma unroll
    for (int m = 0; m < MB; m++) {
        const uint32_t b = b0 + 16u * m + ((uint32_t)lane & 15);
        if (b >= B) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t n = n0 + 4 * j + i;
            if (n >= a.N) continue;
            const float v = acc[m][i];
            const float u = SW ? accu[m][i] : 0.f;
            if (a.ks == 1) {
                emit(a, MODE, b, n, v, u);
            } else {
                const size_t np = SW ? 2 * (size_t)a.N : a.N;
                float* p = a.part + ((size_t)blockIdx.z * B + b) * np;
                p[n] = v;
                if constexpr (SW) p[a.N + n] = u;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// The same GEMM at the f16 matrix-core rate (v_mfma_f32_16x16x32_f16) with
// f32-level accuracy, for Q8_0, F16 and Q4_K weights:
//   X      each row of a 128-column chunk is scaled by a power of two s (its
//          largest |x| brought into [0.5, 1)) and split into f16 hi + lo
//          (x/s = hi + lo to ~22 significant bits; the scaling is exact),
//          staged in LDS as two f16 planes;
//   W      one MFMA covers exactly one 32-column Q8_0 block: lane (j, m) holds
//          weights 8j..8j+7 of the block of row m (int8 -> f16 exactly: the
//          byte biased by 128 is the low mantissa byte of 1024 + q + 128, a
//          packed subtraction removes the bias); F16 weights as they are;
//          Q4_K: one MFMA per 32-column sub-block, a nibble n as the f16
//          1024 + n minus 1024 (exact);
//   sums   D = W (hi + lo) per block in f32, then y_chunk += d * D with the
//          block's scale d (Q8_0; Q4_K: d1 = d * sc, then y_chunk -= m1 *
//          sum(x/s) over the sub-block, m1 = dmin * m, the sums taken while X
//          is staged), and y += s * y_chunk per chunk.  A one-hot x still
//          returns d1 * q - m1 rounded as dequant_row_ref rounds it.
// The products q * (hi or lo) are exact in f32, so the result differs from
// the f32 kernel's only by the split's ~2^-22 and the summation order.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 hh2 __attribute__((ext_vector_type(2)));
constexpr uint32_t HS = KC + 8;  // LDS row stride of an f16 plane (halves)

template <int WT> struct Raw16;
template <> struct Raw16<LK_Q8_0> { uint2 q[4]; uint32_t d; };
template <> struct Raw16<LK_F16> { uint4 q[4]; };
// Q4_K: q[p] = bytes 8j..8j+7 of sub-block pair p of the chunk (low nibbles:
// sub-block 2p, high nibbles: 2p + 1, columns 8j..8j+7 of each); hd = the
// row's 16-byte super-block head (d, dmin, 12 packed scale bytes)
template <> struct Raw16<LK_Q4_K> { uint2 q[2]; uint4 hd; };

// Lane (j, m = row r) of chunk c: weights 8j..8j+7 of each of the chunk's four
// 32-column blocks of row r; Q8_0 also the scale of row r, block 4c + j.
template <int WT>
__device__ __forceinline__ void raw16_load(Raw16<WT>& R, const LkDevW& w, uint32_t r, uint32_t c, uint32_t j,
                                           uint32_t K) {
    if constexpr (WT == LK_Q4_K) {
        // chunk c = half c & 1 of super-block c >> 1 (K is a multiple of 256,
        // so every chunk is whole); 128 qs bytes and a 16-byte head per super-block
        const uint32_t nsb = w.cols / 256, sbk = c >> 1;
        const uint8_t* qs = w.data + ((size_t)r * nsb + sbk) * 128 + (c & 1) * 64 + 8 * j;
        R.q[0] = *(const uint2*)qs;
        R.q[1] = *(const uint2*)(qs + 32);
        R.hd = *(const uint4*)(w.aux + ((size_t)r * nsb + sbk) * 16);
    } else {
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            uint32_t col = c * KC + 32 * blk + 8 * j;
            col = col < K ? col : 0;  // past K: any in-row weights, multiplied by X = 0
            if constexpr (WT == LK_Q8_0) R.q[blk] = *(const uint2*)(w.data + (size_t)r * w.cols + col);
            else R.q[blk] = *(const uint4*)(w.data + ((size_t)r * w.cols + col) * 2);
        }
        if constexpr (WT == LK_Q8_0) {
            const uint32_t b = c * 4 + j;
            R.d = ((const uint16_t*)w.aux)[(size_t)r * (w.cols / 32) + (b < K / 32 ? b : 0)];
        }
    }
}

// 8 weights of block blk as f16.
template <int WT>
__device__ __forceinline__ h8 raw16_w(const Raw16<WT>& R, int blk) {
    if constexpr (WT == LK_F16) {
        return __builtin_bit_cast(h8, R.q[blk]);
    } else if constexpr (WT == LK_Q4_K) {
        // sub-block blk of the chunk: nibbles n -> the f16 1024 + n (bytes
        // [n, 0x64]), minus 1024: exact
        const hh2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
        const uint2 v = R.q[blk >> 1];
        const uint32_t sh = (blk & 1) ? 4u : 0u;
        const uint32_t w0 = (v.x >> sh) & 0x0F0F0F0Fu, w1 = (v.y >> sh) & 0x0F0F0F0Fu;
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
        const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
        const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
        const hh2 q0 = __builtin_bit_cast(hh2, p0) - bias, q1 = __builtin_bit_cast(hh2, p1) - bias;
        const hh2 q2 = __builtin_bit_cast(hh2, p2) - bias, q3 = __builtin_bit_cast(hh2, p3) - bias;
        return h8{q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
    } else {
        const hh2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
        const uint32_t w0 = R.q[blk].x ^ 0x80808080u, w1 = R.q[blk].y ^ 0x80808080u;
        // bytes [u, 0x64, u', 0x64]: the f16 value 1024 + u (u = q + 128)
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
        const uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
        const uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
        const hh2 q0 = __builtin_bit_cast(hh2, p0) - bias, q1 = __builtin_bit_cast(hh2, p1) - bias;
        const hh2 q2 = __builtin_bit_cast(hh2, p2) - bias, q3 = __builtin_bit_cast(hh2, p3) - bias;
        return h8{q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
    }
}

template <int WT, int MB, int MODE>
__global__ __launch_bounds__(256) void gemm16_kernel(const LkGemmArgs a) {
    constexpr bool SW = MODE == LK_MV_SWIGLU;
    constexpr int BR = 16 * MB;
    constexpr int NW = SW ? 2 : 1;
    __shared__ __align__(16) _Float16 xh[2][BR * HS], xl[2][BR * HS];
    __shared__ float xsc[2][BR];
    __shared__ __align__(16) float sd[4][NW][64];  // per wave: the chunk's block scales, [block][row]
    // Q4_K: per wave the chunk's sub-block mins m1 = dmin * m, [block][row]; and
    // per X buffer the sums of each row's scaled values over every 32-column
    // sub-block (the min term is m1 * sum(x) per sub-block)
    __shared__ __align__(16) float sm[WT == LK_Q4_K ? 4 : 1][NW][64];
    __shared__ float xsum[WT == LK_Q4_K ? 2 : 1][BR][4];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t n0 = (blockIdx.x * 4 + wave) * 16;
    const bool live = n0 < a.N;
    const uint32_t B = a.n_rows, K = a.K;
    const uint32_t b0 = blockIdx.y * BR;
    const uint32_t nck = (K + KC - 1) / KC;
    const uint32_t per = (nck + a.ks - 1) / a.ks;
    const uint32_t c_begin = blockIdx.z * per;
    const uint32_t c_end = c_begin + per < nck ? c_begin + per : nck;
    const uint32_t j = (uint32_t)lane >> 4;

    uint32_t si = 0, nb = 0;
    if constexpr (!SW) {
        while (si + 1 < a.nseg && n0 >= nb + a.seg[si].w.rows) {
            nb += a.seg[si].w.rows;
            si++;
        }
    }
    const LkDevW W0 = a.seg[si].w;
    const LkDevW W1 = a.seg[SW ? 1 : si].w;
    uint32_t r = live ? n0 - nb + ((uint32_t)lane & 15) : 0;
    r = r < W0.rows ? r : W0.rows - 1;

    // X staging: thread t takes float4 number t + 256 i of the BR x KC tile; the
    // 32 threads of a row are 32 adjacent lanes (the row's scale by shuffles)
    constexpr int XV = BR * KC / 4 / 256;
    float4 xv[XV];
    auto x_fetch = [&](uint32_t c) {
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const uint32_t e = threadIdx.x + 256u * i;
            const uint32_t row = e / (KC / 4), col = (e % (KC / 4)) * 4;
            uint32_t bb = b0 + row;
            bb = bb < B ? bb : B - 1;
            const uint32_t k = c * KC + col;
            const float4 v = *(const float4*)(a.x + (size_t)bb * a.ldx + (k < K ? k : 0));  // unconditional
            xv[i] = k < K ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto x_store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const uint32_t e = threadIdx.x + 256u * i;
            const uint32_t row = e / (KC / 4), col = (e % (KC / 4)) * 4;
            float mx = fmaxf(fmaxf(fabsf(xv[i].x), fabsf(xv[i].y)), fmaxf(fabsf(xv[i].z), fabsf(xv[i].w)));
#pragma unroll
            for (int o = 1; o < 32; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            int ex = 0;
            (void)frexpf(mx, &ex);                       // mx = f * 2^ex, f in [0.5, 1) (ex = 0 for 0)
            const float inv = ldexpf(1.0f, -ex), sc = ldexpf(1.0f, ex);
            const float v[4] = {xv[i].x * inv, xv[i].y * inv, xv[i].z * inv, xv[i].w * inv};  // exact
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                hi[q] = (_Float16)v[q];
                lo[q] = (_Float16)(v[q] - (float)hi[q]);
            }
            *(uint2*)&xh[buf][row * HS + col] = __builtin_bit_cast(uint2, hi);
            *(uint2*)&xl[buf][row * HS + col] = __builtin_bit_cast(uint2, lo);
            if (col == 0) xsc[buf][row] = sc;
            if constexpr (WT == LK_Q4_K) {
                // the sub-block's 8 float4s sit in 8 adjacent lanes
                float t = (v[0] + v[1]) + (v[2] + v[3]);
                t += __shfl_xor(t, 1, 64);
                t += __shfl_xor(t, 2, 64);
                t += __shfl_xor(t, 4, 64);
                if (col % 32 == 0) xsum[buf][row][col / 32] = t;
            }
        }
    };

    f4 y[MB], yu[SW ? MB : 1];
#pragma unroll
    for (int m = 0; m < MB; m++) {
        y[m] = f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (SW) yu[m] = f4{0.f, 0.f, 0.f, 0.f};
    }
    // unconditional loads, as in gemm_kernel
    Raw16<WT> cur, nxt, curu, nxtu;
    if (c_begin < c_end) {
        x_fetch(c_begin);
        x_store(0);
        raw16_load(cur, W0, r, c_begin, j, K);
        if constexpr (SW) raw16_load(curu, W1, r, c_begin, j, K);
    }
    // one chunk's MFMAs on cur and X buffer buf
    auto chunk = [&](uint32_t c, int buf) {
        if (live) {
            if constexpr (WT == LK_Q8_0) {  // the chunk's block scales: row lane & 15, block j
                sd[wave][0][j * 16 + (lane & 15)] = lk_h2f((uint16_t)cur.d);
                if constexpr (SW) sd[wave][NW - 1][j * 16 + (lane & 15)] = lk_h2f((uint16_t)curu.d);
            } else if constexpr (WT == LK_Q4_K) {
                // sub-block j of the chunk (j + 4 (c & 1) of its super-block):
                // d1 = d * sc and m1 = dmin * m, each rounded once, as
                // dequant_row_ref does (src/gguf/dequant.rs:462-483)
                auto put = [&](const Raw16<WT>& R, int sw) {
                    uint32_t sc, mn;
                    lk::scale_min_k4((c & 1) * 4 + j, R.hd.y, R.hd.z, R.hd.w, sc, mn);
                    const float d = lk_h2f((uint16_t)(R.hd.x & 0xFFFF)), dmin = lk_h2f((uint16_t)(R.hd.x >> 16));
                    sd[wave][sw][j * 16 + (lane & 15)] = __fmul_rn(d, (float)sc);
                    sm[wave][sw][j * 16 + (lane & 15)] = __fmul_rn(dmin, (float)mn);
                };
                put(cur, 0);
                if constexpr (SW) put(curu, NW - 1);
            }
            f4 yc[MB], ycu[SW ? MB : 1];
#pragma unroll
            for (int m = 0; m < MB; m++) {
                yc[m] = f4{0.f, 0.f, 0.f, 0.f};
                if constexpr (SW) ycu[m] = f4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int blk = 0; blk < 4; blk++) {
                const h8 wa = raw16_w<WT>(cur, blk);
                h8 wu;
                if constexpr (SW) wu = raw16_w<WT>(curu, blk);
                float4 dv, du, mv, mu;
                if constexpr (WT == LK_Q8_0 || WT == LK_Q4_K) {
                    dv = *(const float4*)&sd[wave][0][blk * 16 + 4 * j];  // rows 4j..4j+3 of the D layout
                    if constexpr (SW) du = *(const float4*)&sd[wave][NW - 1][blk * 16 + 4 * j];
                }
                if constexpr (WT == LK_Q4_K) {
                    mv = *(const float4*)&sm[wave][0][blk * 16 + 4 * j];
                    if constexpr (SW) mu = *(const float4*)&sm[wave][NW - 1][blk * 16 + 4 * j];
                }
#pragma unroll
                for (int m = 0; m < MB; m++) {
                    const uint32_t xo = (16u * m + ((uint32_t)lane & 15)) * HS + 32 * blk + 8 * j;
                    const h8 bh = *(const h8*)&xh[buf][xo];
                    const h8 bl = *(const h8*)&xl[buf][xo];
                    if constexpr (WT == LK_Q8_0 || WT == LK_Q4_K) {
                        f4 D = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, bh, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, bl, D, 0, 0, 0);
                        yc[m][0] = fmaf(dv.x, D[0], yc[m][0]);
                        yc[m][1] = fmaf(dv.y, D[1], yc[m][1]);
                        yc[m][2] = fmaf(dv.z, D[2], yc[m][2]);
                        yc[m][3] = fmaf(dv.w, D[3], yc[m][3]);
                        float xs = 0.f;
                        if constexpr (WT == LK_Q4_K) {  // minus m1 * sum(x) of the sub-block
                            xs = xsum[buf][16 * m + (lane & 15)][blk];
                            yc[m][0] = fmaf(-mv.x, xs, yc[m][0]);
                            yc[m][1] = fmaf(-mv.y, xs, yc[m][1]);
                            yc[m][2] = fmaf(-mv.z, xs, yc[m][2]);
                            yc[m][3] = fmaf(-mv.w, xs, yc[m][3]);
                        }
                        if constexpr (SW) {
                            f4 E = __builtin_amdgcn_mfma_f32_16x16x32_f16(wu, bh, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                            E = __builtin_amdgcn_mfma_f32_16x16x32_f16(wu, bl, E, 0, 0, 0);
                            ycu[m][0] = fmaf(du.x, E[0], ycu[m][0]);
                            ycu[m][1] = fmaf(du.y, E[1], ycu[m][1]);
                            ycu[m][2] = fmaf(du.z, E[2], ycu[m][2]);
                            ycu[m][3] = fmaf(du.w, E[3], ycu[m][3]);
                            if constexpr (WT == LK_Q4_K) {
                                ycu[m][0] = fmaf(-mu.x, xs, ycu[m][0]);
                                ycu[m][1] = fmaf(-mu.y, xs, ycu[m][1]);
                                ycu[m][2] = fmaf(-mu.z, xs, ycu[m][2]);
                                ycu[m][3] = fmaf(-mu.w, xs, ycu[m][3]);
                            }
                        }
                    } else {
                        yc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, bh, yc[m], 0, 0, 0);
                        yc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, bl, yc[m], 0, 0, 0);
                        if constexpr (SW) {
                            ycu[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wu, bh, ycu[m], 0, 0, 0);
                            ycu[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wu, bl, ycu[m], 0, 0, 0);
                        }
                    }
                }
            }
            // the chunk's row scales: column b = 16m + (lane & 15)
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const float s = xsc[buf][16 * m + (lane & 15)];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    y[m][i] = fmaf(s, yc[m][i], y[m][i]);
                    if constexpr (SW) yu[m][i] = fmaf(s, ycu[m][i], yu[m][i]);
                }
            }
        }
    };
    // every chunk but the last prefetches the next one's X and weights
    uint32_t c = c_begin;
    for (; c + 1 < c_end; c++) {
        const int buf = (int)((c - c_begin) & 1);
        __syncthreads();  // X planes of chunk c are in buffer buf
        x_fetch(c + 1);
        raw16_load(nxt, W0, r, c + 1, j, K);
        if constexpr (SW) raw16_load(nxtu, W1, r, c + 1, j, K);
        chunk(c, buf);
        x_store(buf ^ 1);  // last read in the previous chunk, before this chunk's barrier
        cur = nxt;
        if constexpr (SW) curu = nxtu;
    }
    if (c < c_end) {
        __syncthreads();  // X planes of chunk c are in buffer buf
        chunk(c, (int)((c - c_begin) & 1));
    }
    if (!live) return;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        const uint32_t b = b0 + 16u * m + ((uint32_t)lane & 15);
        if (b >= B) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t n = n0 + 4 * j + i;
            if (n >= a.N) continue;
            const float v = y[m][i];
            const float u = SW ? yu[m][i] : 0.f;
            if (a.ks == 1) {
                emit(a, MODE, b, n, v, u);
            } else {
                const size_t np = SW ? 2 * (size_t)a.N : a.N;
                float* p = a.part + ((size_t)blockIdx.z * B + b) * np;
                p[n] = v;
                if constexpr (SW) p[a.N + n] = u;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// gemm16_kernel for a wide, shallow matrix (the lm_head: N = vocab rows, K =
// hidden <= 1024) and a few activation rows: there every one of the N / 64
// blocks of gemm16_kernel converted the same X tile to its f16 planes
// again, chunk by chunk.  Here a block (8 waves, one per CU: its X planes
// take ~120 KB of LDS) converts its 16 * MB rows of X once, whole K, with
// the same per-(row, chunk) scales, and each wave then streams 16-row weight
// tiles (every chunk of a tile loaded at once, the next tile's loads issued
// before the current tile's MFMAs) against the resident planes.  Per chunk
// the arithmetic is gemm16_kernel's, in the same order, so the results are
// bit-identical to it.
constexpr int WIDE_W = 8;  // waves per block

// NCK: the K chunks of a tile, ceil(K / 128) exactly (a compile-time count,
// so the compiler can count the loads in flight and wait for one chunk at a
// time)
template <int WT, int MB, uint32_t NCK>
__global__ __launch_bounds__(WIDE_W * 64) void gemm16_wide_kernel(const LkGemmArgs a) {
    constexpr int BR = 16 * MB;
    extern __shared__ __align__(16) _Float16 wl[];
    const uint32_t B = a.n_rows, K = a.K, N = a.N;
    const uint32_t nck = (K + KC - 1) / KC;
    const uint32_t xs = nck * KC + 8;  // LDS row stride of a plane (halves)
    _Float16* xh = wl;
    _Float16* xl = wl + BR * xs;
    float* xsc = (float*)(xl + BR * xs);  // [BR][NCK]
    float* sdw = xsc + BR * NCK;     // [WIDE_W][64]: a wave's block scales of one chunk
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t j = (uint32_t)lane >> 4;
    const uint32_t b0 = blockIdx.y * BR;

    const LkDevW W = a.seg[0].w;
    const uint32_t ntile = (N + 15) / 16, step = gridDim.x * WIDE_W;
    Raw16<WT> rw[NCK];
    auto row_of = [&](uint32_t t) {
        const uint32_t r = t * 16 + ((uint32_t)lane & 15);
        return r < N ? r : N - 1;
    };
    // X rows b0 .. b0 + BR - 1, every chunk: gemm16_kernel's x_fetch + x_store
    // (rows past B repeat row B - 1 and are never written out); all of a
    // thread's loads are issued before any conversion
    constexpr int XV = BR * KC / 4 / (WIDE_W * 64);
    float4 xv[NCK][XV];
#pragma unroll
    for (uint32_t c = 0; c < NCK; c++)
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const uint32_t e = threadIdx.x + WIDE_W * 64 * i;
            const uint32_t row = e / (KC / 4), col = (e % (KC / 4)) * 4;
            uint32_t bb = b0 + row;
            bb = bb < B ? bb : B - 1;
            const uint32_t k = c * KC + col;
            const float4 v4 = *(const float4*)(a.x + (size_t)bb * a.ldx + (k < K ? k : 0));
            xv[c][i] = k < K ? v4 : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    {
        // the wave's first weight tile, in flight during the conversion (a
        // wave with no tile reloads the last one, unused)
        const uint32_t t0 = blockIdx.x * WIDE_W + wave;
        const uint32_t r = row_of(t0 < ntile ? t0 : ntile - 1);
#pragma unroll
        for (uint32_t c = 0; c < NCK; c++) raw16_load(rw[c], W, r, c, j, K);
    }
#pragma unroll
    for (uint32_t c = 0; c < NCK; c++)
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const uint32_t e = threadIdx.x + WIDE_W * 64 * i;
            const uint32_t row = e / (KC / 4), col = (e % (KC / 4)) * 4;
            const float4 x4 = xv[c][i];
            float mx = fmaxf(fmaxf(fabsf(x4.x), fabsf(x4.y)), fmaxf(fabsf(x4.z), fabsf(x4.w)));
#pragma unroll
            for (int o = 1; o < 32; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            int ex = 0;
            (void)frexpf(mx, &ex);
            const float inv = ldexpf(1.0f, -ex), sc = ldexpf(1.0f, ex);
            const float v[4] = {x4.x * inv, x4.y * inv, x4.z * inv, x4.w * inv};
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                hi[q] = (_Float16)v[q];
                lo[q] = (_Float16)(v[q] - (float)hi[q]);
            }
            *(uint2*)&xh[row * xs + c * KC + col] = __builtin_bit_cast(uint2, hi);
            *(uint2*)&xl[row * xs + c * KC + col] = __builtin_bit_cast(uint2, lo);
            if (col == 0) xsc[row * NCK + c] = sc;
        }
    __syncthreads();

    // one segment, no bias (checked by the host): outputs are plain stores, so
    // no epilogue load waits (vmcnt) for the next tile's weights in flight
    float* const out = a.seg[0].out;
    const uint32_t ldy = a.ldy;
    float* sd = sdw + wave * 64;
    // one buffer of a tile's chunks: once chunk c is multiplied, its registers
    // take chunk c of the wave's next tile, so a tile's loads are in flight
    // while the current tile is computed (a tile's distance ahead, one buffer)

    // tile t; with NEXT, chunk c's registers are reloaded with tile tn's after use
    auto tile = [&](uint32_t t, auto next, uint32_t tn) {
        constexpr bool NEXT = decltype(next)::value;
        const uint32_t rn = row_of(tn);
        f4 y[MB];
#pragma unroll
        for (int m = 0; m < MB; m++) y[m] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t c = 0; c < NCK; c++) {
            // c < nck always holds (NCK is the chunk count); the uniform branch
            // keeps each chunk's arithmetic in a block of its own, so the
            // compiler does not hoist every chunk's X reads at once (they
            // would spill), while the reload after it stays unconditional
            if (c < nck) {
            if constexpr (WT == LK_Q8_0) sd[j * 16 + (lane & 15)] = lk_h2f((uint16_t)rw[c].d);
            f4 yc[MB];
#pragma unroll
            for (int m = 0; m < MB; m++) yc[m] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int blk = 0; blk < 4; blk++) {
                const h8 wa = raw16_w<WT>(rw[c], blk);
                float4 dv;
                if constexpr (WT == LK_Q8_0) dv = *(const float4*)&sd[blk * 16 + 4 * j];
#pragma unroll
                for (int m = 0; m < MB; m++) {
                    const uint32_t xo = (16u * m + ((uint32_t)lane & 15)) * xs + c * KC + 32 * blk + 8 * j;
                    const h8 bh = *(const h8*)&xh[xo];
                    const h8 bl = *(const h8*)&xl[xo];
                    if constexpr (WT == LK_Q8_0) {
                        f4 D = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, bh, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, bl, D, 0, 0, 0);
                        yc[m][0] = fmaf(dv.x, D[0], yc[m][0]);
                        yc[m][1] = fmaf(dv.y, D[1], yc[m][1]);
                        yc[m][2] = fmaf(dv.z, D[2], yc[m][2]);
                        yc[m][3] = fmaf(dv.w, D[3], yc[m][3]);
                    } else {
                        yc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, bh, yc[m], 0, 0, 0);
                        yc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, bl, yc[m], 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const float sx = xsc[(16 * m + (lane & 15)) * NCK + c];
#pragma unroll
                for (int i = 0; i < 4; i++) y[m][i] = fmaf(sx, yc[m][i], y[m][i]);
            }
            }
            if constexpr (NEXT) raw16_load(rw[c], W, rn, c, j, K);
        }
#pragma unroll
        for (int m = 0; m < MB; m++) {
            const uint32_t b = b0 + 16u * m + ((uint32_t)lane & 15);
            if (b >= B) continue;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t n = t * 16 + 4 * j + i;
                if (n < N) out[(size_t)b * ldy + n] = y[m][i];
            }
        }
    };
    uint32_t t = blockIdx.x * WIDE_W + wave;
    if (t >= ntile) return;  // uniform over the wave; no block barrier follows
    for (; t + step < ntile; t += step) tile(t, std::true_type{}, t + step);
    tile(t, std::false_type{}, t);
}

static size_t wide_lds(int mb, uint32_t nck_hold, uint32_t K) {
    const uint32_t nck = (K + KC - 1) / KC;
    return (size_t)2 * 16 * mb * (nck * KC + 8) * sizeof(_Float16) + 16 * mb * nck_hold * 4 + WIDE_W * 64 * 4;
}

constexpr int WIDE_MAX_DEV = 64;

template <int WT, int MB, uint32_t NCK>
static hipError_t launch_wide_t(const LkGemmArgs& a, hipStream_t st) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= WIDE_MAX_DEV) return hipErrorInvalidDevice;
    // per device: its CU count, and the kernel's dynamic LDS limit raised once
    // (to the largest K this kernel takes)
    static int cus[WIDE_MAX_DEV], ready[WIDE_MAX_DEV];
    if (!ready[dev]) {
        e = hipFuncSetAttribute((const void*)gemm16_wide_kernel<WT, MB, NCK>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)wide_lds(MB, NCK, NCK * KC));
        if (e != hipSuccess) return e;
        e = hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        ready[dev] = 1;
    }
    const dim3 grid((unsigned)cus[dev], (a.n_rows + 16 * MB - 1) / (16 * MB));
    hipLaunchKernelGGL((gemm16_wide_kernel<WT, MB, NCK>), grid, dim3(WIDE_W * 64), wide_lds(MB, NCK, a.K), st, a);
    return hipGetLastError();
}

// The wide kernel's instance for a.K (its chunk count), or
// hipErrorNotSupported: 4-7 chunks (K 385-896) for Q8_0, 4-5 (K 385-640)
// for F16 (the lm_head widths of the shipped configs: 896, 576).
template <int WT, int MB>
static hipError_t launch_wide_k(const LkGemmArgs& a, hipStream_t st) {
    switch ((a.K + KC - 1) / KC) {
    case 4: return launch_wide_t<WT, MB, 4>(a, st);
    case 5: return launch_wide_t<WT, MB, 5>(a, st);
    case 6:
        if constexpr (WT == LK_Q8_0) return launch_wide_t<WT, MB, 6>(a, st);
        break;
    case 7:
        if constexpr (WT == LK_Q8_0) return launch_wide_t<WT, MB, 7>(a, st);
        break;
    default: break;
    }
    return hipErrorNotSupported;
}
static bool wide_k_ok(uint32_t type, uint32_t K) {
    const char* g = getenv("LKHIP_GEMM_WIDE");  // "0": gemm16_kernel for these shapes too
    if (g && strcmp(g, "0") == 0) return false;
    const uint32_t nck = (K + KC - 1) / KC;
    return nck >= 4 && (type == LK_Q8_0 ? nck <= 7 : (type == LK_F16 ? nck <= 5 : false));
}

// Sums the K-split partials of element (b, n) in split order, then the epilogue.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const LkGemmArgs a, int mode) {
    const uint32_t n = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
    if (n >= a.N) return;
    const bool sw = mode == LK_MV_SWIGLU;
    const size_t np = sw ? 2 * (size_t)a.N : a.N;
    const float* p = a.part + (size_t)b * np + n;
    const float v = lk_sum_splits(p, (size_t)a.n_rows * np, a.ks);
    const float u = sw ? lk_sum_splits(p + a.N, (size_t)a.n_rows * np, a.ks) : 0.f;
    emit(a, mode, b, n, v, u);
}

// The f16-rate kernel for Q8_0, F16 and Q4_K (LKHIP_GEMM=f32 keeps the f32 one).
static bool gemm16_on(uint32_t type) {
    if (type != LK_Q8_0 && type != LK_F16 && type != LK_Q4_K) return false;
    static int on = -1;
    if (on < 0) {
        const char* g = getenv("LKHIP_GEMM");
        on = !(g && strcmp(g, "f32") == 0);
    }
    return on == 1;
}

template <int WT, int MB>
hipError_t launch_mb16(const LkGemmArgs& a, int mode, dim3 grid, hipStream_t st) {
    if constexpr (WT == LK_Q8_0 || WT == LK_F16 || WT == LK_Q4_K) {
        switch (mode) {
        case LK_MV_STORE: hipLaunchKernelGGL((gemm16_kernel<WT, MB, LK_MV_STORE>), grid, dim3(256), 0, st, a); break;
        case LK_MV_ACC: hipLaunchKernelGGL((gemm16_kernel<WT, MB, LK_MV_ACC>), grid, dim3(256), 0, st, a); break;
        case LK_MV_SWIGLU: hipLaunchKernelGGL((gemm16_kernel<WT, MB, LK_MV_SWIGLU>), grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

template <int WT, int MB>
hipError_t launch_mb(const LkGemmArgs& a, int mode, dim3 grid, hipStream_t st) {
    if (gemm16_on(WT)) return launch_mb16<WT, MB>(a, mode, grid, st);
    switch (mode) {
    case LK_MV_STORE: hipLaunchKernelGGL((gemm_kernel<WT, MB, LK_MV_STORE>), grid, dim3(256), 0, st, a); break;
    case LK_MV_ACC: hipLaunchKernelGGL((gemm_kernel<WT, MB, LK_MV_ACC>), grid, dim3(256), 0, st, a); break;
    case LK_MV_SWIGLU: hipLaunchKernelGGL((gemm_kernel<WT, MB, LK_MV_SWIGLU>), grid, dim3(256), 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int WT>
hipError_t launch_t(const LkGemmArgs& a, int mode, uint32_t mb, dim3 grid, hipStream_t st) {
    if (mb == 1) return launch_mb<WT, 1>(a, mode, grid, st);
    if (mb == 2) return launch_mb<WT, 2>(a, mode, grid, st);
    return launch_mb<WT, 2>(a, mode, grid, st);
}

}  // namespace lkg

static uint32_t gemm_mb(uint32_t n_rows) { return n_rows <= 16 ? 1 : 2; }

// Output rows from which a single-segment store GEMM with K <= 1024 takes
// gemm16_wide_kernel (the lm_head; the layers' matrices are narrower)
#ifndef LK_GEMM_WIDE_N
#define LK_GEMM_WIDE_N 16384u
#endif

LkGemmPlan lk_gemm_plan(uint32_t type, uint32_t N, uint32_t K, uint32_t n_rows, int mode) {
    (void)type;
    LkGemmPlan p{};
    p.mb = gemm_mb(n_rows);
    const uint32_t gx = (N + 63) / 64, gy = (n_rows + 16 * p.mb - 1) / (16 * p.mb);
    const uint32_t nck = (K + lkg::KC - 1) / lkg::KC;
    // enough blocks for 2 per CU; every split keeps at least one chunk
    uint32_t ks = (512 + gx * gy - 1) / (gx * gy);
    if (ks > nck) ks = nck;
    if (ks < 1) ks = 1;
    const uint32_t per = (nck + ks - 1) / ks;
    p.ks = (nck + per - 1) / per;
    p.part_floats = p.ks > 1 ? (size_t)p.ks * n_rows * N * (mode == LK_MV_SWIGLU ? 2 : 1) : 0;
    return p;
}

bool lk_gemm_shape_ok(uint32_t type, uint32_t N, uint32_t K) {
    if (N == 0 || K == 0 || K % 32) return false;
    if (type == LK_Q4_K && K % 256) return false;
    return type == LK_Q8_0 || type == LK_F16 || type == LK_Q4_K || type == LK_Q8_SM;
}

hipError_t lk_gemm_launch(LkGemmArgs a, int mode, hipStream_t st, uint32_t* deferred_ks) {
    const uint32_t type = a.seg[0].w.type;
    if (a.n_rows == 0) return hipSuccess;
    if (!lk_gemm_shape_ok(type, a.N, a.K) || (mode != LK_MV_STORE && mode != LK_MV_ACC && mode != LK_MV_SWIGLU))
        return hipErrorInvalidValue;
    for (uint32_t i = 0; i < a.nseg; i++)
        if (a.seg[i].w.type != type || a.seg[i].w.cols != a.K) return hipErrorInvalidValue;
    // a wave's 16-row tile lies in one segment
    if (mode != LK_MV_SWIGLU)
        for (uint32_t i = 0; i + 1 < a.nseg; i++)
            if (a.seg[i].w.rows % 16) return hipErrorInvalidValue;
    if (a.ldx % 4 || (size_t)(uintptr_t)a.x % 16) return hipErrorInvalidValue;  // float4 X loads
    // a wide, shallow matrix (the lm_head: one segment, no bias) without a K split: the kernel that
    // converts X once per block (bit-identical to gemm16_kernel)
    if (mode == LK_MV_STORE && a.nseg == 1 && !a.seg[0].bias && a.ks <= 1 && a.N >= LK_GEMM_WIDE_N &&
        lkg::wide_k_ok(type, a.K) && lkg::gemm16_on(type)) {
        if (deferred_ks) *deferred_ks = 0;
        a.ks = 1;
        const bool one = a.n_rows <= 16;
        if (type == LK_Q8_0) return one ? lkg::launch_wide_k<LK_Q8_0, 1>(a, st) : lkg::launch_wide_k<LK_Q8_0, 2>(a, st);
        return one ? lkg::launch_wide_k<LK_F16, 1>(a, st) : lkg::launch_wide_k<LK_F16, 2>(a, st);
    }
    const LkGemmPlan p = lk_gemm_plan(type, a.N, a.K, a.n_rows, mode);
    if (a.ks == 0) a.ks = p.ks;
    if (a.ks > 1 && !a.part) return hipErrorInvalidValue;
    dim3 grid((a.N + 63) / 64, (a.n_rows + 16 * p.mb - 1) / (16 * p.mb), a.ks);
    hipError_t e;
    switch (type) {
    case LK_Q8_0: e = lkg::launch_t<LK_Q8_0>(a, mode, p.mb, grid, st); break;
    case LK_F16: e = lkg::launch_t<LK_F16>(a, mode, p.mb, grid, st); break;
    case LK_Q8_SM: e = lkg::launch_t<LK_Q8_SM>(a, mode, p.mb, grid, st); break;
    default: e = lkg::launch_t<LK_Q4_K>(a, mode, p.mb, grid, st); break;
    }
    if (deferred_ks) *deferred_ks = a.ks > 1 ? a.ks : 0;
    if (e != hipSuccess || a.ks == 1 || deferred_ks) return e;
    hipLaunchKernelGGL(lkg::gemm_reduce_kernel, dim3((a.N + 255) / 256, a.n_rows), dim3(256), 0, st, a, mode);
    return hipGetLastError();
}
