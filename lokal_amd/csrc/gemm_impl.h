// gemm_impl.h -- the multi-row GEMM's weight loads and exact dequantization
// (gemm.hip), shared with the Batcher's persistent step (batch_step.hip).
#pragma once
#include "lkhip_common.h"
#include "matvec_impl.h"

namespace lkg {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr uint32_t KC = 128;   // K columns per chunk
constexpr uint32_t XS = KC + 4;  // LDS row stride of the X tile (floats)

template <int WT> struct Raw;
template <> struct Raw<LK_Q8_0> { uint4 q[2]; uint32_t d; };
template <> struct Raw<LK_F16> { uint4 q[4]; };
template <> struct Raw<LK_Q4_K> { uint4 q[2]; uint4 hd; };
template <> struct Raw<LK_Q8_SM> { uint4 q[2]; uint4 sm; };  // (s, m) of the lane's two 16-weight groups

// Raw bytes of the 32 weights (row r, columns kb..kb+31) of one lane.
template <int WT>
__device__ __forceinline__ void raw_load(Raw<WT>& R, const LkDevW& w, uint32_t r, uint32_t kb) {
    if constexpr (WT == LK_Q8_0) {
        const uint4* p = (const uint4*)(w.data + (size_t)r * w.cols + kb);
        R.q[0] = p[0];
        R.q[1] = p[1];
        R.d = ((const uint16_t*)w.aux)[(size_t)r * (w.cols / 32) + kb / 32];
    } else if constexpr (WT == LK_Q8_SM) {
        const uint4* p = (const uint4*)(w.data + (size_t)r * w.cols + kb);
        R.q[0] = p[0];
        R.q[1] = p[1];
        R.sm = *(const uint4*)(w.aux + ((size_t)r * (w.cols / 16) + kb / 16) * 8);
    } else if constexpr (WT == LK_F16) {
        const uint4* p = (const uint4*)(w.data + ((size_t)r * w.cols + kb) * 2);
#pragma unroll
        for (int i = 0; i < 4; i++) R.q[i] = p[i];
    } else {
        const uint32_t nsb = w.cols / 256, sb = kb / 256, g = (kb % 256) / 64;
        const uint4* p = (const uint4*)(w.data + ((size_t)r * nsb + sb) * 128 + 32 * g);
        R.q[0] = p[0];
        R.q[1] = p[1];
        R.hd = *(const uint4*)(w.aux + ((size_t)r * nsb + sb) * 16);
    }
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Weights 8*s .. 8*s+7 of the lane's 32 as exact f32 (dequant_row_ref,
// src/gguf/dequant.rs:199-203 F16, :231-239 Q8_0, :462-483 Q4_K, :484-533
// Q5_K / Q6_K as Q8_SM); zero when
// the lane's columns lie past K.
template <int WT>
__device__ __forceinline__ void dequant8(const Raw<WT>& R, int s, uint32_t kb, bool ok, float* w) {
    if constexpr (WT == LK_Q8_0) {
        const float d = ok ? lk_h2f((uint16_t)R.d) : 0.f;
        const uint4 v = R.q[s >> 1];
        const uint32_t w0 = word_of(v, (s & 1) * 2), w1 = word_of(v, (s & 1) * 2 + 1);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            w[t] = __fmul_rn((float)((int32_t)(w0 << (24 - 8 * t)) >> 24), d);
            w[4 + t] = __fmul_rn((float)((int32_t)(w1 << (24 - 8 * t)) >> 24), d);
        }
    } else if constexpr (WT == LK_Q8_SM) {
        // weights 8s..8s+7 lie in group s >> 1: y = s*q - m
        const float sv = __uint_as_float(s < 2 ? R.sm.x : R.sm.z), mv = __uint_as_float(s < 2 ? R.sm.y : R.sm.w);
        const uint4 v = R.q[s >> 1];
        const uint32_t w0 = word_of(v, (s & 1) * 2), w1 = word_of(v, (s & 1) * 2 + 1);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float q0 = (float)((int32_t)(w0 << (24 - 8 * t)) >> 24), q1 = (float)((int32_t)(w1 << (24 - 8 * t)) >> 24);
            w[t] = ok ? __fsub_rn(__fmul_rn(sv, q0), mv) : 0.f;
            w[4 + t] = ok ? __fsub_rn(__fmul_rn(sv, q1), mv) : 0.f;
        }
    } else if constexpr (WT == LK_F16) {
        const uint4 v = R.q[s];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t x = word_of(v, i);
            w[2 * i] = ok ? lk_h2f((uint16_t)(x & 0xFFFF)) : 0.f;
            w[2 * i + 1] = ok ? lk_h2f((uint16_t)(x >> 16)) : 0.f;
        }
    } else {
        // sub-block is = (kb % 256) / 32: low nibbles for even, high for odd
        const uint32_t is = (kb % 256) / 32;
        const float d = lk_h2f((uint16_t)(R.hd.x & 0xFFFF));
        const float dmin = lk_h2f((uint16_t)(R.hd.x >> 16));
        uint32_t sc, m;
        lk::scale_min_k4(is, R.hd.y, R.hd.z, R.hd.w, sc, m);
        const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)m);
        const uint4 v = R.q[s >> 1];
        const uint32_t sh = (is & 1) * 4;
        const uint32_t w0 = word_of(v, (s & 1) * 2), w1 = word_of(v, (s & 1) * 2 + 1);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t q0 = (w0 >> (8 * t + sh)) & 15u, q1 = (w1 >> (8 * t + sh)) & 15u;
            w[t] = ok ? __fsub_rn(__fmul_rn(d1, (float)q0), m1) : 0.f;
            w[4 + t] = ok ? __fsub_rn(__fmul_rn(d1, (float)q1), m1) : 0.f;
        }
    }
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }


}  // namespace lkg
