// matvec_impl.h -- the dequant-fused matvec kernel, one template for every
// weight type.  Included by matvec_{q8_0,f16,q4_k,q8_sm}.hip, each of which
// instantiates it for one type so they compile in parallel.
//
// Work split: one wave (64 lanes) owns R output rows.  A row's payload is cut
// into 16-byte "chunks" (Q8_0, Q8_SM: 16 weights, F16: 8, Q4_K: 32 nibbles); lane l
// owns chunks l, l+64, l+128, ...  Every 16-byte chunk is one global_load_dwordx4,
// so a wave load is one contiguous 1 KiB run of the row.  A pass issues all
// R x NCH chunk loads of a lane before any arithmetic, so each lane keeps
// R*NCH*16 bytes in flight; NCH = ceil(chunks/64) covers a row in one pass for
// every shape of the shipped configs.  x (f32) is read from L1/L2 and reused
// across the R rows.  The per-lane f32 partials are reduced across the wave
// by xor-shuffles (DPP/ds_swizzle), then lane 0 runs the epilogue
// (bias, residual add, SwiGLU, or argmax key).
#pragma once
#include "lkhip_common.h"

namespace lk {

template <int WT> struct ChunkTraits;
template <> struct ChunkTraits<LK_Q8_0> { static constexpr uint32_t elems = 16; };
template <> struct ChunkTraits<LK_F16> { static constexpr uint32_t elems = 8; };
template <> struct ChunkTraits<LK_Q4_K> { static constexpr uint32_t elems = 32; };
template <> struct ChunkTraits<LK_Q8_SM> { static constexpr uint32_t elems = 16; };

typedef unsigned int lk_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int lk_u32x2 __attribute__((ext_vector_type(2)));

// The (s, m) pair of Q8_SM chunk ch.
__device__ __forceinline__ uint2 ld_sm(const uint8_t* ap, uint32_t ch) {
    const lk_u32x2 v = lk_g((const lk_u32x2*)ap)[ch];
    return make_uint2(v.x, v.y);
}

// 16-byte streaming load of weight bytes (read once per token: nontemporal).
__device__ __forceinline__ uint4 ld_stream16(const uint8_t* p) {
    const lk_u32x4 v = __builtin_nontemporal_load(lk_g((const lk_u32x4*)p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float sbyte(uint32_t d, int k) {
    return (float)((int32_t)(d << (24 - 8 * k)) >> 24);
}

// Q8_0: sum_j (i8)q_j * x_j over 16 weights; the block scale d is applied by
// the caller (the CPU value (i8)q*d is exact, so a one-hot x returns it bit-for-bit).
__device__ __forceinline__ float dot_q8(uint4 q, const float* __restrict__ x) {
    const float4 x0 = *(const float4*)(x + 0), x1 = *(const float4*)(x + 4);
    const float4 x2 = *(const float4*)(x + 8), x3 = *(const float4*)(x + 12);
    float s0 = sbyte(q.x, 0) * x0.x, s1 = sbyte(q.x, 1) * x0.y;
    s0 = fmaf(sbyte(q.x, 2), x0.z, s0); s1 = fmaf(sbyte(q.x, 3), x0.w, s1);
    s0 = fmaf(sbyte(q.y, 0), x1.x, s0); s1 = fmaf(sbyte(q.y, 1), x1.y, s1);
    s0 = fmaf(sbyte(q.y, 2), x1.z, s0); s1 = fmaf(sbyte(q.y, 3), x1.w, s1);
    s0 = fmaf(sbyte(q.z, 0), x2.x, s0); s1 = fmaf(sbyte(q.z, 1), x2.y, s1);
    s0 = fmaf(sbyte(q.z, 2), x2.z, s0); s1 = fmaf(sbyte(q.z, 3), x2.w, s1);
    s0 = fmaf(sbyte(q.w, 0), x3.x, s0); s1 = fmaf(sbyte(q.w, 1), x3.y, s1);
    s0 = fmaf(sbyte(q.w, 2), x3.z, s0); s1 = fmaf(sbyte(q.w, 3), x3.w, s1);
    return s0 + s1;
}

// Q8_SM: 16 int8 weights sharing one (s, m): s*sum(q x) - m*sum(x), the two
// products rounded before the subtraction, so a one-hot x yields s*q - m, the
// stored element (dequant_row_ref of Q6_K / Q5_K, src/gguf/dequant.rs:484-533).
__device__ __forceinline__ float dot_q8sm(uint4 q, uint2 sm, const float* __restrict__ x) {
    const float sq = dot_q8(q, x);
    const float4 x0 = *(const float4*)(x + 0), x1 = *(const float4*)(x + 4);
    const float4 x2 = *(const float4*)(x + 8), x3 = *(const float4*)(x + 12);
    const float sx = (((x0.x + x0.y) + (x0.z + x0.w)) + ((x1.x + x1.y) + (x1.z + x1.w))) +
                     (((x2.x + x2.y) + (x2.z + x2.w)) + ((x3.x + x3.y) + (x3.z + x3.w)));
    return __fsub_rn(__fmul_rn(__uint_as_float(sm.x), sq), __fmul_rn(__uint_as_float(sm.y), sx));
}

__device__ __forceinline__ float2 h2x2(uint32_t v) {
    return make_float2(__half2float(__ushort_as_half((uint16_t)(v & 0xFFFF))),
                       __half2float(__ushort_as_half((uint16_t)(v >> 16))));
}

// F16: 8 weights.
__device__ __forceinline__ float dot_f16(uint4 q, const float* __restrict__ x) {
    const float4 x0 = *(const float4*)(x + 0), x1 = *(const float4*)(x + 4);
    float2 a = h2x2(q.x), b = h2x2(q.y), c = h2x2(q.z), d = h2x2(q.w);
    float s0 = a.x * x0.x, s1 = a.y * x0.y;
    s0 = fmaf(b.x, x0.z, s0); s1 = fmaf(b.y, x0.w, s1);
    s0 = fmaf(c.x, x1.x, s0); s1 = fmaf(c.y, x1.y, s1);
    s0 = fmaf(d.x, x1.z, s0); s1 = fmaf(d.y, x1.w, s1);
    return s0 + s1;
}

// scale_min_k4 (src/gguf/dequant.rs:141-150) on the 12 packed bytes held in
// three dwords; j is lane-varying, so bytes are picked by shifts.
__device__ __forceinline__ uint32_t kbyte(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t i) {
    uint32_t w = (i < 4) ? s0 : ((i < 8) ? s1 : s2);
    return (w >> (8 * (i & 3))) & 0xFFu;
}
__device__ __forceinline__ void scale_min_k4(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc,
                                             uint32_t& m) {
    if (j < 4) {
        sc = kbyte(s0, s1, s2, j) & 63u;
        m = kbyte(s0, s1, s2, j + 4) & 63u;
    } else {
        sc = (kbyte(s0, s1, s2, j + 4) & 0x0Fu) | ((kbyte(s0, s1, s2, j - 4) >> 6) << 4);
        m = (kbyte(s0, s1, s2, j + 4) >> 4) | ((kbyte(s0, s1, s2, j) >> 6) << 4);
    }
}

// scale_min_k4 for the sub-block pair j = 2g, 2g + 1 (g = 0..3) in
// straight-line bit-field extracts.  Byte jj = j & 3 sits at bit 8*jj of a
// scale dword; for j < 4, sc = s0[jj] & 63 and m = s1[jj] & 63; for j >= 4,
// sc = (s2[jj] & 15) | ((s0[jj] >> 6) << 4) and m = (s2[jj] >> 4) |
// ((s1[jj] >> 6) << 4).  Both forms are "4 low bits from A | 2 bits from
// s0 (s1) << 4", with A and the bit offsets chosen by g alone, so a lane
// whose g is fixed pays two selects and four extracts per value.
__device__ __forceinline__ void scale_min_k4_pair(uint32_t g, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc0,
                                                  uint32_t& m0, uint32_t& sc1, uint32_t& m1) {
    const bool lo = g < 2;
    const uint32_t sh = 16u * (g & 1u);        // byte jj of j = 2g
    const uint32_t A = lo ? s0 : s2, B = lo ? s1 : s2;
    const uint32_t ob = lo ? 0u : 4u, oh = lo ? 4u : 6u;
    auto bf = [](uint32_t v, uint32_t o, uint32_t n) { return (v >> o) & ((1u << n) - 1u); };
    sc0 = bf(A, sh, 4) | (bf(s0, sh + oh, 2) << 4);
    m0 = bf(B, sh + ob, 4) | (bf(s1, sh + oh, 2) << 4);
    sc1 = bf(A, sh + 8, 4) | (bf(s0, sh + 8 + oh, 2) << 4);
    m1 = bf(B, sh + 8 + ob, 4) | (bf(s1, sh + 8 + oh, 2) << 4);
}

// Q4_K: 16 bytes = 16 low nibbles (elements e0..e0+15 of sub-block 2g) and 16
// high nibbles (e0+32.. of sub-block 2g+1).  Returns
//   (d1*sum(q_lo x) - m1*sum(x_lo)) + (d2*sum(q_hi x) - m2*sum(x_hi))
// with d1 = d*sc, m1 = dmin*m rounded first and the products kept unfused,
// so a one-hot x yields d1*q - m1 exactly as dequant_row_ref does
// (src/gguf/dequant.rs:462-483).
__device__ __forceinline__ float dot_q4k(uint4 q, uint4 hdr, uint32_t k, const float* __restrict__ xlo) {
    const float* xhi = xlo + 32;
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float sql = 0.f, sxl = 0.f, sqh = 0.f, sxh = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xl = *(const float4*)(xlo + 4 * i);
        const float4 xh = *(const float4*)(xhi + 4 * i);
        uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
        sql = fmaf((float)(lo & 0xFF), xl.x, sql);
        sql = fmaf((float)((lo >> 8) & 0xFF), xl.y, sql);
        sql = fmaf((float)((lo >> 16) & 0xFF), xl.z, sql);
        sql = fmaf((float)(lo >> 24), xl.w, sql);
        sqh = fmaf((float)(hi & 0xFF), xh.x, sqh);
        sqh = fmaf((float)((hi >> 8) & 0xFF), xh.y, sqh);
        sqh = fmaf((float)((hi >> 16) & 0xFF), xh.z, sqh);
        sqh = fmaf((float)(hi >> 24), xh.w, sqh);
        sxl += (xl.x + xl.y) + (xl.z + xl.w);
        sxh += (xh.x + xh.y) + (xh.z + xh.w);
    }
    const float d = __half2float(__ushort_as_half((uint16_t)(hdr.x & 0xFFFF)));
    const float dmin = __half2float(__ushort_as_half((uint16_t)(hdr.x >> 16)));
    uint32_t sca, ma, scb, mb;
    scale_min_k4_pair(k >> 1, hdr.y, hdr.z, hdr.w, sca, ma, scb, mb);
    const float d1 = __fmul_rn(d, (float)sca), m1 = __fmul_rn(dmin, (float)ma);
    const float d2 = __fmul_rn(d, (float)scb), m2 = __fmul_rn(dmin, (float)mb);
    const float lo_part = __fsub_rn(__fmul_rn(d1, sql), __fmul_rn(m1, sxl));
    const float hi_part = __fsub_rn(__fmul_rn(d2, sqh), __fmul_rn(m2, sxh));
    return lo_part + hi_part;
}

// One element of a weight row, exactly as dequant_row_ref computes it
// (src/gguf/dequant.rs:199-203 F16, :231-239 Q8_0, :462-483 Q4_K,
// :484-533 Q5_K / Q6_K as Q8_SM; Q4_0 / Q5_0 are stored as Q8_0).
}  // namespace lk
__device__ __forceinline__ float lk_embed_elem(const LkDevW& w, uint32_t r, uint32_t j) {
    if (w.type == LK_F16) {
        return lk_h2f(((const uint16_t*)w.data)[(size_t)r * w.cols + j]);
    } else if (w.type == LK_Q8_0) {
        const int8_t q = ((const int8_t*)w.data)[(size_t)r * w.cols + j];
        const float d = lk_h2f(((const uint16_t*)w.aux)[(size_t)r * (w.cols / 32) + j / 32]);
        return __fmul_rn((float)q, d);
    } else if (w.type == LK_Q4_K) {
        const uint32_t nsb = w.cols / 256, sb = j / 256, e = j % 256;
        const uint8_t* hdr = w.aux + ((size_t)r * nsb + sb) * 16;
        const uint8_t* qs = w.data + ((size_t)r * nsb + sb) * 128;
        const float d = lk_h2f((uint16_t)(hdr[0] | (hdr[1] << 8)));
        const float dmin = lk_h2f((uint16_t)(hdr[2] | (hdr[3] << 8)));
        const uint32_t grp = e / 64, within = e % 64, hi = within / 32, l = within % 32;
        const uint32_t is = 2 * grp + hi;
        const uint32_t* s = (const uint32_t*)(hdr + 4);
        uint32_t sc, m;
        lk::scale_min_k4(is, s[0], s[1], s[2], sc, m);
        const uint8_t byte = qs[grp * 32 + l];
        const uint32_t q = hi ? (byte >> 4) : (byte & 0x0F);
        const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)m);
        return __fsub_rn(__fmul_rn(d1, (float)q), m1);
    } else if (w.type == LK_Q8_SM) {
        const int8_t q = ((const int8_t*)w.data)[(size_t)r * w.cols + j];
        const float2 sm = ((const float2*)w.aux)[(size_t)r * (w.cols / 16) + j / 16];
        return __fsub_rn(__fmul_rn(sm.x, (float)q), sm.y);
    } else {  // F32
        return ((const float*)w.data)[(size_t)r * w.cols + j];
    }
}

namespace lk {

template <int WT>
__device__ __forceinline__ size_t row_data_bytes(uint32_t cols) {
    if constexpr (WT == LK_Q8_0 || WT == LK_Q8_SM) return cols;
    else if constexpr (WT == LK_F16) return (size_t)cols * 2;
    else return (size_t)(cols / 256) * 128;
}
template <int WT>
__device__ __forceinline__ size_t row_aux_bytes(uint32_t cols) {
    if constexpr (WT == LK_Q8_0) return (size_t)(cols / 32) * 2;
    else if constexpr (WT == LK_Q8_SM) return (size_t)(cols / 16) * 8;
    else if constexpr (WT == LK_F16) return 0;
    else return (size_t)(cols / 256) * 16;
}

// One weight row held in registers: its 16-byte chunks for this lane.
template <int WT, int NCH>
struct Row {
    uint4 q[NCH];
    uint32_t hd[NCH];  // Q4_K: dword (lane & 3) of the chunk's 16-byte super-block head (see q4k_head)
    uint32_t d[NCH];  // Q8_0 block scales, raw f16 bits: converted at use, so issuing never waits
    uint2 sm[NCH];    // Q8_SM (s, m) bits
};

template <int WT>
__device__ __forceinline__ const uint8_t* row_ptr(const LkDevW& w, uint32_t r) {
    return w.data + (size_t)r * row_data_bytes<WT>(w.cols);
}
template <int WT>
__device__ __forceinline__ const uint8_t* aux_ptr(const LkDevW& w, uint32_t r) {
    return w.aux + (size_t)r * row_aux_bytes<WT>(w.cols);
}

// Issues the row's loads.  Every lane loads (lanes past the row end reload
// chunk 0 and their products are dropped in row_dot): a lane-dependent branch
// here would let the compiler pull the scale conversion, and with it a wait
// for the load, into the branch, serialising the rows of a batch.
template <int WT, int NCH>
__device__ __forceinline__ void row_issue(Row<WT, NCH>& R, const LkDevW& w, uint32_t r, int lane) {
    const uint32_t nchunk = w.cols / ChunkTraits<WT>::elems;
    const uint8_t* rp = row_ptr<WT>(w, r);
    const uint8_t* ap = aux_ptr<WT>(w, r);
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const uint32_t ch0 = (uint32_t)lane + 64u * i;
        const uint32_t ch = ch0 < nchunk ? ch0 : 0u;
        R.q[i] = ld_stream16(rp + 16u * ch);
        if constexpr (WT == LK_Q8_0) R.d[i] = (uint32_t)lk_g((const uint16_t*)ap)[ch >> 1];
        if constexpr (WT == LK_Q8_SM) R.sm[i] = ld_sm(ap, ch);
        if constexpr (WT == LK_Q4_K) R.hd[i] = lk_g((const uint32_t*)(ap + 16u * (ch >> 3)))[lane & 3];
    }
}

// A Q4_K chunk's super-block head from the dwords its quad of lanes holds:
// lanes 8m..8m+7 share one head (8 chunks of 32 values per super-block, and
// a row's chunk count is a multiple of 8), and lane l holds its dword l & 3,
// so each lane rebuilds the whole head by 4 quad-broadcast moves -- 1 VGPR
// per held chunk instead of 4.  Every lane of the wave must execute this.
__device__ __forceinline__ uint4 q4k_head(uint32_t w) {
    const int v = (int)w;
    return make_uint4((uint32_t)__builtin_amdgcn_mov_dpp(v, 0x00, 0xF, 0xF, true),
                      (uint32_t)__builtin_amdgcn_mov_dpp(v, 0x55, 0xF, 0xF, true),
                      (uint32_t)__builtin_amdgcn_mov_dpp(v, 0xAA, 0xF, 0xF, true),
                      (uint32_t)__builtin_amdgcn_mov_dpp(v, 0xFF, 0xF, 0xF, true));
}

// This lane's partial dot of the row with x (LDS); reduce across the wave after.
// Straight-line: lanes past the row end compute on chunk 0 and drop the term.
template <int WT, int NCH>
__device__ __forceinline__ float row_dot(const Row<WT, NCH>& R, const float* x, uint32_t cols, int lane) {
    const uint32_t nchunk = cols / ChunkTraits<WT>::elems;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const uint32_t ch0 = (uint32_t)lane + 64u * i;
        const bool ok = ch0 < nchunk;
        const uint32_t ch = ok ? ch0 : 0u;
        float t;
        if constexpr (WT == LK_Q8_0) {
            const float s = fmaf(lk_h2f((uint16_t)R.d[i]), dot_q8(R.q[i], x + ch * 16), acc);
            acc = ok ? s : acc;
            continue;
        } else if constexpr (WT == LK_F16) {
            t = dot_f16(R.q[i], x + ch * 8);
        } else if constexpr (WT == LK_Q8_SM) {
            t = dot_q8sm(R.q[i], R.sm[i], x + ch * 16);
        } else {
            const uint32_t sb = ch >> 3, k = ch & 7;
            t = dot_q4k(R.q[i], q4k_head(R.hd[i]), k, x + sb * 256 + (k >> 1) * 64 + (k & 1) * 16);
        }
        acc += ok ? t : 0.f;
    }
    return acc;
}

// row_dot with this lane's x slice already in registers (xr[i] = the x values
// chunk i of the lane multiplies; Q4_K: 16 low-nibble then 16 high-nibble values).
template <int WT, int NCH>
__device__ __forceinline__ float row_dot_reg(const Row<WT, NCH>& R, const float (&xr)[NCH][ChunkTraits<WT>::elems],
                                             uint32_t cols, int lane) {
    const uint32_t nchunk = cols / ChunkTraits<WT>::elems;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const uint32_t ch = (uint32_t)lane + 64u * i;
        float t;
        if constexpr (WT == LK_Q8_0) {
            const float s = fmaf(lk_h2f((uint16_t)R.d[i]), dot_q8(R.q[i], xr[i]), acc);
            acc = ch < nchunk ? s : acc;
            continue;
        } else if constexpr (WT == LK_F16) {
            t = dot_f16(R.q[i], xr[i]);
        } else if constexpr (WT == LK_Q8_SM) {
            t = dot_q8sm(R.q[i], R.sm[i], xr[i]);
        } else {
            float xx[64];  // dot_q4k reads x[0..15] and x[32..47]
#pragma unroll
            for (int e = 0; e < 16; e++) {
                xx[e] = xr[i][e];
                xx[32 + e] = xr[i][16 + e];
            }
            t = dot_q4k(R.q[i], q4k_head(R.hd[i]), ch & 7, xx);
        }
        acc += ch < nchunk ? t : 0.f;
    }
    return acc;
}

template <int WT, int NCH, int R, int MODE>
__global__ __launch_bounds__(256) void matvec_kernel(const LkMvArgs a) {
    constexpr int NR = (MODE == LK_MV_SWIGLU) ? 2 * R : R;
    constexpr uint32_t CE = ChunkTraits<WT>::elems;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t cols = a.cols;
    const uint32_t nchunk = cols / CE;
    const float* __restrict__ x = a.x;
    uint64_t key = 0;  // LK_MV_ARGMAX: this wave's best (value, row) key
    // A row in one pass with a small x slice per lane (Q8_0 / Q8_SM up to 2
    // chunks, F16 up to 4): the slice is read once into registers for every
    // row group of the wave, instead of from L1/L2 for each group.
    constexpr bool XREG = (WT == LK_Q8_0 || WT == LK_Q8_SM) ? NCH <= 2 : (WT == LK_F16 ? NCH <= 4 : false);
    float xr[XREG ? NCH : 1][CE];
    if constexpr (XREG) {
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const uint32_t c = (uint32_t)lane + 64u * i;
#pragma unroll
            for (int e = 0; e < (int)CE; e += 4) {
                const float4 v = c < nchunk ? *(const float4*)(x + (size_t)c * CE + e) : make_float4(0.f, 0.f, 0.f, 0.f);
                xr[i][e] = v.x;
                xr[i][e + 1] = v.y;
                xr[i][e + 2] = v.z;
                xr[i][e + 3] = v.w;
            }
        }
    }
    // grid-stride over R-row groups: the grid is capped (lk_matvec_plan), so
    // large matrices keep a chip-filling set of waves that each take several
    // groups instead of launching one short-lived wave per group
    for (uint32_t row_base = wave * R; row_base < a.total_rows; row_base += gridDim.x * 4u * R) {

    const uint8_t* rp[NR];
    const uint8_t* ap[NR];
    bool rv[NR];
    uint32_t rr[NR];
    int rs[NR];
#pragma unroll
    for (int j = 0; j < NR; j++) {
        uint32_t gr = row_base + (uint32_t)(j % R);
        int si = 0;
        uint32_t r = gr;
        if constexpr (MODE == LK_MV_SWIGLU) {
            si = j / R;
        } else {
            if (a.nseg > 1 && r >= a.seg[0].w.rows) {
                r -= a.seg[0].w.rows;
                si = 1;
                if (a.nseg > 2 && r >= a.seg[1].w.rows) {
                    r -= a.seg[1].w.rows;
                    si = 2;
                }
            }
        }
        rv[j] = gr < a.total_rows;
        if (!rv[j]) r = 0;
        rr[j] = r;
        rs[j] = si;
        const LkDevW& w = a.seg[si].w;
        rp[j] = w.data + (size_t)r * row_data_bytes<WT>(cols);
        ap[j] = w.aux + (size_t)r * row_aux_bytes<WT>(cols);
    }

    float acc[NR];
#pragma unroll
    for (int j = 0; j < NR; j++) acc[j] = 0.f;

    for (uint32_t base = 0; base < nchunk; base += 64 * NCH) {
        // Straight-line loads (a chunk past the row end reloads chunk 0, an
        // invalid row is row 0 of its segment; both are dropped below): a
        // lane-dependent guard here would pull the scale conversion, and with
        // it a wait for the loads, into the guarded block row by row.
        uint4 wq[NR][NCH];
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const uint32_t c = base + (uint32_t)lane + 64u * i;
            const uint32_t cc = c < nchunk ? c : 0u;
#pragma unroll
            for (int j = 0; j < NR; j++) wq[j][i] = ld_stream16(rp[j] + 16u * cc);
        }
        if constexpr (WT == LK_Q8_0) {
            uint32_t dbits[NR][NCH];  // raw f16 scale bits, converted at use
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const uint32_t c = base + (uint32_t)lane + 64u * i;
                const uint32_t cc = c < nchunk ? c : 0u;
#pragma unroll
                for (int j = 0; j < NR; j++) dbits[j][i] = lk_g((const uint16_t*)ap[j])[cc >> 1];
            }
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const uint32_t c = base + (uint32_t)lane + 64u * i;
                const float* xc = XREG ? xr[XREG ? i : 0] : x + (size_t)(c < nchunk ? c : 0u) * 16;
#pragma unroll
                for (int j = 0; j < NR; j++) {
                    const float t = fmaf(lk_h2f((uint16_t)dbits[j][i]), dot_q8(wq[j][i], xc), acc[j]);
                    acc[j] = c < nchunk ? t : acc[j];
                }
            }
        } else if constexpr (WT == LK_Q8_SM) {
            uint2 sm[NR][NCH];
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const uint32_t c = base + (uint32_t)lane + 64u * i;
#pragma unroll
                for (int j = 0; j < NR; j++) sm[j][i] = ld_sm(ap[j], c < nchunk ? c : 0u);
            }
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const uint32_t c = base + (uint32_t)lane + 64u * i;
                const float* xc = XREG ? xr[XREG ? i : 0] : x + (size_t)(c < nchunk ? c : 0u) * 16;
#pragma unroll
                for (int j = 0; j < NR; j++) {
                    const float t = dot_q8sm(wq[j][i], sm[j][i], xc);
                    acc[j] += c < nchunk ? t : 0.f;
                }
            }
        } else if constexpr (WT == LK_F16) {
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const uint32_t c = base + (uint32_t)lane + 64u * i;
                const float* xc = XREG ? xr[XREG ? i : 0] : x + (size_t)(c < nchunk ? c : 0u) * 8;
#pragma unroll
                for (int j = 0; j < NR; j++) {
                    const float t = dot_f16(wq[j][i], xc);
                    acc[j] += c < nchunk ? t : 0.f;
                }
            }
        } else {  // Q4_K
            uint4 hd[NR][NCH];
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const uint32_t c = base + (uint32_t)lane + 64u * i;
#pragma unroll
                for (int j = 0; j < NR; j++) {
                    const lk_u32x4 hv = *lk_g((const lk_u32x4*)(ap[j] + 16u * ((c < nchunk ? c : 0u) >> 3)));
                    hd[j][i] = make_uint4(hv.x, hv.y, hv.z, hv.w);
                }
            }
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const uint32_t c = base + (uint32_t)lane + 64u * i;
                const uint32_t cc = c < nchunk ? c : 0u;
                const uint32_t sb = cc >> 3, k = cc & 7;
                const float* xc = x + (size_t)sb * 256 + (k >> 1) * 64 + (k & 1) * 16;
#pragma unroll
                for (int j = 0; j < NR; j++) {
                    const float t = dot_q4k(wq[j][i], hd[j][i], k, xc);
                    acc[j] += c < nchunk ? t : 0.f;
                }
            }
        }
    }

#pragma unroll
    for (int j = 0; j < NR; j++) acc[j] = lk_wave_sum(acc[j]);

    if constexpr (MODE == LK_MV_SWIGLU) {
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < R; j++) {
                if (rv[j]) {
                    const float g = acc[j], u = acc[R + j];
                    a.seg[0].out[rr[j]] = g / (1.0f + expf(-g)) * u;
                }
            }
        }
    } else if constexpr (MODE == LK_MV_ARGMAX) {
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < R; j++) {
                if (rv[j]) {
                    const float v = acc[j];
                    a.seg[0].out[rr[j]] = v;
                    const uint64_t kk = lk_argmax_key(v, rr[j]);
                    key = kk > key ? kk : key;
                }
            }
        }
    } else {
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < NR; j++) {
                if (rv[j]) {
                    const LkSeg& s = a.seg[rs[j]];
                    float v = acc[j];
                    if (s.bias) v += s.bias[rr[j]];
                    if constexpr (MODE == LK_MV_ACC) s.out[rr[j]] += v;
                    else s.out[rr[j]] = v;
                }
            }
        }
    }
    }  // row groups
    if constexpr (MODE == LK_MV_ARGMAX) {
        __shared__ uint64_t best[4];
        if (lane == 0) best[threadIdx.x >> 6] = key;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t k = best[0];
            for (int w = 1; w < 4; w++) k = best[w] > k ? best[w] : k;
            a.keys[blockIdx.x] = k;
        }
    }
}

template <int WT, int NCH, int R, int MODE>
hipError_t launch_one(const LkMvArgs& a, unsigned blocks, hipStream_t st) {
    hipLaunchKernelGGL((matvec_kernel<WT, NCH, R, MODE>), dim3(blocks), dim3(256), 0, st, a);
    return hipGetLastError();
}

template <int WT, int NCH>
hipError_t launch_r(const LkMvArgs& a, int mode, int R, unsigned blocks, hipStream_t st) {
    switch (mode) {
    case LK_MV_STORE:
        if (R == 1) return launch_one<WT, NCH, 1, LK_MV_STORE>(a, blocks, st);
        if (R == 2) return launch_one<WT, NCH, 2, LK_MV_STORE>(a, blocks, st);
        return launch_one<WT, NCH, 4, LK_MV_STORE>(a, blocks, st);
    case LK_MV_ACC:
        if (R == 1) return launch_one<WT, NCH, 1, LK_MV_ACC>(a, blocks, st);
        if (R == 2) return launch_one<WT, NCH, 2, LK_MV_ACC>(a, blocks, st);
        return launch_one<WT, NCH, 4, LK_MV_ACC>(a, blocks, st);
    case LK_MV_SWIGLU:
        if (R == 1) return launch_one<WT, NCH, 1, LK_MV_SWIGLU>(a, blocks, st);
        return launch_one<WT, NCH, 2, LK_MV_SWIGLU>(a, blocks, st);
    case LK_MV_ARGMAX:
        return launch_one<WT, NCH, 4, LK_MV_ARGMAX>(a, blocks, st);
    }
    return hipErrorInvalidValue;
}

template <int WT>
hipError_t launch_type(const LkMvArgs& a, int mode, int R, int nch, unsigned blocks, hipStream_t st) {
    switch (nch) {
    case 1: return launch_r<WT, 1>(a, mode, R, blocks, st);
    case 2: return launch_r<WT, 2>(a, mode, R, blocks, st);
    case 3: return launch_r<WT, 3>(a, mode, R, blocks, st);
    case 4: return launch_r<WT, 4>(a, mode, R, blocks, st);
    case 5: return launch_r<WT, 5>(a, mode, R, blocks, st);
    case 6: return launch_r<WT, 6>(a, mode, R, blocks, st);
    default: return launch_r<WT, 8>(a, mode, R, blocks, st);
    }
}

}  // namespace lk

hipError_t lk_matvec_launch_q8_0(const LkMvArgs& a, int mode, int R, int nch, unsigned blocks, hipStream_t st);
hipError_t lk_matvec_launch_f16(const LkMvArgs& a, int mode, int R, int nch, unsigned blocks, hipStream_t st);
hipError_t lk_matvec_launch_q4_k(const LkMvArgs& a, int mode, int R, int nch, unsigned blocks, hipStream_t st);
hipError_t lk_matvec_launch_q8_sm(const LkMvArgs& a, int mode, int R, int nch, unsigned blocks, hipStream_t st);
