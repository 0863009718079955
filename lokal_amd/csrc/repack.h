// repack.h -- host-side repacking of GGUF weight rows into the device layouts
// (lkhip_common.h, LkDevW).  Values are unchanged: every device element
// dequantizes to the f32 that dequant_row_ref (src/gguf/dequant.rs:191-535)
// produces for the same GGUF element.
//
//   GGUF type   device type   how
//   F32, F16    same          copied
//   Q8_0        Q8_0          scale split from the 32 int8 values
//   Q4_0, Q5_0  Q8_0          q - 8 / q - 16 stored as int8 beside the same f16 d:
//                             (q-8)*d is the one product both forms compute
//   Q4_K        Q4_K          the 16-byte head split from the 128 nibble bytes
//   Q5_K, Q6_K  Q8_SM         int8 q per element, (s, m) f32 per 16 elements
//
// Plain C++ (no HIP): the engine links it, and a CPU build can check it.
#pragma once
#include <stdint.h>
#include <string.h>

namespace lkr {

enum : uint32_t { G_F32 = 0, G_F16 = 1, G_Q4_0 = 2, G_Q5_0 = 6, G_Q8_0 = 8, G_Q4_K = 12, G_Q5_K = 13, G_Q6_K = 14 };
enum : uint32_t { D_Q8_SM = 64 };

// IEEE half -> float, exact (half::f16::to_f32, src/gguf/dequant.rs:135-137).
inline float h2f(uint16_t hbits) {
    uint32_t sign = (uint32_t)(hbits >> 15) << 31, e = (hbits >> 10) & 31, m = hbits & 1023, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int k = -1;
            do {
                m <<= 1;
                k++;
            } while (!(m & 1024));
            bits = sign | ((uint32_t)(112 - k) << 23) | ((m & 1023) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
inline uint16_t u16_at(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// GGUF block geometry (src/gguf/dequant.rs:21-40 type ids; block sizes of
// the dequant arms).  0 for a type the backend does not take.
inline size_t blk_elems(uint32_t t) {
    switch (t) {
    case G_F32: case G_F16: return 1;
    case G_Q4_0: case G_Q5_0: case G_Q8_0: return 32;
    case G_Q4_K: case G_Q5_K: case G_Q6_K: return 256;
    default: return 0;
    }
}
inline size_t blk_bytes(uint32_t t) {
    switch (t) {
    case G_F32: return 4;
    case G_F16: return 2;
    case G_Q4_0: return 18;
    case G_Q5_0: return 22;
    case G_Q8_0: return 34;
    case G_Q4_K: return 144;
    case G_Q5_K: return 176;
    case G_Q6_K: return 210;
    default: return 0;
    }
}

// The device type a GGUF type is stored as.
inline uint32_t device_type(uint32_t t) {
    switch (t) {
    case G_Q4_0: case G_Q5_0: return G_Q8_0;
    case G_Q5_K: case G_Q6_K: return D_Q8_SM;
    default: return t;
    }
}
// Device bytes per row: data and aux (block scales / heads).
inline size_t data_row_bytes(uint32_t dev, size_t cols) {
    switch (dev) {
    case G_F32: return cols * 4;
    case G_F16: return cols * 2;
    case G_Q4_K: return cols / 256 * 128;
    default: return cols;  // Q8_0, Q8_SM: one int8 per element
    }
}
inline size_t aux_row_bytes(uint32_t dev, size_t cols) {
    switch (dev) {
    case G_Q8_0: return cols / 32 * 2;
    case G_Q4_K: return cols / 256 * 16;
    case D_Q8_SM: return cols / 16 * 8;
    default: return 0;
    }
}

// scale_min_k4, src/gguf/dequant.rs:141-150.
inline void scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

// One GGUF row (cols elements, src) into device data d and aux a.
inline void repack_row(uint32_t t, const uint8_t* s, size_t cols, uint8_t* d, uint8_t* a) {
    switch (t) {
    case G_F32: memcpy(d, s, cols * 4); break;
    case G_F16: memcpy(d, s, cols * 2); break;
    case G_Q8_0:
        for (size_t b = 0; b < cols / 32; b++) {
            memcpy(a + 2 * b, s + 34 * b, 2);
            memcpy(d + 32 * b, s + 34 * b + 2, 32);
        }
        break;
    case G_Q4_0:  // :203-214  y[j] = ((q & 15) - 8) * d, y[j+16] = ((q >> 4) - 8) * d
        for (size_t b = 0; b < cols / 32; b++) {
            const uint8_t* blk = s + 18 * b;
            memcpy(a + 2 * b, blk, 2);
            int8_t* q = (int8_t*)(d + 32 * b);
            for (int j = 0; j < 16; j++) {
                q[j] = (int8_t)((blk[2 + j] & 0x0F) - 8);
                q[j + 16] = (int8_t)((blk[2 + j] >> 4) - 8);
            }
        }
        break;
    case G_Q5_0:  // :215-230  the fifth bit of element j is bit j of qh
        for (size_t b = 0; b < cols / 32; b++) {
            const uint8_t* blk = s + 22 * b;
            memcpy(a + 2 * b, blk, 2);
            const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                                ((uint32_t)blk[5] << 24);
            int8_t* q = (int8_t*)(d + 32 * b);
            for (int j = 0; j < 16; j++) {
                const int lo = (blk[6 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4);
                const int hi = (blk[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
                q[j] = (int8_t)(lo - 16);
                q[j + 16] = (int8_t)(hi - 16);
            }
        }
        break;
    case G_Q4_K:
        for (size_t b = 0; b < cols / 256; b++) {
            memcpy(a + 16 * b, s + 144 * b, 16);
            memcpy(d + 128 * b, s + 144 * b + 16, 128);
        }
        break;
    case G_Q5_K:  // :484-509  element e: sub-block g = e/32, q = nibble + 16 * bit g of qh[e % 32]
        for (size_t b = 0; b < cols / 256; b++) {
            const uint8_t* blk = s + 176 * b;
            const float dd = h2f(u16_at(blk)), dmin = h2f(u16_at(blk + 2));
            const uint8_t* scales = blk + 4;
            const uint8_t* qh = blk + 16;
            const uint8_t* qs = blk + 48;
            int8_t* q = (int8_t*)(d + 256 * b);
            float* sm = (float*)(a + 256 / 16 * 8 * b);
            for (int g = 0; g < 8; g++) {
                uint8_t sc, m;
                scale_min_k4(g, scales, &sc, &m);
                const float d1 = dd * (float)sc, m1 = dmin * (float)m;  // exact: f16 x 6-bit
                for (int h = 0; h < 2; h++) {
                    sm[2 * (2 * g + h)] = d1;
                    sm[2 * (2 * g + h) + 1] = m1;
                }
                for (int l = 0; l < 32; l++) {
                    const uint8_t byte = qs[32 * (g / 2) + l];
                    const int nib = (g & 1) ? (byte >> 4) : (byte & 0x0F);
                    q[32 * g + l] = (int8_t)(nib + (((qh[l] >> g) & 1) ? 16 : 0));
                }
            }
        }
        break;
    case G_Q6_K:  // :510-533  element e of a 128-half: scale sc[e/16], q from ql/qh
        for (size_t b = 0; b < cols / 256; b++) {
            const uint8_t* blk = s + 210 * b;
            const float dd = h2f(u16_at(blk + 208));
            int8_t* q = (int8_t*)(d + 256 * b);
            float* sm = (float*)(a + 256 / 16 * 8 * b);
            for (int g = 0; g < 16; g++) {
                sm[2 * g] = dd * (float)(int8_t)blk[192 + g];  // exact: f16 x int8
                sm[2 * g + 1] = 0.f;
            }
            for (int n = 0; n < 256; n += 128) {
                const uint8_t* ql = blk + n / 2;
                const uint8_t* qh = blk + 128 + n / 4;
                for (int l = 0; l < 32; l++) {
                    q[n + l] = (int8_t)(((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32);
                    q[n + l + 32] = (int8_t)(((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32);
                    q[n + l + 64] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                    q[n + l + 96] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                }
            }
        }
        break;
    }
}

}  // namespace lkr
