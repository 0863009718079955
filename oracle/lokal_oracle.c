/*
 * lokal_oracle.c -- CPU restatement of lokal's reference decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * backend in lokal_amd/.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path never does.
 *
 * It restates, function by function, the Rust CPU path of AssetsArt/lokal:
 *   src/math.rs            dot / matvec / rmsnorm / softmax / silu
 *   src/model.rs           Model::forward, rope, attention, KvCache
 *   src/gguf/dequant.rs    f16_bits_at, scale_min_k4, dequant_row_ref arms
 *   src/gguf/arch.rs       unpermute_llama_qk
 *   src/sampler.rs         argmax (first max wins)
 * Each function cites the file:line it follows.  Arithmetic order is kept
 * exactly (Rust never contracts a*b+c into an FMA, so this file is built with
 * -ffp-contract=off), and libm is glibc's expf/powf/sinf/cosf/sqrtf, which is
 * what a Linux build of the Rust would call.
 *
 * Pinning (see tests/test_oracle.py): every hand vector of the reference's
 * dequant.rs / math.rs / sampler.rs / arch.rs tests, closed forms in f64,
 * exhaustive scale_min_k4, and invariants of rope/attention.  The libm
 * boundary (expf/powf/sinf/cosf against Apple libm) is "parity unpinned": no
 * reference test fixes those bits.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_API __attribute__((visibility("default")))

/* ggml type ids, src/gguf/dequant.rs:21-40 */
enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14 };

/* ------------------------------------------------------------------ f16 */

/* half::f16::to_f32 is exact; src/gguf/dequant.rs:135-137 (f16_bits_at). */
ORACLE_API float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400));
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* f32 -> f16 bits, round to nearest even (what half::f16::from_f32 and the
 * GPU's v_cvt_f16_f32 compute), with subnormals, overflow to inf and NaN. */
ORACLE_API uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds past 65504 */
    if (ax < 0x38800000u) {                                    /* f16 subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;           /* below half the smallest subnormal */
        uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e; /* value = m * 2^(e-150); target unit 2^-24 */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112, m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13), rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

static float f16_at(const uint8_t* p) { return oracle_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ------------------------------------------------------------- dequant */

/* GgmlType::blk_elems / blk_bytes, src/gguf/dequant.rs:83-120 */
ORACLE_API int oracle_blk_elems(uint32_t t) {
    switch (t) {
    case T_F32: case T_F16: return 1;
    case T_Q4_0: case T_Q5_0: case T_Q8_0: return 32;
    case T_Q4_K: case T_Q5_K: case T_Q6_K: return 256;
    default: return 0;
    }
}
ORACLE_API int oracle_blk_bytes(uint32_t t) {
    switch (t) {
    case T_F32: return 4;
    case T_F16: return 2;
    case T_Q4_0: return 18;
    case T_Q5_0: return 22;
    case T_Q8_0: return 34;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    default: return 0;
    }
}
/* GgmlType::row_bytes, src/gguf/dequant.rs:117-120 */
ORACLE_API size_t oracle_row_bytes(uint32_t t, size_t n) {
    int e = oracle_blk_elems(t);
    return e ? n / (size_t)e * (size_t)oracle_blk_bytes(t) : 0;
}

/* scale_min_k4, src/gguf/dequant.rs:141-150 */
ORACLE_API void oracle_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* dequant_row_ref, src/gguf/dequant.rs:191-535 (F32, F16, Q4_0, Q5_0, Q8_0,
 * Q4_K, Q5_K, Q6_K arms).  Returns 0, or -1 on a size mismatch or an
 * unsupported type (the Rust asserts / refuses; here the caller sees -1). */
ORACLE_API int oracle_dequant_row(uint32_t t, const uint8_t* src, size_t nbytes, float* y, size_t n) {
    if (oracle_blk_elems(t) == 0 || n % (size_t)oracle_blk_elems(t) != 0) return -1;
    if (nbytes != oracle_row_bytes(t, n)) return -1;
    switch (t) {
    case T_F32:
        for (size_t i = 0; i < n; i++) memcpy(&y[i], src + 4 * i, 4);
        break;
    case T_F16:
        for (size_t i = 0; i < n; i++) y[i] = f16_at(src + 2 * i);
        break;
    case T_Q4_0: /* :203-214 */
        for (size_t b = 0; b < n / 32; b++) {
            const uint8_t* blk = src + b * 18;
            float d = f16_at(blk);
            for (int j = 0; j < 16; j++) {
                uint8_t q = blk[2 + j];
                y[b * 32 + j] = (float)((int)(q & 0x0F) - 8) * d;
                y[b * 32 + j + 16] = (float)((int)(q >> 4) - 8) * d;
            }
        }
        break;
    case T_Q5_0: /* :215-230 */
        for (size_t b = 0; b < n / 32; b++) {
            const uint8_t* blk = src + b * 22;
            float d = f16_at(blk);
            uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
            for (int j = 0; j < 16; j++) {
                uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10);
                uint8_t xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
                uint8_t q = blk[6 + j];
                y[b * 32 + j] = (float)((int)((q & 0x0F) | xh0) - 16) * d;
                y[b * 32 + j + 16] = (float)((int)((q >> 4) | xh1) - 16) * d;
            }
        }
        break;
    case T_Q8_0: /* :231-239 -- (i8)q * d, exact in f32 */
        for (size_t b = 0; b < n / 32; b++) {
            const uint8_t* blk = src + b * 34;
            float d = f16_at(blk);
            for (int j = 0; j < 32; j++) y[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
        }
        break;
    case T_Q4_K: /* :462-483 -- d1 = d*sc, m1 = dmin*m rounded first, then d1*q - m1 */
        for (size_t b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + b * 144;
            float d = f16_at(blk), dmin = f16_at(blk + 2);
            const uint8_t* scales = blk + 4;
            const uint8_t* qs = blk + 16;
            float* yb = y + b * 256;
            int is = 0;
            for (int j = 0; j < 256; j += 64) {
                const uint8_t* q = qs + j / 2;
                uint8_t sc, m;
                oracle_scale_min_k4(is, scales, &sc, &m);
                float d1 = d * (float)sc, m1 = dmin * (float)m;
                oracle_scale_min_k4(is + 1, scales, &sc, &m);
                float d2 = d * (float)sc, m2 = dmin * (float)m;
                for (int l = 0; l < 32; l++) {
                    yb[j + l] = d1 * (float)(q[l] & 0x0F) - m1;
                    yb[j + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
                }
                is += 2;
            }
        }
        break;
    case T_Q5_K: /* :484-509 */
        for (size_t b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + b * 176;
            float d = f16_at(blk), dmin = f16_at(blk + 2);
            const uint8_t* scales = blk + 4;
            const uint8_t* qh = blk + 16;
            const uint8_t* qs = blk + 48;
            float* yb = y + b * 256;
            int is = 0;
            uint8_t u1 = 1, u2 = 2;
            for (int j = 0; j < 256; j += 64) {
                const uint8_t* ql = qs + j / 2;
                uint8_t sc, m;
                oracle_scale_min_k4(is, scales, &sc, &m);
                float d1 = d * (float)sc, m1 = dmin * (float)m;
                oracle_scale_min_k4(is + 1, scales, &sc, &m);
                float d2 = d * (float)sc, m2 = dmin * (float)m;
                for (int l = 0; l < 32; l++) {
                    int hi1 = (qh[l] & u1) ? 16 : 0;
                    int hi2 = (qh[l] & u2) ? 16 : 0;
                    yb[j + l] = d1 * (float)((ql[l] & 0x0F) + hi1) - m1;
                    yb[j + 32 + l] = d2 * (float)((ql[l] >> 4) + hi2) - m2;
                }
                is += 2;
                u1 = (uint8_t)(u1 << 2);
                u2 = (uint8_t)(u2 << 2);
            }
        }
        break;
    case T_Q6_K: /* :510-533 -- d * sc first, then * q */
        for (size_t b = 0; b < n / 256; b++) {
            const uint8_t* blk = src + b * 210;
            float d = f16_at(blk + 208);
            float* yb = y + b * 256;
            for (int nn = 0; nn < 256; nn += 128) {
                const uint8_t* ql = blk + nn / 2;
                const uint8_t* qh = blk + 128 + nn / 4;
                const int8_t* sc = (const int8_t*)(blk + 192 + nn / 16);
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = (int8_t)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    int q2 = (int8_t)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = (int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    yb[nn + l] = d * (float)sc[is] * (float)q1;
                    yb[nn + l + 32] = d * (float)sc[is + 2] * (float)q2;
                    yb[nn + l + 64] = d * (float)sc[is + 4] * (float)q3;
                    yb[nn + l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
        }
        break;
    default:
        return -1;
    }
    return 0;
}

/* unpermute_llama_qk, src/gguf/arch.rs:274-286 */
ORACLE_API void oracle_unpermute_llama_qk(float* data, size_t rows, size_t cols, size_t head_dim) {
    float* out = (float*)malloc(rows * cols * sizeof(float));
    for (size_t h = 0; h < rows / head_dim; h++)
        for (size_t j = 0; j < head_dim; j++) {
            size_t a = j / (head_dim / 2), d = j % (head_dim / 2);
            size_t src = h * head_dim + d * 2 + a;
            memcpy(out + (h * head_dim + j) * cols, data + src * cols, cols * sizeof(float));
        }
    memcpy(data, out, rows * cols * sizeof(float));
    free(out);
}

/* ---------------------------------------------------------------- math */

/* math::dot, src/math.rs:25-38: 8 independent lanes, lanes summed 0..7, then
 * the tail added one by one. */
ORACLE_API float oracle_dot(const float* a, const float* b, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t chunks = n / 8;
    for (size_t c = 0; c < chunks; c++)
        for (int i = 0; i < 8; i++) acc[i] += a[c * 8 + i] * b[c * 8 + i];
    float sum = -0.0f; /* core::iter::Sum for f32 folds from -0.0 */
    for (int i = 0; i < 8; i++) sum += acc[i];
    for (size_t i = chunks * 8; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* math::matvec, src/math.rs:10-18: rows in parallel, each row one dot. */
ORACLE_API void oracle_matvec(const float* w, const float* x, size_t out_dim, size_t in_dim, float* y) {
#pragma omp parallel for schedule(static)
    for (long o = 0; o < (long)out_dim; o++) y[o] = oracle_dot(w + (size_t)o * in_dim, x, in_dim);
}

/* math::rmsnorm, src/math.rs:45-49 */
ORACLE_API void oracle_rmsnorm(const float* x, const float* w, size_t n, float eps, float* y) {
    float mean_sq = oracle_dot(x, x, n) / (float)n;
    float scale = 1.0f / sqrtf(mean_sq + eps);
    for (size_t i = 0; i < n; i++) y[i] = x[i] * scale * w[i];
}

/* math::softmax, src/math.rs:55-66 */
ORACLE_API void oracle_softmax(float* x, size_t n) {
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    for (size_t i = 0; i < n; i++) x[i] /= sum;
}

/* math::silu, src/math.rs:68-70 */
ORACLE_API float oracle_silu(float x) { return x / (1.0f + expf(-x)); }

/* SwiGLU inner product of Model::forward, src/model.rs:247-249 */
ORACLE_API void oracle_swiglu(const float* g, const float* u, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_silu(g[i]) * u[i];
}

/* model::rope, src/model.rs:268-279: pair (i, i+hd/2) of every head rotated by
 * pos * theta^(-2i/hd). */
ORACLE_API void oracle_rope(float* x, size_t n, size_t pos, size_t head_dim, float theta) {
    size_t half = head_dim / 2;
    for (size_t h = 0; h + head_dim <= n; h += head_dim) {
        float* head = x + h;
        for (size_t i = 0; i < half; i++) {
            float freq = powf(theta, -(2.0f * (float)i) / (float)head_dim);
            float ang = (float)pos * freq;
            float s = sinf(ang), c = cosf(ang);
            float a = head[i], b = head[i + half];
            head[i] = a * c - b * s;
            head[i + half] = a * s + b * c;
        }
    }
}

/* model::attention, src/model.rs:286-318.  k_cache / v_cache are
 * [max_seq][kvd]; positions 0..=pos are live. */
ORACLE_API void oracle_attention(const float* q, const float* k_cache, const float* v_cache, size_t pos,
                                 size_t n_heads, size_t n_kv_heads, size_t hd, size_t kvd, float* out) {
    size_t group = n_heads / n_kv_heads;
    float scale = 1.0f / sqrtf((float)hd);
    float* scores = (float*)malloc((pos + 1) * sizeof(float));
    memset(out, 0, n_heads * hd * sizeof(float));
    for (size_t h = 0; h < n_heads; h++) {
        const float* qh = q + h * hd;
        size_t kv_off = (h / group) * hd;
        for (size_t t = 0; t <= pos; t++) scores[t] = oracle_dot(qh, k_cache + t * kvd + kv_off, hd) * scale;
        oracle_softmax(scores, pos + 1);
        float* o = out + h * hd;
        for (size_t t = 0; t <= pos; t++) {
            const float* vt = v_cache + t * kvd + kv_off;
            float s = scores[t];
            for (size_t i = 0; i < hd; i++) o[i] += s * vt[i];
        }
    }
    free(scores);
}

/* sampler::argmax, src/sampler.rs:67-75: first index of the maximum. */
ORACLE_API uint32_t oracle_argmax(const float* x, size_t n) {
    size_t best = 0;
    for (size_t i = 0; i < n; i++)
        if (x[i] > x[best]) best = i;
    return (uint32_t)best;
}

ORACLE_API void oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
ORACLE_API int oracle_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* --------------------------------------------------------------- model */

/* ModelConfig fields used by Model::forward, src/config.rs:10-30 */
typedef struct {
    uint32_t hidden, intermediate, n_layers, n_heads, n_kv_heads, vocab;
    uint32_t head_dim; /* 0 = hidden / n_heads (ModelConfig::head_dim) */
    float rms_eps, rope_theta;
} oracle_config;

typedef struct {
    float* w;
    float* bias;
    size_t in_dim, out_dim;
} lin_t; /* model::Linear, src/model.rs:19-24 */

typedef struct {
    float *in_norm, *post_norm;
    lin_t q, k, v, o, gate, up, down;
} block_t; /* model::Block, src/model.rs:68-78 */

typedef struct oracle_model {
    oracle_config cfg;
    size_t hd, q_dim, kv_dim;
    float* embed;
    float* norm;
    lin_t lm_head;
    block_t* blocks;
    int tied;
} oracle_model;

typedef struct oracle_session {
    const oracle_model* m;
    size_t max_seq;
    uint32_t n_layers; /* kept so the session can be freed after its model */
    int kv_f16;        /* store K/V rounded through f16, as the GPU cache does */
    float** k; /* per layer [max_seq * kv_dim], model::KvCache src/model.rs:114-128 */
    float** v;
    float *x, *xn, *q, *kk, *vv, *att, *ao, *gate, *up, *inner, *down;
} oracle_session;

ORACLE_API oracle_model* oracle_model_new(const oracle_config* cfg) {
    oracle_model* m = (oracle_model*)calloc(1, sizeof(oracle_model));
    m->cfg = *cfg;
    m->hd = cfg->head_dim ? cfg->head_dim : cfg->hidden / cfg->n_heads;
    m->q_dim = cfg->n_heads * m->hd;
    m->kv_dim = cfg->n_kv_heads * m->hd;
    m->blocks = (block_t*)calloc(cfg->n_layers, sizeof(block_t));
    return m;
}

static int set_lin(lin_t* l, const float* w, size_t rows, size_t cols) {
    l->w = (float*)malloc(rows * cols * sizeof(float));
    memcpy(l->w, w, rows * cols * sizeof(float));
    l->out_dim = rows;
    l->in_dim = cols;
    return 0;
}
static float* dup(const float* w, size_t n) {
    float* p = (float*)malloc(n * sizeof(float));
    memcpy(p, w, n * sizeof(float));
    return p;
}

/* Model::from_store's wiring (src/model.rs:140-193), fed one dequantized f32
 * tensor at a time under its HF name. */
ORACLE_API int oracle_model_set_f32(oracle_model* m, const char* name, const float* w, size_t rows, size_t cols) {
    int layer = -1;
    char rest[128];
    if (sscanf(name, "model.layers.%d.%127s", &layer, rest) == 2) {
        if (layer < 0 || (uint32_t)layer >= m->cfg.n_layers) return -1;
        block_t* b = &m->blocks[layer];
        size_t n = rows * cols;
        if (!strcmp(rest, "input_layernorm.weight")) b->in_norm = dup(w, n);
        else if (!strcmp(rest, "post_attention_layernorm.weight")) b->post_norm = dup(w, n);
        else if (!strcmp(rest, "self_attn.q_proj.weight")) set_lin(&b->q, w, rows, cols);
        else if (!strcmp(rest, "self_attn.k_proj.weight")) set_lin(&b->k, w, rows, cols);
        else if (!strcmp(rest, "self_attn.v_proj.weight")) set_lin(&b->v, w, rows, cols);
        else if (!strcmp(rest, "self_attn.o_proj.weight")) set_lin(&b->o, w, rows, cols);
        else if (!strcmp(rest, "self_attn.q_proj.bias")) b->q.bias = dup(w, n);
        else if (!strcmp(rest, "self_attn.k_proj.bias")) b->k.bias = dup(w, n);
        else if (!strcmp(rest, "self_attn.v_proj.bias")) b->v.bias = dup(w, n);
        else if (!strcmp(rest, "mlp.gate_proj.weight")) set_lin(&b->gate, w, rows, cols);
        else if (!strcmp(rest, "mlp.up_proj.weight")) set_lin(&b->up, w, rows, cols);
        else if (!strcmp(rest, "mlp.down_proj.weight")) set_lin(&b->down, w, rows, cols);
        else return -1;
        return 0;
    }
    if (!strcmp(name, "model.embed_tokens.weight")) m->embed = dup(w, rows * cols);
    else if (!strcmp(name, "model.norm.weight")) m->norm = dup(w, rows * cols);
    else if (!strcmp(name, "lm_head.weight")) set_lin(&m->lm_head, w, rows, cols);
    else return -1;
    return 0;
}

/* Same, from raw GGUF-layout bytes: dequant_row_ref on the whole tensor, as
 * load_f32 does (src/gguf/dequant.rs:539-557), then the llama q/k unpermute
 * when asked (:548-553). */
ORACLE_API int oracle_model_set(oracle_model* m, const char* name, uint32_t type, const uint8_t* data, size_t nbytes,
                                size_t rows, size_t cols, int unpermute) {
    float* tmp = (float*)malloc(rows * cols * sizeof(float));
    if (!tmp) return -1;
    int rc = oracle_dequant_row(type, data, nbytes, tmp, rows * cols);
    if (rc == 0 && unpermute) oracle_unpermute_llama_qk(tmp, rows, cols, m->hd);
    if (rc == 0) rc = oracle_model_set_f32(m, name, tmp, rows, cols);
    free(tmp);
    return rc;
}

/* Checks every tensor is present; ties lm_head to the embedding when absent
 * (src/model.rs:181-186). */
ORACLE_API int oracle_model_finalize(oracle_model* m) {
    const oracle_config* c = &m->cfg;
    if (!m->embed || !m->norm) return -1;
    for (uint32_t i = 0; i < c->n_layers; i++) {
        block_t* b = &m->blocks[i];
        if (!b->in_norm || !b->post_norm || !b->q.w || !b->k.w || !b->v.w || !b->o.w || !b->gate.w || !b->up.w ||
            !b->down.w)
            return -1 - (int)i;
    }
    if (!m->lm_head.w) {
        m->lm_head.w = m->embed;
        m->lm_head.in_dim = c->hidden;
        m->lm_head.out_dim = c->vocab;
        m->tied = 1;
    }
    return 0;
}

static void free_lin(lin_t* l) {
    free(l->w);
    free(l->bias);
}
ORACLE_API void oracle_model_free(oracle_model* m) {
    if (!m) return;
    for (uint32_t i = 0; i < m->cfg.n_layers; i++) {
        block_t* b = &m->blocks[i];
        free(b->in_norm);
        free(b->post_norm);
        free_lin(&b->q); free_lin(&b->k); free_lin(&b->v); free_lin(&b->o);
        free_lin(&b->gate); free_lin(&b->up); free_lin(&b->down);
    }
    free(m->blocks);
    if (!m->tied) free(m->lm_head.w);
    free(m->embed);
    free(m->norm);
    free(m);
}

ORACLE_API oracle_session* oracle_session_new(const oracle_model* m, size_t max_seq) {
    oracle_session* s = (oracle_session*)calloc(1, sizeof(oracle_session));
    const oracle_config* c = &m->cfg;
    s->m = m;
    s->max_seq = max_seq;
    s->n_layers = c->n_layers;
    s->k = (float**)calloc(c->n_layers, sizeof(float*));
    s->v = (float**)calloc(c->n_layers, sizeof(float*));
    for (uint32_t i = 0; i < c->n_layers; i++) {
        s->k[i] = (float*)calloc(max_seq * m->kv_dim, sizeof(float));
        s->v[i] = (float*)calloc(max_seq * m->kv_dim, sizeof(float));
    }
    s->x = (float*)calloc(c->hidden, 4);
    s->xn = (float*)calloc(c->hidden, 4);
    s->q = (float*)calloc(m->q_dim, 4);
    s->kk = (float*)calloc(m->kv_dim, 4);
    s->vv = (float*)calloc(m->kv_dim, 4);
    s->att = (float*)calloc(m->q_dim, 4);
    s->ao = (float*)calloc(c->hidden, 4);
    s->gate = (float*)calloc(c->intermediate, 4);
    s->up = (float*)calloc(c->intermediate, 4);
    s->inner = (float*)calloc(c->intermediate, 4);
    s->down = (float*)calloc(c->hidden, 4);
    return s;
}

ORACLE_API void oracle_session_free(oracle_session* s) {
    if (!s) return;
    for (uint32_t i = 0; i < s->n_layers; i++) {
        free(s->k[i]);
        free(s->v[i]);
    }
    free(s->k); free(s->v);
    free(s->x); free(s->xn); free(s->q); free(s->kk); free(s->vv); free(s->att); free(s->ao);
    free(s->gate); free(s->up); free(s->inner); free(s->down);
    free(s);
}

/* Linear::forward, src/model.rs:27-35 */
static void lin_fwd(const lin_t* l, const float* x, float* y) {
    oracle_matvec(l->w, x, l->out_dim, l->in_dim, y);
    if (l->bias)
        for (size_t i = 0; i < l->out_dim; i++) y[i] += l->bias[i];
}

/* Model::forward, src/model.rs:196-262.  Writes vocab logits. */
ORACLE_API int oracle_forward(oracle_session* s, uint32_t token, size_t pos, float* logits) {
    const oracle_model* m = s->m;
    const oracle_config* c = &m->cfg;
    size_t h = c->hidden;
    if (token >= c->vocab || pos >= s->max_seq) return -1;
    memcpy(s->x, m->embed + (size_t)token * h, h * sizeof(float));
    for (uint32_t layer = 0; layer < c->n_layers; layer++) {
        const block_t* b = &m->blocks[layer];
        oracle_rmsnorm(s->x, b->in_norm, h, c->rms_eps, s->xn);
        lin_fwd(&b->q, s->xn, s->q);
        lin_fwd(&b->k, s->xn, s->kk);
        lin_fwd(&b->v, s->xn, s->vv);
        oracle_rope(s->q, m->q_dim, pos, m->hd, c->rope_theta);
        oracle_rope(s->kk, m->kv_dim, pos, m->hd, c->rope_theta);
        if (s->kv_f16) {
            for (size_t i = 0; i < m->kv_dim; i++) {
                s->kk[i] = oracle_f16_to_f32(oracle_f32_to_f16(s->kk[i]));
                s->vv[i] = oracle_f16_to_f32(oracle_f32_to_f16(s->vv[i]));
            }
        }
        memcpy(s->k[layer] + pos * m->kv_dim, s->kk, m->kv_dim * 4);
        memcpy(s->v[layer] + pos * m->kv_dim, s->vv, m->kv_dim * 4);
        oracle_attention(s->q, s->k[layer], s->v[layer], pos, c->n_heads, c->n_kv_heads, m->hd, m->kv_dim, s->att);
        lin_fwd(&b->o, s->att, s->ao);
        for (size_t i = 0; i < h; i++) s->x[i] += s->ao[i];
        oracle_rmsnorm(s->x, b->post_norm, h, c->rms_eps, s->xn);
        lin_fwd(&b->gate, s->xn, s->gate);
        lin_fwd(&b->up, s->xn, s->up);
        oracle_swiglu(s->gate, s->up, c->intermediate, s->inner);
        lin_fwd(&b->down, s->inner, s->down);
        for (size_t i = 0; i < h; i++) s->x[i] += s->down[i];
    }
    oracle_rmsnorm(s->x, m->norm, h, c->rms_eps, s->xn);
    lin_fwd(&m->lm_head, s->xn, logits);
    return 0;
}

/* Test-only variant: keep the KV cache in f16 precision (values rounded
 * through f16 on store), the storage format of lokal's GPU path
 * (src/gpu/metal.rs:3234-3235).  Off by default: the CPU path is f32. */
ORACLE_API void oracle_session_set_kv_f16(oracle_session* s, int on) { s->kv_f16 = on; }

/* The hidden state after the last block and before the final norm; lets a
 * test compare intermediate state. */
ORACLE_API void oracle_session_hidden(const oracle_session* s, float* out) {
    memcpy(out, s->x, s->m->cfg.hidden * sizeof(float));
}

/* Test-only: overwrite n cached K or V rows of one layer from position pos0
 * (f32 rows of kv_dim), so that a test can continue a session from a cache
 * another implementation filled.  No counterpart in lokal. */
ORACLE_API int oracle_session_load_kv(oracle_session* s, uint32_t layer, size_t pos0, size_t n, int which_v,
                                      const float* rows) {
    if (layer >= s->m->cfg.n_layers || pos0 > s->max_seq || n > s->max_seq - pos0) return -1;
    float* dst = (which_v ? s->v[layer] : s->k[layer]) + pos0 * s->m->kv_dim;
    memcpy(dst, rows, n * s->m->kv_dim * sizeof(float));
    return 0;
}

/* Read one layer's cached K or V row (f32) at position pos. */
ORACLE_API int oracle_session_kv(const oracle_session* s, uint32_t layer, size_t pos, int which_v, float* out) {
    if (layer >= s->m->cfg.n_layers || pos >= s->max_seq) return -1;
    const float* src = (which_v ? s->v[layer] : s->k[layer]) + pos * s->m->kv_dim;
    memcpy(out, src, s->m->kv_dim * sizeof(float));
    return 0;
}
