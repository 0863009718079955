// fused_rows.hip -- one decode step of a few Batcher rows (src/engine.rs:42-47:
// one token of each of NB sequences, each at its own position and KV slot) as
// ONE persistent kernel, like fused_step_kernel does for one sequence.
//
// Why: at small batch sizes the multi-row path (one launch per linear layer
// and per row-kernel, ~220 per step) pays launch gaps, not bytes; a decode
// step is latency-bound, and one launch with six grid-wide exchanges per
// layer serves NB rows for little more than the time it serves one.  Every
// weight row is read once per step and dotted with all NB activation rows.
//
// Stage map per layer (the same as fused.hip, each stage for NB rows):
//   S1 QKV      RMSNorm of each row + q/k/v rows (i, i+32) + bias + RoPE at the
//               row's position; k/v rounded to f16, written to the row's slot
//   S2 attn     one wave per (row, query head, 64-position tile) item
//   S3 merge    one wave per (row, query head)
//   S4 o_proj   + residual
//   S5 gate/up  RMSNorm + SwiGLU
//   S6 down     + residual -> the next layer's x, or, after the last layer,
//               plain f32 rows in x_out (final norm and lm_head run in the
//               multi-row kernels: one GEMM over all rows)
// Rows past nrows are padding: computed on token 0 at position 0 (reading
// slot of row 0) and never written to the KV cache or to x_out.
// Exchange buffers are (f32 | epoch) words laid out [2 by layer parity][NB][..].
#include "fused_impl.h"

#include <algorithm>

// gate/up units per wave of half 1 (issued after S2) and of half 0 (issued
// in S4); the rest are issued and used in S5, which exposes a load latency
#ifndef LKR_KB_F16
#define LKR_KB_F16 2
#define LKR_KA_F16 2
#endif
// Q4_K: one of each (its rows are wider; holding 3 + 2 spilled 68 bytes per
// lane, 2 + 2 24 bytes; TinyLlama shape, 2 / 4 rows: 0.894 / 1.337 ms per step
// at 3 + 2, 0.857 / 1.318 at 2 + 2, 0.852 / 1.312 at 1 + 1, measured)
#ifndef LKR_KB_Q4K
#define LKR_KB_Q4K 1
#define LKR_KA_Q4K 1
#endif
#define LKR_KB (WT == LK_F16 ? LKR_KB_F16 : (WT == LK_Q4_K ? LKR_KB_Q4K : 3))
#define LKR_KA (WT == LK_F16 ? LKR_KA_F16 : (WT == LK_Q4_K ? LKR_KA_Q4K : 2))

// Rows of the SwiGLU input the down stage takes per pass (the last pass takes
// what is left, so every pass covers rows that exist): at most 4 where the
// LDS needs it (8 rows: 2 passes of 4; 7 rows: 4 + 3; 6 rows: 3 + 3; 5 rows:
// one pass of 5).
__host__ __device__ constexpr int lkr_s6_rows(int nb) {
    return nb <= 5 ? nb : (nb == 6 ? 3 : 4);
}

namespace lkf {

using namespace lk;

template <int WT, int NCHH, int NCHI, int G, int NB>
__global__ __launch_bounds__(FT, 1) void fused_rows_kernel(const LkFusedArgs a) {
    extern __shared__ __align__(16) float lds[];  // 16-byte aligned after the static LDS (16-byte LDS accesses)
    const uint32_t h = a.h, I = a.I, nh = a.nh, nkv = a.nkv;
    const uint32_t qd = nh * 64, kvd = nkv * 64, qkvd = qd + 2 * kvd;
    // the down stage takes its input S6R rows at a time, so that NB = 8 fits
    constexpr int S6R = lkr_s6_rows(NB);
    const uint32_t hq_max = h > qd ? h : qd;
    const uint32_t xin_n = NB * hq_max > S6R * I ? NB * hq_max : S6R * I;
    float* xin = lds;                   // xin_n: the (normalised) input rows of a stage
    float* xres = xin + xin_n;          // NB * h: the residual rows
    float* red = xres + NB * h;         // NB * FW: block reductions
    float* gin = red + NB * FW;         // h
    float* gpost = gin + h;             // h
    float* wv = gpost + h;              // FW * 256: per wave q, this token's k and v, P
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* wq = wv + wave * 256;
    float* wk = wq + 64;
    float* wvc = wk + 64;
    float* wP = wvc + 64;
    LkFusedLayer* lay = (LkFusedLayer*)(wv + FW * 256);
    {
        const uint32_t* src = (const uint32_t*)a.layers;
        uint32_t* dst = (uint32_t*)lay;
        const uint32_t n32 = a.n_layers * (uint32_t)(sizeof(LkFusedLayer) / 4);
        for (uint32_t i = threadIdx.x; i < n32; i += FT) dst[i] = src[i];
        lds_barrier();
    }

    Ctx c{&a, a.err, lane, wave, (int)(wave * gridDim.x + blockIdx.x), (int)(FW * gridDim.x)};
    constexpr int KC = 8;  // 16-byte chunks in a 64-element f16 cache row
    const uint32_t base = a.epoch[0];
    const uint32_t nL = a.n_layers;
    const uint32_t nps = a.max_chunks;
    const uint32_t nrows = a.nrows;
    // per-row token, position and slot (wave-uniform: scalar registers)
    uint32_t tok[NB], posr[NB], slotr[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const bool live = (uint32_t)b < nrows;
        tok[b] = __builtin_amdgcn_readfirstlane(live ? a.meta[b] : 0u);
        posr[b] = __builtin_amdgcn_readfirstlane(live ? a.meta[a.meta_cap + b] : 0u);
        slotr[b] = __builtin_amdgcn_readfirstlane(a.meta[2 * a.meta_cap + (live ? b : 0)]);
    }
    // the same in LDS for loops kept rolled (an indexed register array would
    // live in scratch, and a scratch read waits for every load in flight)
    __shared__ uint32_t rpos[NB], rslot[NB];
    __shared__ float rcs[NB][32][2];  // RoPE (cos, sin) of pair ip at row b's position
    if (threadIdx.x < NB) {
#pragma unroll
        for (int b = 0; b < NB; b++)
            if ((int)threadIdx.x == b) {
                rpos[b] = posr[b];
                rslot[b] = slotr[b];
            }
    }
    if (threadIdx.x < NB * 32) {  // pos * theta^(-2 ip / 64)
        const uint32_t b = threadIdx.x / 32, ipp = threadIdx.x % 32;
        uint32_t pb = posr[0];
#pragma unroll
        for (int k = 1; k < NB; k++) pb = b == (uint32_t)k ? posr[k] : pb;
        const float ang = __fmul_rn((float)pb, a.freq.f[ipp]);
        rcs[b][ipp][0] = cosf(ang);
        rcs[b][ipp][1] = sinf(ang);
    }
    // (visible after the barrier that ends the embedding stage)
    // attention items of row b: nh * ntile(b), one wave each
    uint32_t item0[NB + 1];
    item0[0] = 0;
#pragma unroll
    for (int b = 0; b < NB; b++) item0[b + 1] = item0[b] + nh * (posr[b] / 64 + 1);
    if (item0[NB] > (uint32_t)c.nw) {  // the host sizes batches so this never holds
        if (threadIdx.x == 0) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    const uint32_t U1 = (nh + 2 * nkv) * 32;
    const bool has1 = c.gw < (int)U1;
    uint32_t kind = 0, head = 0, ip = 0;
    if (has1) {
        const uint32_t hh = (uint32_t)c.gw / 32;
        ip = (uint32_t)c.gw % 32;
        if (hh < nh) { kind = 0; head = hh; }
        else if (hh < nh + nkv) { kind = 1; head = hh - nh; }
        else { kind = 2; head = hh - nh - nkv; }
    }
    Row<WT, NCHH> q1, q2;
    auto issue_qkv = [&](const LkFusedLayer& l) {
        const LkDevW& w = kind == 0 ? l.q : (kind == 1 ? l.k : l.v);
        row_issue(q1, w, head * 64 + ip, lane);
        row_issue(q2, w, head * 64 + ip + 32, lane);
    };
    if (has1) issue_qkv(lay[0]);
    for (uint32_t i = threadIdx.x; i < h; i += FT) {
        gin[i] = lk_g(lay[0].in_norm)[i];
        gpost[i] = lk_g(lay[0].post_norm)[i];
    }
    // S0: the embedding rows (src/model.rs:200-202)
#pragma unroll
    for (int b = 0; b < NB; b++)
        for (uint32_t j = threadIdx.x; j < h; j += FT) xres[b * h + j] = lk_embed_elem(a.embed, tok[b], j);
    lds_barrier();

    const uint16_t* kc0 = (const uint16_t*)a.kc;
    const uint16_t* vc0 = (const uint16_t*)a.vc;
    for (uint32_t L = 0; L < nL; L++) {
        const LkFusedLayer& ly = lay[L];
        const uint32_t ep = base * (nL + 1) + L + 1;
        const uint32_t par = L & 1;
        uint64_t* QB = a.qb + (size_t)par * NB * qkvd;
        uint64_t* PB = a.pb + (size_t)par * NB * nh * nps * 66;
        uint64_t* AB = a.ab + (size_t)par * NB * qd;
        uint64_t* XP = a.xpb + (size_t)par * NB * h;
        uint64_t* IB = a.ib + (size_t)par * NB * I;
        const size_t lay_off = (size_t)L * a.kv_layer;
        const int nwh = c.nw / 2;
        const bool half1 = wave >= FW / 2;
        auto unit_of = [&](int k) -> int {
            return half1 ? (c.gw - nwh) + k * nwh : LKR_KB * nwh + c.gw + k * nwh;
        };
        static_assert(LKR_KA <= LKR_KB, "half 0's units are held in the same registers as half 1's");
        const int nunits = half1 ? LKR_KB : LKR_KA;
        Row<WT, NCHH> orow;
        Row<WT, NCHH> gq[LKR_KB], uq[LKR_KB];
        Row<WT, NCHI> dn;
        // ---------------- S1: RMSNorm + QKV + bias + RoPE + KV append
        float b1 = 0.f, b2 = 0.f;
        if (has1) {
            const float* bias = kind == 0 ? ly.bq : (kind == 1 ? ly.bk : ly.bv);
            if (bias) {
                b1 = lk_g(bias)[head * 64 + ip];
                b2 = lk_g(bias)[head * 64 + ip + 32];
            }
        }
        if (L > 0) stage_in<16>(c, a.xb + (size_t)par * NB * h, NB * h, ep, xres, 1);
        rmsnorm_rows<NB>(xres, gin, h, a.eps, xin, red);
        // the row loops below stay rolled: unrolled, every row's LDS
        // addresses stay live and spill
        if (has1) {
            float d1r[NB], d2r[NB];  // every row's dots first: their LDS reads overlap
#pragma unroll
            for (int b = 0; b < NB; b++) {
                d1r[b] = lk_wave_sum(row_dot(q1, xin + b * h, h, lane));
                d2r[b] = lk_wave_sum(row_dot(q2, xin + b * h, h, lane));
            }
#pragma unroll
            for (int b = 0; b < NB; b++) {
                float d1 = d1r[b], d2 = d2r[b];
                if (lane == 0) {
                    const uint32_t r = head * 64 + ip;
                    d1 += b1;
                    d2 += b2;
                    if (kind < 2) rot(d1, d2, rcs[b][ip][0], rcs[b][ip][1]);
                    uint64_t* qb = QB + (size_t)b * qkvd;
                    if (kind == 0) {
                        publish(qb + r, d1, ep);
                        publish(qb + r + 32, d2, ep);
                    } else {
                        if ((uint32_t)b < nrows) {
                            uint16_t* cache = (uint16_t*)(kind == 1 ? a.kc : a.vc) + lay_off +
                                              (size_t)rslot[b] * a.slot_elems +
                                              ((size_t)head * a.max_seq + rpos[b]) * 64;
                            kv_put(cache + ip, d1);
                            kv_put(cache + ip + 32, d2);
                        }
                        const uint32_t off = qd + (kind == 2 ? kvd : 0) + r;
                        publish(qb + off, kv_round(d1, false), ep);
                        publish(qb + off + 32, kv_round(d2, false), ep);
                    }
                }
            }
        }
        // this wave's attention item: (row, query head, 64-position tile)
        const bool has2 = c.gw < (int)item0[NB];
        // row rb = the last row whose items start at or before this wave's;
        // per-row values are picked by selects (an indexed register array
        // would live in scratch)
        uint32_t rb = 0, i0 = 0, pos = posr[0], slot = slotr[0];
#pragma unroll
        for (int b = 1; b < NB; b++) {
            if ((uint32_t)c.gw >= item0[b]) {
                rb = (uint32_t)b;
                i0 = item0[b];
                pos = posr[b];
                slot = slotr[b];
            }
        }
        const uint32_t nt = pos / 64 + 1;
        const uint32_t hq = has2 ? ((uint32_t)c.gw - i0) / nt : 0, t = has2 ? ((uint32_t)c.gw - i0) % nt : 0;
        const uint32_t j = hq / G;
        const size_t kvb = lay_off + (size_t)slot * a.slot_elems + (size_t)j * a.max_seq * 64;
        lk_u32x4 kraw[KC], vraw[KC];
        if (has2) {  // cached rows (< pos) first; rows from pos on are replaced or masked
            uint32_t krow = t * 64u + (uint32_t)lane;
            krow = krow < pos ? krow : (pos ? pos - 1 : 0);
            const uint16_t* Kl = kc0 + kvb + krow * 64u;
            const uint16_t* Vl = vc0 + kvb + (t * 64u + ((uint32_t)lane & 7)) * 64u + ((uint32_t)lane >> 3) * 8;
#pragma unroll
            for (int q = 0; q < KC; q++) kraw[q] = *(const lk_u32x4*)((const uint8_t*)Kl + 16 * q);
#pragma unroll
            for (int q = 0; q < KC; q++) vraw[q] = *(const lk_u32x4*)(Vl + q * 8 * 64);
        }
        // ---------------- S2: attention partials (as fused.hip, per row)
        if (has2) {
            const uint32_t ntile = pos / 64 + 1;
            const bool has_cur = t + 1 == ntile;
            const uint32_t sub = (uint32_t)lane & 7, dq = ((uint32_t)lane >> 3) * 8;
            {
                const uint64_t* qb = QB + (size_t)rb * qkvd;
                const uint64_t* sq = qb + hq * 64 + lane;
                const uint64_t* sk = qb + qd + j * 64 + lane;
                const uint64_t* sv = qb + qd + kvd + j * 64 + lane;
                const uint64_t w0 = ld_word(sq);
                const uint64_t w1 = has_cur ? ld_word(sk) : 0;
                const uint64_t w2 = has_cur ? ld_word(sv) : 0;
                wq[lane] = (uint32_t)(w0 >> 32) == ep ? __uint_as_float((uint32_t)w0) : await(c, sq, ep);
                if (has_cur) {
                    wk[lane] = (uint32_t)(w1 >> 32) == ep ? __uint_as_float((uint32_t)w1) : await(c, sk, ep);
                    wvc[lane] = (uint32_t)(w2 >> 32) == ep ? __uint_as_float((uint32_t)w2) : await(c, sv, ep);
                }
            }
            wave_sync_lds();
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = 0.f;
            float m, l;
            {
                const uint32_t p = t * 64 + (uint32_t)lane;
                const bool valid = p <= pos;
                const bool cur = p == pos;
                float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    float k8[8];
                    unpack8(kraw, q, false, k8);
                    const float4 qa = *(const float4*)(wq + 8 * q);
                    const float4 qb = *(const float4*)(wq + 8 * q + 4);
                    s4[0] = fmaf(k8[0], qa.x, s4[0]); s4[1] = fmaf(k8[1], qa.y, s4[1]);
                    s4[2] = fmaf(k8[2], qa.z, s4[2]); s4[3] = fmaf(k8[3], qa.w, s4[3]);
                    s4[0] = fmaf(k8[4], qb.x, s4[0]); s4[1] = fmaf(k8[5], qb.y, s4[1]);
                    s4[2] = fmaf(k8[6], qb.z, s4[2]); s4[3] = fmaf(k8[7], qb.w, s4[3]);
                }
                float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
                if (has_cur) {
                    const float sc = lk_wave_sum(wk[lane] * wq[lane]);
                    if (cur) s = sc;
                }
                const float sg = valid ? s * 0.125f : -INFINITY;
                m = lk_wave_max(sg);
                const float pe = valid ? expf(sg - m) : 0.f;
                l = lk_wave_sum(pe);
                wP[(lane & 7) * 8 + (lane >> 3)] = pe;
                wave_sync_lds();
                const float4 pwa = *(const float4*)(wP + sub * 8), pwb = *(const float4*)(wP + sub * 8 + 4);
                const float pw8[8] = {pwa.x, pwa.y, pwa.z, pwa.w, pwb.x, pwb.y, pwb.z, pwb.w};
                if (!has_cur) {
#pragma unroll
                    for (int jj = 0; jj < 8; jj++) {
                        float v8[8];
                        unpack8(vraw, jj, false, v8);
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[e] = fmaf(pw8[jj], v8[e], acc[e]);
                    }
                } else {
                    const float4 va = *(const float4*)(wvc + dq), vb = *(const float4*)(wvc + dq + 4);
                    const float vc8[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
                    for (int jj = 0; jj < 8; jj++) {
                        const uint32_t pj = t * 64 + jj * 8 + sub;
                        float v8[8];
                        unpack8(vraw, jj, false, v8);
                        const float pw = pj <= pos ? pw8[jj] : 0.f;
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            const float v = pj == pos ? vc8[e] : (pj < pos ? v8[e] : 0.f);
                            acc[e] = fmaf(pw, v, acc[e]);
                        }
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float v = acc[e];
                v += lk_dpp<0xB1, 0xF>(v, 0.f);
                v += lk_dpp<0x4E, 0xF>(v, 0.f);
                v += lk_dpp<0x124, 0xF>(v, 0.f);
                acc[e] = v;
            }
            uint64_t* out = PB + (((size_t)rb * nh + hq) * nps + t) * 66;
            if (lane == 0) {
                publish(out, m, ep);
                publish(out + 1, l, ep);
            }
            if ((lane & 7) == 4) {
#pragma unroll
                for (int e = 0; e < 8; e++) publish(out + 2 + dq + e, acc[e], ep);
            }
        }
        // o_proj rows (and half 1's gate/up rows) are issued after the
        // attention stage: held across it they would push its K/V tile out of
        // registers
        if (c.gw < (int)h) row_issue(orow, ly.o, (uint32_t)c.gw, lane);
        if (half1) {
#pragma unroll
            for (int k = 0; k < LKR_KB; k++) {
                const int uu = unit_of(k);
                if (uu < (int)I) {
                    row_issue(gq[k], ly.gate, (uint32_t)uu, lane);
                    row_issue(uq[k], ly.up, (uint32_t)uu, lane);
                }
            }
        }
        // ---------------- S3: merge each (row, head)'s tiles -> attention output (lane = dim)
        if (c.gw < (int)(NB * nh)) {
            const uint32_t b3 = (uint32_t)c.gw / nh, h3 = (uint32_t)c.gw % nh;
            uint32_t p3 = posr[0];
#pragma unroll
            for (int b = 1; b < NB; b++)
                if ((uint32_t)b == b3) p3 = posr[b];
            const uint32_t nch = p3 / 64 + 1;
            const uint64_t* pp = PB + ((size_t)b3 * nh + h3) * nps * 66;
            const bool mk = lane < (int)nch;
            const uint64_t* pm = pp + (mk ? lane : 0) * 66;
            const uint64_t epw = (uint64_t)ep << 32;
            uint64_t wmw = mk ? ld_word(pm) : epw, wlw = mk ? ld_word(pm + 1) : epw;
            float mv = -INFINITY, lv = 0.f, M = 0.f, sc = 0.f, Ls = 0.f, A = 0.f;
            for (uint32_t k0 = 0; k0 < nch; k0 += 16) {
                uint64_t wa[16];
#pragma unroll
                for (int k = 0; k < 16; k++) wa[k] = k0 + k < nch ? ld_word(pp + (k0 + k) * 66 + 2 + lane) : epw;
                for (uint32_t r = 0;; r++) {
                    bool done = (uint32_t)(wmw >> 32) == ep && (uint32_t)(wlw >> 32) == ep;
#pragma unroll
                    for (int k = 0; k < 16; k++) done &= (uint32_t)(wa[k] >> 32) == ep;
                    if (done) break;
                    if ((r & 255) == 255) {
                        if (__hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
                        if (r > (1u << 21)) {
                            __hip_atomic_store(c.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            break;
                        }
                    }
                    __builtin_amdgcn_s_sleep(1);
                    if ((uint32_t)(wmw >> 32) != ep) wmw = ld_word(pm);
                    if ((uint32_t)(wlw >> 32) != ep) wlw = ld_word(pm + 1);
#pragma unroll
                    for (int k = 0; k < 16; k++)
                        if ((uint32_t)(wa[k] >> 32) != ep) wa[k] = ld_word(pp + (k0 + k) * 66 + 2 + lane);
                }
                if (k0 == 0) {
                    if (mk) {
                        mv = __uint_as_float((uint32_t)wmw);
                        lv = __uint_as_float((uint32_t)wlw);
                    }
                    M = lk_wave_max(mv);
                    sc = mk ? expf(mv - M) : 0.f;
                    Ls = lk_wave_sum(sc * lv);
                }
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    if (k0 + k < nch) {
                        const float sk = __builtin_bit_cast(
                            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), k0 + k));
                        A = fmaf(sk, __uint_as_float((uint32_t)wa[k]), A);
                    }
                }
            }
            publish(AB + (size_t)b3 * qd + h3 * 64 + lane, A / Ls, ep);
        }
        // ---------------- S4: o_proj + residual -> x'
        {
            stage_in<8>(c, AB, NB * qd, ep, xin, -1);
            if (c.gw < (int)h) {
#pragma unroll 1
                for (int b = 0; b < NB; b++) {
                    const float d = lk_wave_sum(row_dot(orow, xin + b * qd, qd, lane));
                    if (lane == 0) publish(XP + (size_t)b * h + c.gw, xres[b * h + c.gw] + d, ep);
                }
            }
            if (!half1) {
#pragma unroll
                for (int k = 0; k < LKR_KA; k++) {
                    const int uu = unit_of(k);
                    if (uu < (int)I) {
                        row_issue(gq[k], ly.gate, (uint32_t)uu, lane);
                        row_issue(uq[k], ly.up, (uint32_t)uu, lane);
                    }
                }
            }
        }
        // ---------------- S5: RMSNorm + gate/up + SwiGLU -> inner
        {
            stage_in<16>(c, XP, NB * h, ep, xres, 1);
            rmsnorm_rows<NB>(xres, gpost, h, a.eps, xin, red);
#pragma unroll
            for (int k = 0; k < LKR_KB; k++) {
                const int uu = unit_of(k);
                if (k < nunits && uu < (int)I) {
#pragma unroll 1
                    for (int b = 0; b < NB; b++) {
                        float gu[2] = {row_dot(gq[k], xin + b * h, h, lane), row_dot(uq[k], xin + b * h, h, lane)};
                        wave_sums(gu);  // the two sums interleaved
                        if (lane == 0) publish(IB + (size_t)b * I + uu, gu[0] / (1.0f + expf(-gu[0])) * gu[1], ep);
                    }
                }
            }
            for (int uu = (LKR_KA + LKR_KB) * nwh + c.gw; uu < (int)I; uu += c.nw) {
                Row<WT, NCHH> gr, pr;
                row_issue(gr, ly.gate, (uint32_t)uu, lane);
                row_issue(pr, ly.up, (uint32_t)uu, lane);
#pragma unroll 1
                for (int b = 0; b < NB; b++) {
                    float gu[2] = {row_dot(gr, xin + b * h, h, lane), row_dot(pr, xin + b * h, h, lane)};
                    wave_sums(gu);
                    if (lane == 0) publish(IB + (size_t)b * I + uu, gu[0] / (1.0f + expf(-gu[0])) * gu[1], ep);
                }
            }
            if (c.gw < (int)h) row_issue(dn, ly.down, (uint32_t)c.gw, lane);
            if (has1 && L + 1 < nL) issue_qkv(lay[L + 1]);
        }
        // ---------------- S6: down + residual -> x of layer L+1 (or x_out)
        {
            const uint32_t epn = ep + 1;
            uint64_t* XN = a.xb + (size_t)((L + 1) & 1) * NB * h;
            const bool last = L + 1 == nL;
            auto put = [&](int b, int u, float v) {
                if (!last) publish(XN + (size_t)b * h + u, v, epn);
                else if ((uint32_t)b < nrows) a.x_out[(size_t)b * h + u] = v;
            };
#pragma unroll 1
            for (int p0 = 0; p0 < NB; p0 += S6R) {  // S6R rows of the SwiGLU input at a time
                const int nr = NB - p0 < S6R ? NB - p0 : S6R;  // the last pass: the rows left
                stage_in<24>(c, IB + (size_t)p0 * I, (uint32_t)nr * I, ep, xin, -1);
                if (c.gw < (int)h) {
#pragma unroll 1
                    for (int b = 0; b < nr; b++) {
                        const float d = lk_wave_sum(row_dot(dn, xin + b * I, I, lane));
                        if (lane == 0) put(p0 + b, c.gw, xres[(p0 + b) * h + c.gw] + d);
                    }
                }
                for (int uu = c.gw + c.nw; uu < (int)h; uu += c.nw) {
                    Row<WT, NCHI> rr;
                    row_issue(rr, ly.down, (uint32_t)uu, lane);
#pragma unroll 1
                    for (int b = 0; b < nr; b++) {
                        const float d = lk_wave_sum(row_dot(rr, xin + b * I, I, lane));
                        if (lane == 0) put(p0 + b, uu, xres[(p0 + b) * h + uu] + d);
                    }
                }
            }
            // the next layer's gains, by half 0 (half 1 polls first in S1);
            // this layer's last gain reads were before S6's input barrier,
            // and S1's first barrier orders these writes before its reads
            if (!last && !half1) {
                for (uint32_t i = threadIdx.x; i < h; i += FT / 2) {
                    gin[i] = lk_g(lay[L + 1].in_norm)[i];
                    gpost[i] = lk_g(lay[L + 1].post_norm)[i];
                }
            }
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) a.epoch[0] = base + 1;
}

}  // namespace lkf

size_t lk_fused_rows_lds_bytes(uint32_t h, uint32_t I, uint32_t nh, uint32_t nb) {
    const size_t s6r = (size_t)lkr_s6_rows((int)nb);
    const size_t hq_max = h > nh * 64 ? h : nh * 64;
    const size_t xin_n = std::max((size_t)nb * hq_max, s6r * I);
    return (xin_n + (size_t)nb * h + (size_t)nb * FW + 2 * (size_t)h + (size_t)FW * 256) * 4 +
           LK_FUSED_MAX_LAYERS * sizeof(LkFusedLayer);
}

template <int WT, int NCHH, int NCHI, int G, int NB>
static hipError_t launch_rows_t(const LkFusedArgs& a, unsigned blocks, size_t lds, hipStream_t st, bool setup) {
    auto kfn = lkf::fused_rows_kernel<WT, NCHH, NCHI, G, NB>;
    if (setup) {
        hipError_t e = hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        int nb = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kfn, FT, lds);
        if (e != hipSuccess) return e;
        return nb >= 1 ? hipSuccess : hipErrorInvalidConfiguration;
    }
    hipLaunchKernelGGL(kfn, dim3(blocks), dim3(FT), lds, st, a);
    return hipGetLastError();
}

// Instantiated shapes: (weight type, 16-byte chunks per lane for rows of
// hidden / intermediate width, GQA group), f16 KV, 2-7 or LK_FUSED_ROWS rows.
#define LKR_SHAPES(X)                       \
    X(LK_Q8_0, 1, 5, 7)  /* Qwen2.5-0.5B */ \
    X(LK_F16, 2, 3, 3)   /* SmolLM2-135M */ \
    X(LK_Q4_K, 1, 3, 8)  /* TinyLlama-1.1B */

hipError_t lk_fused_rows_launch(const LkFusedArgs& a, uint32_t wt, int nchh, int nchi, int G, uint32_t nb,
                                unsigned blocks, size_t lds, hipStream_t st, bool setup) {
#define X(T, NH, NI, GG)                                                                           \
    if (wt == T && nchh == NH && nchi == NI && G == GG)                                            \
        return nb <= 2    ? launch_rows_t<T, NH, NI, GG, 2>(a, blocks, lds, st, setup)             \
               : nb == 3 ? launch_rows_t<T, NH, NI, GG, 3>(a, blocks, lds, st, setup)              \
               : nb <= 4 ? launch_rows_t<T, NH, NI, GG, 4>(a, blocks, lds, st, setup)              \
               : nb == 5 ? launch_rows_t<T, NH, NI, GG, 5>(a, blocks, lds, st, setup)              \
               : nb == 6 ? launch_rows_t<T, NH, NI, GG, 6>(a, blocks, lds, st, setup)              \
               : nb == 7 ? launch_rows_t<T, NH, NI, GG, 7>(a, blocks, lds, st, setup)              \
                         : launch_rows_t<T, NH, NI, GG, LK_FUSED_ROWS>(a, blocks, lds, st, setup);
    LKR_SHAPES(X)
#undef X
    return hipErrorNotSupported;
}
