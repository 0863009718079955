// fused.hip -- the whole decode step of one token (Model::forward,
// src/model.rs:196-262) as ONE persistent kernel on gfx950.
//
// Why: batch-1 decode is a chain of ~5 dependent stages per layer (QKV ->
// attention -> o_proj -> gate/up -> down).  As separate kernels every stage
// pays a kernel boundary (~1.6 us in a HIP graph on MI355X) plus a cold
// weight fetch on the critical path.  Here one workgroup per CU runs every
// stage; a stage
//   1. issues the HBM loads of its own weight rows (they do not depend on
//      the activations, so they are in flight while the wave waits),
//   2. waits for its input vector, which the producing stage published as
//      64-bit words (f32 value | 32-bit epoch) with agent-coherent stores --
//      the wait and the data read are the same memory round trip, no
//      atomics and no grid barrier,
//   3. computes and publishes its outputs the same way.
// The epoch is (token counter, layer), so buffers never need clearing;
// consecutive layers alternate between two copies of each buffer.
//
// Stage map (matvec units are spread wave-major over all CUs):
//   S1 QKV      RMSNorm(x) + q/k/v rows in (i, i+32) pairs + bias + RoPE;
//               k/v rounded to the cache type, written to the KV cache and
//               published for this token's attention
//   S2 attn     one wave per (query head, chunk of 64-position tiles), spread
//               over the whole grid: K/V of the chunk's first tile loaded
//               before the wait for q; online softmax across the chunk's
//               tiles; one (m, l, acc[64]) partial each
//   S3 merge    one wave per query head folds its chunks -> attention output
//   S4 o_proj   o_proj + residual -> x'
//   S5 gate/up  RMSNorm(x') + SwiGLU  -> inner
//   S6 down     + residual            -> x of the next layer
// The final RMSNorm + lm_head + argmax is the next launch (lmhead.hip): the
// 145 MB lm_head stream wants 4 blocks per CU, this kernel holds one.
// Weight rows of a stage are issued one stage early (o_proj with gate/up,
// gate/up with down, down with the next layer's q/k/v).
// Every wait is bounded: on timeout the kernel raises an error flag, stops
// waiting everywhere, and the host reports the failure.
#include "fused_impl.h"

#define FCH 64
#define LKF_TRACE_MAX 256
// gate/up units per wave of half 1 (issued in S1) and of half 0 (issued in
// S4); the rest are issued and used in S5.  Measured per type: holding more
// rows ahead raises register pressure (Q4_K rows carry 16-byte super-block
// heads and spilled at 3 + 2; a spill reload waits for every load in
// flight), holding fewer serialises S5.  Qwen2.5 Q8_0: 2 + 2 (2265 tok/s;
// 3 + 2: 2217, 1 + 1: 2197); SmolLM2 F16: 1 + 1 (2207; 3 + 2: 2071);
// TinyLlama Q4_K: 1 + 1 (1493; 3 + 2: 1226).
#define LKF_KB (WT == LK_Q8_0 ? 2 : 1)
#define LKF_KA (WT == LK_Q8_0 ? 2 : 1)
// gate/up units in flight together in S5 beyond the held ones (Qwen2.5 Q8_0:
// 2 -> 2319 tok/s, 1 -> 2294; TinyLlama Q4_K: 2 spills, 1347 against 1487)
#define LKF_XU (WT == LK_Q4_K ? 1 : 2)
#ifndef LKF_X1
#define LKF_X1 (WT == LK_Q8_0)
#endif
// Stage timestamps of every block (thread 0), kept in LDS and copied out at
// the end so that tracing adds no global-memory traffic mid-stage;
// LKF_SUB marks sub-steps of layer 1.
#define LKF_MARK(k)                                                 \
    do {                                                            \
        if (tracing && threadIdx.x == 0) ltr[(k)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define LKF_SUB(k)                                                  \
    do {                                                            \
        if (L == 1) LKF_MARK(2 + 6 * nL + 1 + (k));                 \
    } while (0)

namespace lkf {

using namespace lk;

// XCD-local exchange words: plain stores land in the XCD's L2, nontemporal
// loads bypass the CU's L1 and read that L2.  Valid only between workgroups
// of one XCD.
__device__ __forceinline__ void publish_x(uint64_t* p, float v, uint32_t ep) {
    *(__attribute__((address_space(1))) uint64_t*)p = word(v, ep);
}
__device__ __forceinline__ uint64_t ld_x(const uint64_t* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) uint64_t*)p);
}
__device__ __forceinline__ float await_x(const Ctx& c, const uint64_t* p, uint32_t ep) {
    uint64_t w = ld_x(p);
    for (uint32_t n = 0; (uint32_t)(w >> 32) != ep; n++) {
        __builtin_amdgcn_s_sleep(1);
        w = ld_x(p);
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

template <int WT, int NCHH, int NCHI, typename KV, int G>
__global__ __launch_bounds__(FT, 1) void fused_step_kernel(const LkFusedArgs a) {
    extern __shared__ __align__(16) float lds[];  // 16-byte aligned after the static LDS (16-byte LDS accesses)
    const uint32_t h = a.h, I = a.I, nh = a.nh, nkv = a.nkv;
    const uint32_t qd = nh * 64, kvd = nkv * 64, qkvd = qd + 2 * kvd;
    const uint32_t vmax = (I > h ? I : h) > qd ? (I > h ? I : h) : qd;
    float* xin = lds;                 // vmax: the (normalised) input vector of a stage
    float* xres = xin + vmax;         // h: the residual stream of this layer
    float* red = xres + h;            // 16: block reductions
    float* gin = red + 16;            // h: this layer's input_layernorm gains
    float* gpost = gin + h;           // h: this layer's post_attention_layernorm gains
    uint64_t* ltr = (uint64_t*)(gpost + h + (h & 1));  // LKF_TRACE_MAX stage timestamps
    float* wv = (float*)(ltr + LKF_TRACE_MAX);  // FW * 256: per wave q, this token's k and v, P
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: stage branches stay scalar
    float* wq = wv + wave * 256;      // [64] the query head's q
    float* wk = wq + 64;              // [64] this token's k (the chunk holding pos)
    float* wvc = wk + 64;             // [64] this token's v
    float* wP = wvc + 64;             // [64] softmax weights of a tile, [group][jj] order
    // The layer descriptors (weight pointers, shapes) in LDS: read from global
    // memory mid-kernel they would be vector loads, and the s_waitcnt before
    // the address arithmetic would also wait for every weight row already in
    // flight (vector loads retire in order) -- a full HBM round trip per
    // row issue.  LDS reads wait on their own counter.
    LkFusedLayer* lay = (LkFusedLayer*)(wv + FW * 256);
    uint32_t* slot_lds = (uint32_t*)(lay + LK_FUSED_MAX_LAYERS);
    // This workgroup's XCD (hardware id) and its slot among the XCD's
    // gridDim / LK_XCDS workgroups: the CP hands workgroups to the XCDs in
    // turn, so each XCD holds the same number of them, and an arrival counter
    // per XCD numbers them (counters only grow: slot = count mod the XCD's
    // share).  The counter wraps at the share (atomic increment modulo nslot),
    // so it never passes 2^32 and hands out duplicate slots there when nslot
    // is not a power of two.
    const uint32_t xcd = __builtin_amdgcn_s_getreg(LK_HWREG_XCC_ID) & (LK_XCDS - 1);
    const uint32_t nslot = gridDim.x / LK_XCDS;
    // The slot counter, the session's step state, the lm_head keys to fold
    // and the layer descriptors are loaded together: one memory round trip
    // before the fold and the first rows, not one after another.
    uint32_t slot_raw = 0;
    if (threadIdx.x == 0)
        slot_raw = __builtin_amdgcn_atomic_inc32(a.xcd_cnt + xcd * LK_XCD_CNT_STRIDE, nslot - 1, __ATOMIC_RELAXED,
                                                 "agent");
    static_assert(LK_HEAD_MAX_BLOCKS <= 2 * FT, "two lm_head blocks' keys per thread");
    uint4 s0 = make_uint4(0, 0, 0, 0);  // token, pos, n_out, n_feed
    uint2 s1 = make_uint2(0, 0);        // fed, pending
    uint64_t kw[4] = {0, 0, 0, 0};
    uint32_t hep = 0;  // the epoch of the keys to fold
    if (!a.meta) {
        s0 = *(const uint4*)lk_g((const uint32_t*)a.st);
        s1 = *(const uint2*)lk_g((const uint32_t*)a.st + 4);
        if (a.head_keys) {
            hep = *lk_g(a.head_epoch) + 1;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t i = threadIdx.x + (uint32_t)(k >> 1) * FT;
                if (i < a.head_blocks)
                    kw[k] = __hip_atomic_load(a.head_keys + 2 * i + (k & 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    {
        const uint32_t* src = (const uint32_t*)a.layers;
        uint32_t* dst = (uint32_t*)lay;
        const uint32_t n32 = a.n_layers * (uint32_t)(sizeof(LkFusedLayer) / 4);
        for (uint32_t i = threadIdx.x; i < n32; i += FT) dst[i] = src[i];
        if (threadIdx.x == 0) *slot_lds = slot_raw % nslot;
        lds_barrier();
    }

    Ctx c{&a, a.err, lane, wave, (int)(wave * gridDim.x + blockIdx.x), (int)(FW * gridDim.x)};
    constexpr bool KV32 = sizeof(KV) == 4;
    constexpr int KC = KV32 ? 16 : 8;  // 16-byte chunks in a 64-element cache row
    const uint32_t base = a.epoch[0];
    // the step's token and position: the session's device state, or (a
    // Batcher row, meta set) row 0 of the Batcher's row table, whose cache
    // slot selects the KV rows
    uint32_t pos, token, slot = 0;
    // the session's step state (and, for block 0, what it writes back at the end)
    // (kept in LDS until block 0 writes it back at the end: held in registers
    // across the layers it would spill, and a spill reload waits for every
    // weight row in flight)
    __shared__ uint32_t st_keep[9];
    uint32_t n_out = 0, n_feed = 0, fed = 0, best_id = 0, out_at = 0;
    bool folded = false, took_argmax = false;
    if (a.meta) {
        token = __builtin_amdgcn_readfirstlane(a.meta[0]);
        pos = __builtin_amdgcn_readfirstlane(a.meta[a.meta_cap]);
        slot = __builtin_amdgcn_readfirstlane(a.meta[2 * a.meta_cap]);
    } else {
        // the state, the key epoch and this thread's key words were loaded
        // at the start (the keys whether or not they turn out to be pending)
        token = s0.x;
        pos = s0.y;
        n_out = s0.z;
        n_feed = s0.w;
        fed = s1.x;
        if (s1.y && a.head_keys) {
            // The previous step's lm_head left its per-block argmax keys:
            // fold them here, where the token is consumed (every workgroup
            // does, from the same words), and advance the step as the greedy
            // loop does.  wv (per-wave LDS) is free until the layers start.
            uint64_t* kb = (uint64_t*)(wv);
            bool ok = true;
            uint64_t b = 0;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const uint32_t i = threadIdx.x + (uint32_t)k * FT;
                if (i < a.head_blocks) {
                    ok &= (uint32_t)(kw[2 * k] >> 32) == hep && (uint32_t)(kw[2 * k + 1] >> 32) == hep;
                    const uint64_t kk = (kw[2 * k] << 32) | (kw[2 * k + 1] & 0xFFFFFFFFu);
                    b = kk > b ? kk : b;
                }
            }
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) {
                const uint64_t o = __shfl_xor(b, m, 64);
                b = o > b ? o : b;
            }
            if (lane == 0) kb[wave] = b;
            if (!ok) (void)__hip_atomic_fetch_or(a.err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lds_barrier();
            b = kb[0];
#pragma unroll
            for (int w2 = 1; w2 < FW; w2++) b = kb[w2] > b ? kb[w2] : b;
            best_id = lk_argmax_idx(b);
            took_argmax = n_feed == 0;
            out_at = n_out;
            lk_step_advance(token, pos, n_out, n_feed, fed, best_id, a.feed, nullptr, false);
            folded = true;
            lds_barrier();  // kb is reused as wave scratch below
        }
        token = __builtin_amdgcn_readfirstlane(token);
        pos = __builtin_amdgcn_readfirstlane(pos);
        if (threadIdx.x == 0) {
            st_keep[0] = token;
            st_keep[1] = pos;
            st_keep[2] = n_out;
            st_keep[3] = n_feed;
            st_keep[4] = fed;
            st_keep[5] = (folded ? 1u : 0u) | (took_argmax ? 2u : 0u);
            st_keep[6] = best_id;
            st_keep[7] = out_at;
            st_keep[8] = hep;
        }
    }
    KV* const kc0 = (KV*)a.kc + (size_t)slot * a.slot_elems;
    KV* const vc0 = (KV*)a.vc + (size_t)slot * a.slot_elems;
    const uint32_t nL = a.n_layers;
    const float fpos = (float)pos;
    // attention unit: a 64-position cache tile, or half of one with an f32
    // cache (a whole f32 tile's K and V would take 128 registers per lane)
    constexpr uint32_t UNIT = lk_fused_unit(KV32);
    const uint32_t ntile = pos / UNIT + 1;          // units holding positions 0..pos
    // attention items: (query head, chunk of tpw consecutive tiles), one wave
    // each; tpw grows with the context so a head never has more than
    // LK_FUSED_MAX_CH chunks (S3 holds one chunk per lane)
    const uint32_t tpw = (ntile + LK_FUSED_MAX_CH - 1) / LK_FUSED_MAX_CH;
    const uint32_t nch = (ntile + tpw - 1) / tpw;  // partials per head
    const uint32_t nps = a.max_chunks;             // partial slots per head

    // XCD-local work.  Query head hq belongs to XCD hq * 8 / nh, so XCD x
    // owns heads [h0, h1) and the kv heads [j0, j1] they read.  The q/k/v rows
    // of those heads (S1), their attention chunks (S2) and merges (S3) run on
    // XCD x's workgroups, and the words these three stages exchange stay in
    // its L2: plain stores, nontemporal (L1-bypassing) loads -- a hop inside
    // an XCD costs ~0.28 us against ~0.6 us through the memory-side cache.
    // Each XCD computes the k/v rows of its kv heads itself; the XCD owning a
    // kv head's first query head writes them to the cache.
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the slot's LDS store
    __builtin_amdgcn_s_barrier();
    const uint32_t lw = (uint32_t)wave * nslot + __builtin_amdgcn_readfirstlane(*slot_lds);  // XCD-local wave index
    const uint32_t h0 = (xcd * nh + LK_XCDS - 1) / LK_XCDS, h1 = ((xcd + 1) * nh + LK_XCDS - 1) / LK_XCDS;
    const uint32_t nq = h1 - h0;
    const uint32_t j0 = nq ? h0 / G : 0, nj = nq ? (h1 - 1) / G - j0 + 1 : 0;
    // S1 work of this wave: q/k/v rows (i, i+32) of one head
    const uint32_t U1 = (nq + 2 * nj) * 32;
    const bool has1 = lw < U1;
    uint32_t kind = 0, head = 0, ip = 0;
    bool kv_writer = false;
    if (has1) {
        ip = lw % 32;
        const uint32_t it = lw / 32;
        if (it < nq) { kind = 0; head = h0 + it; }
        else {
            const uint32_t jt = it - nq;
            kind = 1 + (jt & 1);
            head = j0 + jt / 2;
            kv_writer = (head * G) * LK_XCDS / nh == xcd;
        }
    }
    uint64_t* QX = a.qb + (size_t)xcd * qkvd;  // this XCD's q/k/v words (parity copies LK_XCDS * qkvd apart)
    const bool tracing = a.trace != nullptr;  // every workgroup records its own row
    if (tracing && threadIdx.x == 0)
        for (uint32_t k = 0; k < lk_fused_trace_len(nL); k++) ltr[k] = 0;
    Row<WT, NCHH> q1, q2;  // prefetched one stage ahead (layer L's rows during layer L-1's down)
    auto issue_qkv = [&](const LkFusedLayer& l) {
        const LkDevW& w = kind == 0 ? l.q : (kind == 1 ? l.k : l.v);
        row_issue(q1, w, head * 64 + ip, lane);
        row_issue(q2, w, head * 64 + ip + 32, lane);
    };
    if (has1) issue_qkv(lay[0]);
    // the same rotation angle every layer: pos * theta^(-2 ip / 64).  It is
    // wave-uniform, so it lives in scalar registers: a value the register
    // allocator spills to scratch is reloaded with a vector-memory wait that
    // also waits for every weight row in flight.
    float rc = 1.f, rsn = 0.f;
    if (has1 && kind < 2) {
        const float ang = __fmul_rn(fpos, a.freq.f[ip]);
        rsn = sinf(ang);
        rc = cosf(ang);
    }
    rc = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, rc)));
    rsn = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, rsn)));
    // a layer's RMSNorm gains go to LDS one layer ahead (loaded into
    // registers during the previous layer's down stage)
    // (loaded by half 0 only: half 1 polls first in the next layer)
    constexpr int LKF_NPT = (NCHH * 64 * (int)ChunkTraits<WT>::elems + FT / 2 - 1) / (FT / 2);  // gains per thread
    float ngi[LKF_NPT], ngp[LKF_NPT];
    auto gains_issue = [&](const LkFusedLayer& l) {
#pragma unroll
        for (int k = 0; k < LKF_NPT; k++) {
            const uint32_t i = threadIdx.x + k * (FT / 2);
            ngi[k] = (threadIdx.x < FT / 2 && i < h) ? lk_g(l.in_norm)[i] : 0.f;
            ngp[k] = (threadIdx.x < FT / 2 && i < h) ? lk_g(l.post_norm)[i] : 0.f;
        }
    };
    auto gains_store = [&]() {
#pragma unroll
        for (int k = 0; k < LKF_NPT; k++) {
            const uint32_t i = threadIdx.x + k * (FT / 2);
            if (threadIdx.x < FT / 2 && i < h) {
                gin[i] = ngi[k];
                gpost[i] = ngp[k];
            }
        }
    };
    gains_issue(lay[0]);
    gains_store();

    LKF_MARK(0);
    // S0: every block takes the embedding row itself (src/model.rs:200-202).
    for (uint32_t j = threadIdx.x; j < h; j += FT) xres[j] = lk_embed_elem(a.embed, token, j);
    lds_barrier();
    LKF_MARK(1);

    for (uint32_t L = 0; L < nL; L++) {
        const LkFusedLayer& ly = lay[L];
        const uint32_t ep = base * (nL + 1) + L + 1;
        const uint32_t par = L & 1;
        uint64_t* QB = QX + (size_t)par * LK_XCDS * qkvd;
        uint64_t* PB = a.pb + (size_t)par * nh * nps * 66;  // [head][chunk][m, l, acc[64]]
        // x, the attention output and x' are published in `rep` copies (one
        // per XCD at rep = 8: a vector polled by every workgroup is then read
        // from 8 places instead of one); a workgroup polls copy blockIdx % rep
        const uint32_t rep = a.rep, cp = blockIdx.x % rep;
        uint64_t* AB = a.ab + (size_t)par * LK_FUSED_REP * qd;
        uint64_t* XP = a.xpb + (size_t)par * LK_FUSED_REP * h;
        uint64_t* IB = a.ib + (size_t)par * I;
        // Weight rows are issued one or two stages before they are used, after
        // the stage's own outputs are published: vector loads retire in issue
        // order (a prefetch issued before a wait delays that wait) and issuing
        // stalls while the CU's memory queue is full.  (The attention stage
        // needs most registers, so only the o_proj row is held across it.)
        const uint32_t U5 = I;              // gate/up rows
        // gate/up units: half 1 (waves FW/2..) holds LKF_KB units, issued in S1
        // (it has no other work before S5); half 0 holds LKF_KA, issued in S4
        // after its o_proj rows; the rest (wide models) are done in S5 directly.
        const int nwh = c.nw / 2;
        const bool half1 = wave >= FW / 2;
        auto unit_of = [&](int k) -> int {
            return half1 ? (c.gw - nwh) + k * nwh : LKF_KB * nwh + c.gw + k * nwh;
        };
        static_assert(LKF_KA <= LKF_KB, "half 0's units are held in the same registers as half 1's");
        const int nunits = half1 ? LKF_KB : LKF_KA;
        Row<WT, NCHH> orow;                 // issued in S1, used in S4
        Row<WT, NCHH> gq[LKF_KB], uq[LKF_KB];  // issued in S1 (half 1) or S4 (half 0), used in S5
        Row<WT, NCHI> dn;                   // issued in S5, used in S6
        // the first unit past the held ones of a half-1 wave (which has no
        // o_proj row): issued in S4 after its input arrived, used in S5
        const int ux1 = (LKF_KA + LKF_KB) * nwh + (c.gw - nwh);
        const bool has_x1 = LKF_X1 && half1 && ux1 < (int)U5;
        Row<WT, NCHH> gx, ux;
        // ---------------- S1: RMSNorm + QKV + bias + RoPE + KV append
        // biases load while the input vector is awaited (held across stages
        // they would be spilled, see rc above)
        float b1 = 0.f, b2 = 0.f;
        if (has1) {
            const float* bias = kind == 0 ? ly.bq : (kind == 1 ? ly.bk : ly.bv);
            if (bias) {
                b1 = lk_g(bias)[head * 64 + ip];
                b2 = lk_g(bias)[head * 64 + ip + 32];
            }
        }
        // ---- this wave's attention item (S2)
        const bool has2 = lw < nq * nch;  // this wave has an attention item on its XCD
        const uint32_t hq = h0 + lw / nch, ck = lw % nch;
        const uint32_t j = hq / G;
        const uint32_t t0 = ck * tpw, t1 = t0 + tpw < ntile ? t0 + tpw : ntile;
        const bool chunk_cur = t1 == ntile;  // the chunk holding position pos
        const KV* K = kc0 + (size_t)L * a.kv_layer + (size_t)j * a.max_seq * 64;
        const KV* V = vc0 + (size_t)L * a.kv_layer + (size_t)j * a.max_seq * 64;
        const uint32_t sub = (uint32_t)lane & 7, dq = ((uint32_t)lane >> 3) * 8;
        // Cached positions (< pos) do not depend on this token: the first
        // tile is loaded before the wait for q.  The cache holds whole
        // 64-position tiles (its per-head stride is max_seq rounded up to
        // 64), so every row of a tile is in bounds; rows >= pos are
        // replaced (pos) or masked (> pos) below.
        // a unit's K and V per wave; with 32-position units lanes l and l + 32
        // hold the two halves of a position's dims (K)
        constexpr int KH = UNIT == 64 ? KC : KC / 2;
        uint4 kraw[KH], vraw[KH];
        // K rows from pos on are this token's (in flight from S1) or
        // unwritten: read row pos - 1 instead (the lane's score is
        // replaced or masked below)
        auto load_k = [&](uint32_t t) {
            uint32_t krow = t * UNIT + ((uint32_t)lane & (UNIT - 1));
            krow = krow < pos ? krow : (pos ? pos - 1 : 0);
            const KV* Kl = K + krow * 64u + (UNIT == 64 ? 0u : 32u * ((uint32_t)lane >> 5));
#pragma unroll
            for (int q = 0; q < KH; q++) kraw[q] = *(const uint4*)((const uint8_t*)Kl + 16 * q);
        };
        auto load_v = [&](uint32_t t) {
            const KV* Vl = V + (t * UNIT + sub) * 64u + dq;
#pragma unroll
            for (int q = 0; q < KH; q++)
                vraw[q] = *(const uint4*)(Vl + (KV32 ? (q / 2) * 8 * 64 + (q & 1) * 4 : q * 8 * 64));
        };
        // f16: a tile's K and V fit in registers together; f32: V follows the scores
        auto load_tile = [&](uint32_t t) {
            load_k(t);
            if constexpr (!KV32) load_v(t);
        };
        if (L > 0) stage_in<8>(c, a.xb + ((size_t)par * LK_FUSED_REP + cp) * h, h, ep, xres, 1);
        LKF_SUB(15);
        LKF_SUB(16);
        if (has1) {
            // RMSNorm of the lane's slice of x (per wave, no block barrier) and
            // both rows' dots, their wave sums interleaved
            float xr[NCHH][ChunkTraits<WT>::elems];
            norm_slice<WT, NCHH>(xres, gin, h, a.eps, lane, xr);
            float dd[2] = {row_dot_reg(q1, xr, h, lane), row_dot_reg(q2, xr, h, lane)};
            wave_sums(dd);
            float d1 = dd[0], d2 = dd[1];
            LKF_SUB(17);
            if (lane == 0) {
                const uint32_t r = head * 64 + ip;
                d1 += b1;  // zero when the model has no q/k/v biases
                d2 += b2;
                if (kind < 2) rot(d1, d2, rc, rsn);
                if (kind == 0) {
                    publish_x(QB + r, d1, ep);
                    publish_x(QB + r + 32, d2, ep);
                } else {
                    if (kv_writer) {
                        KV* cache = (kind == 1 ? kc0 : vc0) + (size_t)L * a.kv_layer +
                                    ((size_t)head * a.max_seq + pos) * 64;
                        kv_put(cache + ip, d1);
                        kv_put(cache + ip + 32, d2);
                    }
                    const uint32_t off = qd + (kind == 2 ? kvd : 0) + r;
                    publish_x(QB + off, kv_round(d1, KV32), ep);
                    publish_x(QB + off + 32, kv_round(d2, KV32), ep);
                }
            }
        }
        LKF_SUB(18);
        // o_proj rows (and half 1's gate/up rows) for S4 / S5: issued after
        // this wave's attention K/V loads, so the tile is not queued behind
        // this layer's weight stream
        auto issue_ahead = [&]() {
            if (c.gw < (int)h) row_issue(orow, ly.o, (uint32_t)c.gw, lane);
            if (half1) {
#pragma unroll
                for (int k = 0; k < LKF_KB; k++) {
                    const int uu = unit_of(k);
                    if (uu < (int)U5) {
                        row_issue(gq[k], ly.gate, (uint32_t)uu, lane);
                        row_issue(uq[k], ly.up, (uint32_t)uu, lane);
                    }
                }
            }
        };
        if (!has2) issue_ahead();
        LKF_MARK(2 + 6 * L + 0);
        // ---------------- S2: attention partials.  Item = (query head, chunk
        // of tpw tiles of 64 positions), one wave each, spread over the grid
        // (items past the first half's waves, at long contexts, go to the
        // second half): per tile the wave scores its 64 positions (lane =
        // position), folds the tile's max and sum into its running softmax,
        // and accumulates P.V with lane = (position group lane & 7, dims
        // 8 * (lane >> 3) ..+7).
        if (has2) {
            LKF_SUB(0);
            load_tile(t0);
            issue_ahead();
            LKF_SUB(1);
            {  // this head's q; this token's k and v for the chunk that holds pos
                const uint64_t* sq = QB + hq * 64 + lane;
                const uint64_t* sk = QB + qd + j * 64 + lane;
                const uint64_t* sv = QB + qd + kvd + j * 64 + lane;
                const uint64_t w0 = ld_x(sq);
                const uint64_t w1 = chunk_cur ? ld_x(sk) : 0;
                const uint64_t w2 = chunk_cur ? ld_x(sv) : 0;
                wq[lane] = (uint32_t)(w0 >> 32) == ep ? __uint_as_float((uint32_t)w0) : await_x(c, sq, ep);
                if (chunk_cur) {
                    wk[lane] = (uint32_t)(w1 >> 32) == ep ? __uint_as_float((uint32_t)w1) : await_x(c, sk, ep);
                    wvc[lane] = (uint32_t)(w2 >> 32) == ep ? __uint_as_float((uint32_t)w2) : await_x(c, sv, ep);
                }
            }
            wave_sync_lds();
            LKF_SUB(2);
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = 0.f;
            float m = -INFINITY, l = 0.f;
            for (uint32_t t = t0; t < t1; t++) {
                if (t > t0) {
                    wave_sync_lds();  // the previous tile's weight reads are done
                    load_tile(t);
                }
                const bool has_cur = t + 1 == ntile;  // the unit holding position pos
                const uint32_t p = t * UNIT + ((uint32_t)lane & (UNIT - 1));
                const bool own = UNIT == 64 || lane < 32;  // 32-position units: lanes 32.. repeat positions
                const bool valid = p <= pos;
                // this token's k (lane p == pos) comes from LDS: its cache row
                // is being written in this stage.  Selected per value rather
                // than written into kraw, which would make the wave wait for
                // every load still in flight into those registers (the V tile).
                const bool cur = p == pos;
                // four independent chains: one wave per SIMD has nothing to
                // hide a 64-long dependent FMA chain behind
                float s4[4] = {0.f, 0.f, 0.f, 0.f};
                const float* wqh = wq + (UNIT == 64 ? 0 : 32 * (lane >> 5));
#pragma unroll
                for (int q = 0; q < (UNIT == 64 ? 8 : 4); q++) {  // 8 dims at a time
                    float k8[8];
                    unpack8(kraw, q, KV32, k8);
                    const float4 qa = *(const float4*)(wqh + 8 * q);
                    const float4 qb = *(const float4*)(wqh + 8 * q + 4);
                    s4[0] = fmaf(k8[0], qa.x, s4[0]); s4[1] = fmaf(k8[1], qa.y, s4[1]);
                    s4[2] = fmaf(k8[2], qa.z, s4[2]); s4[3] = fmaf(k8[3], qa.w, s4[3]);
                    s4[0] = fmaf(k8[4], qb.x, s4[0]); s4[1] = fmaf(k8[5], qb.y, s4[1]);
                    s4[2] = fmaf(k8[6], qb.z, s4[2]); s4[3] = fmaf(k8[7], qb.w, s4[3]);
                }
                float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
                if constexpr (UNIT == 32) s += __shfl_xor(s, 32);  // the other 32 dims (lane +- 32)
                if (has_cur) {  // wave-uniform: lane = dim, then the wave sum
                    const float sc = lk_wave_sum(wk[lane] * wq[lane]);
                    if (cur) s = sc;
                }
                LKF_SUB(3);
                if constexpr (KV32) load_v(t);
                // the tile's part of math::softmax (src/math.rs:55-66), folded
                // into the chunk's running max and sum; chunks are combined in
                // S3 with the same split-invariant rescaling
                const float sg = valid && own ? s * 0.125f : -INFINITY;
                const float mn = fmaxf(m, lk_wave_max(sg));  // finite: the unit holds position <= pos
                const float fo = expf(m - mn);                // 0 on the chunk's first unit
                const float pe = valid && own ? expf(sg - mn) : 0.f;
                l = fmaf(l, fo, lk_wave_sum(pe));
                m = mn;
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] *= fo;
                constexpr int NJ = UNIT / 8;  // positions per lane in P.V (position groups of 8)
                if (own) wP[(lane & 7) * NJ + (lane >> 3)] = pe;  // [group][jj]: a lane's weights are adjacent
                wave_sync_lds();
                LKF_SUB(4);
                // this lane's NJ weights in one or two LDS reads; no
                // per-position branches (each would serialise an LDS round trip)
                float pw8[NJ];
                {
                    const float4 pwa = *(const float4*)(wP + sub * NJ);
                    pw8[0] = pwa.x; pw8[1] = pwa.y; pw8[2] = pwa.z; pw8[3] = pwa.w;
                    if constexpr (NJ == 8) {
                        const float4 pwb = *(const float4*)(wP + sub * NJ + 4);
                        pw8[4] = pwb.x; pw8[5] = pwb.y; pw8[6] = pwb.z; pw8[7] = pwb.w;
                    }
                }
                if (!has_cur) {  // wave-uniform: every position of the unit is < pos
#pragma unroll
                    for (int jj = 0; jj < NJ; jj++) {
                        float v8[8];
                        unpack8(vraw, jj, KV32, v8);
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[e] = fmaf(pw8[jj], v8[e], acc[e]);
                    }
                } else {
                    // position pos takes this token's v from LDS (as k above);
                    // positions past pos (unwritten rows) contribute nothing
                    const float4 va = *(const float4*)(wvc + dq), vb = *(const float4*)(wvc + dq + 4);
                    const float vc8[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
                    for (int jj = 0; jj < NJ; jj++) {
                        const uint32_t pj = t * UNIT + jj * 8 + sub;
                        float v8[8];
                        unpack8(vraw, jj, KV32, v8);
                        const float pw = pj <= pos ? pw8[jj] : 0.f;
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            const float v = pj == pos ? vc8[e] : (pj < pos ? v8[e] : 0.f);
                            acc[e] = fmaf(pw, v, acc[e]);
                        }
                    }
                }
            }
            LKF_SUB(5);
            // Sum the 8 position groups of each dims chunk (8 adjacent lanes):
            // quad_perm pairs, quad halves, then row_ror 4 (lane l takes lane
            // l-4 of its row), after which lanes 4..7 of each 8 hold the total.
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float v = acc[e];
                v += lk_dpp<0xB1, 0xF>(v, 0.f);
                v += lk_dpp<0x4E, 0xF>(v, 0.f);
                v += lk_dpp<0x124, 0xF>(v, 0.f);
                acc[e] = v;
            }
            uint64_t* out = PB + ((size_t)hq * nps + ck) * 66;
            if (lane == 0) {
                publish_x(out, m, ep);
                publish_x(out + 1, l, ep);
            }
            if ((lane & 7) == 4) {
#pragma unroll
                for (int e = 0; e < 8; e++) publish_x(out + 2 + dq + e, acc[e], ep);
            }
            LKF_SUB(6);
        }
        LKF_MARK(2 + 6 * L + 1);
        // ---------------- S3: merge each head's chunks -> attention output (lane = dim)
        if (lw < nq) {
            const uint32_t hq = h0 + lw;
            const uint64_t* pp = PB + (size_t)hq * nps * 66;
            // lane k < nch fetches tile k's (m, l); every lane fetches its dim
            // of every tile's acc, 16 tiles' words in flight at a time, and
            // every round re-polls all the words still missing together
            const bool mk = lane < (int)nch;
            const uint64_t* pm = pp + (mk ? lane : 0) * 66;
            const uint64_t epw = (uint64_t)ep << 32;
            uint64_t wmw = mk ? ld_x(pm) : epw, wlw = mk ? ld_x(pm + 1) : epw;
            float mv = -INFINITY, lv = 0.f, M = 0.f, sc = 0.f, Ls = 0.f, A = 0.f;
            for (uint32_t k0 = 0; k0 < nch; k0 += 16) {
                uint64_t wa[16];
#pragma unroll
                for (int k = 0; k < 16; k++) wa[k] = k0 + k < nch ? ld_x(pp + (k0 + k) * 66 + 2 + lane) : epw;
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
                    if ((uint32_t)(wmw >> 32) != ep) wmw = ld_x(pm);
                    if ((uint32_t)(wlw >> 32) != ep) wlw = ld_x(pm + 1);
#pragma unroll
                    for (int k = 0; k < 16; k++)
                        if ((uint32_t)(wa[k] >> 32) != ep) wa[k] = ld_x(pp + (k0 + k) * 66 + 2 + lane);
                }
                if (k0 == 0) LKF_SUB(20);
                if (k0 == 0) {
                    if (mk) {
                        mv = __uint_as_float((uint32_t)wmw);
                        lv = __uint_as_float((uint32_t)wlw);
                    }
                    M = lk_wave_max(mv);
                    sc = mk ? expf(mv - M) : 0.f;  // tile k's weight, held by lane k
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
            LKF_SUB(21);
            for (uint32_t k = 0; k < rep; k++) publish(AB + (size_t)k * qd + hq * 64 + lane, A / Ls, ep);
        }
        LKF_MARK(2 + 6 * L + 2);
        // ---------------- S4: o_proj + residual -> x'
        {
            const int u = c.gw;
            stage_in<4>(c, AB + (size_t)cp * qd, qd, ep, xin, -1);
            LKF_SUB(12);
            if (has_x1) {
                row_issue(gx, ly.gate, (uint32_t)ux1, lane);
                row_issue(ux, ly.up, (uint32_t)ux1, lane);
            }
            if (u < (int)h) {
                const float d = lk_wave_sum(row_dot(orow, xin, qd, lane));
                if (lane < (int)rep) publish(XP + (size_t)lane * h + u, xres[u] + d, ep);
            }
            LKF_SUB(13);
            // the next stage's rows: issued after the publish, because a wave
            // stalls at issue while its own earlier loads fill its queue
            if (!half1) {
#pragma unroll
                for (int k = 0; k < LKF_KA; k++) {
                    const int uu = unit_of(k);
                    if (uu < (int)U5) {
                        row_issue(gq[k], ly.gate, (uint32_t)uu, lane);
                        row_issue(uq[k], ly.up, (uint32_t)uu, lane);
                    }
                }
            }
            LKF_SUB(14);
        }
        LKF_MARK(2 + 6 * L + 3);
        // ---------------- S5: RMSNorm + gate/up + SwiGLU -> inner
        {
            stage_in<8>(c, XP + (size_t)cp * h, h, ep, xres, 1);
            LKF_SUB(8);
            // RMSNorm of the lane's slice of x' by every wave (no block
            // barrier), reused by all of the wave's gate/up rows
            float xr[NCHH][ChunkTraits<WT>::elems];
            norm_slice<WT, NCHH>(xres, gpost, h, a.eps, lane, xr);
            LKF_SUB(9);
            {
                float dd[2 * LKF_KB];
#pragma unroll
                for (int k = 0; k < LKF_KB; k++) {
                    dd[2 * k] = row_dot_reg(gq[k], xr, h, lane);
                    dd[2 * k + 1] = row_dot_reg(uq[k], xr, h, lane);
                }
                wave_sums(dd);
#pragma unroll
                for (int k = 0; k < LKF_KB; k++) {
                    const int uu = unit_of(k);
                    const float gg = dd[2 * k], up = dd[2 * k + 1];
                    if (k < nunits && uu < (int)U5 && lane == 0) publish(IB + uu, gg / (1.0f + expf(-gg)) * up, ep);
                }
            }
            if (has_x1) {
                float gu[2] = {row_dot_reg(gx, xr, h, lane), row_dot_reg(ux, xr, h, lane)};
                wave_sums(gu);
                if (lane == 0) publish(IB + ux1, gu[0] / (1.0f + expf(-gu[0])) * gu[1], ep);
            }
            LKF_SUB(10);
            if (L == 1 && tracing && threadIdx.x == FT - 64)  // the block's last wave (half 1)
                ltr[2 + 6 * nL + 1 + 22] = __builtin_amdgcn_s_memrealtime();
            LKF_SUB(11);
            // wider models: the remaining units, two at a time in flight
            // (Q4_K: one at a time, the second pair of rows would spill)
            constexpr int XU = LKF_XU;
            // (with LKF_X1 the first nwh of them went to half 1 in S4)
            for (int uu = (LKF_KA + LKF_KB) * nwh + c.gw + (LKF_X1 ? nwh : 0); uu < (int)U5; uu += XU * c.nw) {
                Row<WT, NCHH> gr[XU], pr[XU];
#pragma unroll
                for (int x = 0; x < XU; x++) {
                    const int ux = uu + x * c.nw;
                    if (ux < (int)U5) {  // wave-uniform
                        row_issue(gr[x], ly.gate, (uint32_t)ux, lane);
                        row_issue(pr[x], ly.up, (uint32_t)ux, lane);
                    }
                }
                float dd[2 * XU];
#pragma unroll
                for (int x = 0; x < XU; x++) {
                    dd[2 * x] = row_dot_reg(gr[x], xr, h, lane);
                    dd[2 * x + 1] = row_dot_reg(pr[x], xr, h, lane);
                }
                wave_sums(dd);
#pragma unroll
                for (int x = 0; x < XU; x++) {
                    const int ux = uu + x * c.nw;
                    const float gg = dd[2 * x], up = dd[2 * x + 1];
                    if (ux < (int)U5 && lane == 0) publish(IB + ux, gg / (1.0f + expf(-gg)) * up, ep);
                }
            }
            if (c.gw < (int)h) row_issue(dn, ly.down, (uint32_t)c.gw, lane);
            if (has1 && L + 1 < nL) issue_qkv(lay[L + 1]);  // the next layer's q/k/v rows
        }
        LKF_MARK(2 + 6 * L + 4);
        // ---------------- S6: down + residual -> x of layer L+1
        {
            const uint32_t epn = ep + 1;
            uint64_t* XN = a.xb + (size_t)((L + 1) & 1) * LK_FUSED_REP * h;
            stage_in<24>(c, IB, I, ep, xin, 1);
            LKF_SUB(7);
            if (c.gw < (int)h) {
                const float d = lk_wave_sum(row_dot(dn, xin, I, lane));
                LKF_SUB(19);
                if (lane < (int)rep) publish(XN + (size_t)lane * h + c.gw, xres[c.gw] + d, epn);
                if (a.x_out && L + 1 == nL && lane == 0) a.x_out[c.gw] = xres[c.gw] + d;  // a Batcher row's final x
            }
            for (int uu = c.gw + c.nw; uu < (int)h; uu += c.nw) {
                Row<WT, NCHI> rr;
                row_issue(rr, ly.down, (uint32_t)uu, lane);
                const float d = lk_wave_sum(row_dot(rr, xin, I, lane));
                if (lane < (int)rep) publish(XN + (size_t)lane * h + uu, xres[uu] + d, epn);
                if (a.x_out && L + 1 == nL && lane == 0) a.x_out[uu] = xres[uu] + d;
            }
            if (L + 1 < nL) {  // read after the next stage_in's barrier
                gains_issue(lay[L + 1]);
                gains_store();
            }
        }
        LKF_MARK(2 + 6 * L + 5);
    }

    // The final RMSNorm, lm_head and argmax run in the next launch
    // (lmhead.hip); every block has read `base`, so the epoch may advance.
    LKF_MARK(2 + 6 * nL);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.epoch[0] = base + 1;
        if (!a.meta && a.head_keys) {
            // every block has read the state: write this step's back, pending
            // the lm_head launch that follows
            const uint32_t fl = st_keep[5];
            if (fl & 1) {
                if (a.ids_out && (fl & 2)) a.ids_out[st_keep[7]] = st_keep[6];
                *a.head_epoch = st_keep[8];  // the folded launch's epoch
            }
            uint32_t* sp = (uint32_t*)a.st;
            *(uint4*)sp = make_uint4(st_keep[0], st_keep[1], st_keep[2], st_keep[3]);
            sp[4] = st_keep[4];
            sp[5] = 1;
        }
    }
    if (tracing && threadIdx.x == 0)
        for (uint32_t k = 0; k < lk_fused_trace_len(nL); k++) a.trace[(size_t)blockIdx.x * lk_fused_trace_len(nL) + k] = ltr[k];
}

}  // namespace lkf

size_t lk_fused_lds_bytes(uint32_t h, uint32_t I, uint32_t nh, uint32_t nkv, uint32_t G, uint32_t max_chunks) {
    (void)nkv;
    (void)G;
    (void)max_chunks;
    uint32_t vmax = I > h ? I : h;
    if (nh * 64 > vmax) vmax = nh * 64;
    return ((size_t)vmax + h + 16 + 2 * (size_t)h + (h & 1) + 2 * LKF_TRACE_MAX + (size_t)FW * 256) * 4 +
           LK_FUSED_MAX_LAYERS * sizeof(LkFusedLayer) + 16;
}
int lk_fused_threads() { return FT; }

// The XCD id of every workgroup of a `blocks`-workgroup launch (one thread
// each), for the host to check the placement the one-kernel step relies on.
__global__ void xcd_probe_kernel(uint32_t* out) {
    if (threadIdx.x == 0) out[blockIdx.x] = __builtin_amdgcn_s_getreg(LK_HWREG_XCC_ID) & 15u;
}
hipError_t lk_xcd_probe_launch(uint32_t* out, unsigned blocks, hipStream_t st) {
    hipLaunchKernelGGL(xcd_probe_kernel, dim3(blocks), dim3(64), 0, st, out);
    return hipGetLastError();
}

template <int WT, int NCHH, int NCHI, typename KV, int G>
static hipError_t launch_t(const LkFusedArgs& a, unsigned blocks, size_t lds, hipStream_t st, bool setup) {
    auto kfn = lkf::fused_step_kernel<WT, NCHH, NCHI, KV, G>;
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
// hidden / intermediate width, KV cache type, GQA group).
#define LKF_SHAPES(X)                        \
    X(LK_Q8_0, 1, 5, 7)  /* Qwen2.5-0.5B */  \
    X(LK_F16, 2, 3, 3)   /* SmolLM2-135M */  \
    X(LK_Q4_K, 1, 3, 8)  /* TinyLlama-1.1B */

hipError_t lk_fused_launch(const LkFusedArgs& a, uint32_t wt, int nchh, int nchi, int G, int kv_f32, unsigned blocks,
                           size_t lds, hipStream_t st, bool setup) {
#define X(T, NH, NI, GG)                                                                             \
    if (wt == T && nchh == NH && nchi == NI && G == GG) {                                            \
        return kv_f32 ? launch_t<T, NH, NI, float, GG>(a, blocks, lds, st, setup)                   \
                      : launch_t<T, NH, NI, uint16_t, GG>(a, blocks, lds, st, setup);              \
    }
    LKF_SHAPES(X)
#undef X
    return hipErrorNotSupported;
}
