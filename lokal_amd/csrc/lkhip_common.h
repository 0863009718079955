// lkhip_common.h -- shared device helpers and launch declarations for the
// gfx950 decode kernels.  Wave size is 64 everywhere (CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define LK_WAVE 64

// Weight types as stored on the device (GGUF ids; values unchanged, layout
// repacked).  LK_Q8_SM is not a GGUF type: it is the device form of Q6_K and
// Q5_K (see LkDevW).  Q4_0 and Q5_0 are stored as LK_Q8_0.
enum LkType : uint32_t { LK_F32 = 0, LK_F16 = 1, LK_Q8_0 = 8, LK_Q4_K = 12, LK_Q8_SM = 64 };

// f16 bits -> f32, exact (IEEE conversion; what half::f16::to_f32 computes,
// src/gguf/dequant.rs:135-137).
__device__ __forceinline__ float lk_h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// A pointer as a global-memory (address space 1) pointer.  Loads through a
// generic pointer whose origin the compiler cannot see (one read from memory
// or LDS) become flat loads, which count against lgkmcnt as well as vmcnt: every
// later wait for an LDS read would then also wait for those loads to return
// from HBM.  Weight, gain and bias pointers are always device allocations.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* lk_g(const T* p) {
    return (const __attribute__((address_space(1))) T*)p;
}

// RoPE of one pair (i, i + hd/2) turned by ang = pos * theta^(-2i/hd)
// (model::rope, src/model.rs:268-279).  The inverse frequencies come from the
// host (same powf as the CPU path), so pos * f is bit-identical and only
// sinf / cosf can differ.  Products are kept unfused, as the CPU computes
// them.  Every multi-row kernel that rotates q or k calls this one.
__device__ __forceinline__ void lk_rot_pair(float& a, float& b, float ang) {
    const float s = sinf(ang), c = cosf(ang);
    const float na = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
    const float nb = __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c));
    a = na;
    b = nb;
}

// Sum of ks split-K partials p[z * stride], z = 0..ks-1, added in split
// order (bit-identical to the plain loop).  The loads go out W at a time
// (clamped in-range addresses, unused values dropped by a select), so a
// thread waits one memory round trip per W splits, not one per split (a
// runtime-count loop of dependent adds is issued load by load); W is the
// smallest of 2, 4, 8, 16 that covers ks (a uniform branch), so few splits
// do not issue 16 loads each.
template <int W>
__device__ __forceinline__ float lk_sum_splits_w(const float* __restrict__ p, size_t stride, uint32_t ks) {
    float a = 0.f;
    for (uint32_t z0 = 0; z0 < ks; z0 += W) {
        float t[W];
#pragma unroll
        for (uint32_t j = 0; j < W; j++) t[j] = p[(size_t)(z0 + j < ks ? z0 + j : z0) * stride];
#pragma unroll
        for (uint32_t j = 0; j < W; j++) a = z0 + j < ks ? a + t[j] : a;
    }
    return a;
}
__device__ __forceinline__ float lk_sum_splits(const float* __restrict__ p, size_t stride, uint32_t ks) {
    if (ks <= 2) return lk_sum_splits_w<2>(p, stride, ks);
    if (ks <= 4) return lk_sum_splits_w<4>(p, stride, ks);
    if (ks <= 8) return lk_sum_splits_w<8>(p, stride, ks);
    return lk_sum_splits_w<16>(p, stride, ks);
}

// Wave-64 reductions on the DPP network (no LDS round trips): quad_perm
// pairs, row_ror 4 / 8 give every lane its 16-lane row total, row_bcast 15 /
// 31 carry the row totals up to lane 63, whose value is broadcast.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float lk_dpp(float v, float old) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                   __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF,
                                                                   false));
}
__device__ __forceinline__ float lk_wave_sum(float v) {
    v += lk_dpp<0xB1, 0xF>(v, 0.f);   // quad_perm [1,0,3,2]
    v += lk_dpp<0x4E, 0xF>(v, 0.f);   // quad_perm [2,3,0,1]
    v += lk_dpp<0x124, 0xF>(v, 0.f);  // row_ror 4
    v += lk_dpp<0x128, 0xF>(v, 0.f);  // row_ror 8
    v += lk_dpp<0x142, 0xA>(v, 0.f);  // row_bcast 15
    v += lk_dpp<0x143, 0xC>(v, 0.f);  // row_bcast 31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float lk_wave_max(float v) {
    const float ninf = -INFINITY;
    v = fmaxf(v, lk_dpp<0xB1, 0xF>(v, ninf));
    v = fmaxf(v, lk_dpp<0x4E, 0xF>(v, ninf));
    v = fmaxf(v, lk_dpp<0x124, 0xF>(v, ninf));
    v = fmaxf(v, lk_dpp<0x128, 0xF>(v, ninf));
    v = fmaxf(v, lk_dpp<0x142, 0xA>(v, ninf));
    v = fmaxf(v, lk_dpp<0x143, 0xC>(v, ninf));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Sum over the four lanes {l, l^8, l^16 .. within one 32-lane half}: row_ror 8
// then an xor-16 swizzle.  Lane l of each half then holds the sum of the four
// lanes of that half with the same (l & 7).
__device__ __forceinline__ float lk_half_sum_mod8(float v) {
    v += lk_dpp<0x128, 0xF>(v, 0.f);
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    return v;
}

// A float made order-preserving as an unsigned key; the argmax key packs it
// above the inverted index so that max(key) = (largest value, smallest index),
// which is the "first max wins" rule of src/sampler.rs:67-75.
__device__ __forceinline__ uint64_t lk_argmax_key(float v, uint32_t idx) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)b << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ uint32_t lk_argmax_idx(uint64_t key) { return 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu); }

// A device weight matrix, repacked at upload (values unchanged):
//   F16  : data = half  [rows][cols]
//   Q8_0 : data = int8  [rows][cols]          aux = half [rows][cols/32]  (block scales d)
//   Q4_K : data = uint8 [rows][cols/256][128] aux = uint8 [rows][cols/256][16]
//          (aux = the super-block head: d, dmin f16 + 12 packed 6-bit scale/min bytes)
//   Q8_SM: data = int8  [rows][cols]          aux = float2 [rows][cols/16]  (s, m per 16)
//          y = s*q - m, the product rounded before the subtraction.  Q6_K
//          (y = (d*sc)*q, src/gguf/dequant.rs:510-533) stores s = d*sc, m = 0;
//          Q5_K (y = d1*q - m1, :484-509) stores s = d1, m = m1.  Both
//          products d*sc, dmin*m of an f16 and a 6/8-bit integer are exact in
//          f32, so the stored pair reproduces the reference's values bit for bit.
struct LkDevW {
    uint32_t type;
    uint32_t rows, cols;
    const uint8_t* data;
    const uint8_t* aux;
};

// One output segment of a fused matvec launch (Q, K and V share one launch;
// gate and up share one launch).
struct LkSeg {
    LkDevW w;
    const float* bias;
    float* out;
};

enum LkMvMode : int {
    LK_MV_STORE = 0,   // out = W x (+ b)
    LK_MV_ACC = 1,     // out += W x (+ b)       (residual add)
    LK_MV_SWIGLU = 2,  // out = silu(W0 x) * (W1 x)  with seg[0] = gate, seg[1] = up
    LK_MV_ARGMAX = 3   // out = W x, and per-block (max, first index) key into keys[blockIdx]
};

struct LkMvArgs {
    LkSeg seg[3];
    uint32_t nseg;
    uint32_t total_rows;   // rows over all segments (SWIGLU: rows of one)
    uint32_t cols;
    const float* x;
    uint64_t* keys;        // ARGMAX partial keys, one per block
};

// Host-side launchers (matvec.hip).
struct LkMvPlan {
    int rows_per_wave;
    int nch;
    unsigned blocks;
};
LkMvPlan lk_matvec_plan(uint32_t type, uint32_t total_rows, uint32_t cols, int mode);
hipError_t lk_matvec_launch(const LkMvArgs& a, int mode, hipStream_t st, LkMvPlan* plan_out = nullptr);
hipError_t lk_dequant_launch(const LkDevW& w, uint32_t row0, uint32_t nrows, float* out, hipStream_t st);
hipError_t lk_gather_launch(const LkDevW& table, const uint32_t* ids, uint32_t n_ids, float* out, hipStream_t st);

// Layer kernels (layer.hip).
hipError_t lk_rmsnorm_launch(const float* x, const float* w, uint32_t rows, uint32_t n, float eps, float* y,
                             hipStream_t st);
// RoPE inverse frequencies theta^(-2i/hd), computed on the host with the
// same powf the CPU path calls (src/model.rs:273) and passed by value.
struct LkFreq {
    float f[64];
};
hipError_t lk_rope_launch(float* x, uint32_t rows, uint32_t n, uint32_t head_dim, const uint32_t* pos,
                          const LkFreq& freq, hipStream_t st);
hipError_t lk_swiglu_launch(const float* g, const float* u, uint32_t n, float* out, hipStream_t st);
hipError_t lk_argmax_rows_launch(const float* x, uint32_t rows, uint32_t n, uint32_t* out, hipStream_t st);

// Decode-step glue kernels (layer.hip).
struct LkStepState {
    uint32_t token;   // token fed at this step
    uint32_t pos;     // position of this step
    uint32_t n_out;   // argmax ids written so far
    uint32_t n_feed;  // prompt ids still to feed before argmax takes over
    uint32_t fed;     // prompt ids fed so far
    // 1 when the last step's lm_head launch published its per-block argmax
    // keys without folding them (LkHeadArgs::defer): the state above is that
    // step's, and whoever reads it next (the one-kernel step's start, or
    // lk_head_finish) folds the keys and advances it first
    uint32_t pending;
    uint32_t pad[2];
};
static_assert(sizeof(LkStepState) == 32, "read as two 16-byte words");

// The lm_head's per-block argmax keys (lk_argmax_key), each published as two
// words (epoch | high half) and (epoch | low half): a word carrying the
// launch's epoch is that launch's, so the buffer never needs clearing.
// Thread t of nt folds blocks t, t + nt, ... of n; ok turns false if a word
// does not carry ep (read after the launch ended, every word must).
__device__ __forceinline__ uint64_t lk_head_keys_fold(const uint64_t* keys, uint32_t n, uint32_t ep, uint32_t t,
                                                      uint32_t nt, bool& ok) {
    uint64_t best = 0;
    for (uint32_t i = t; i < n; i += nt) {
        const uint64_t hi = __hip_atomic_load(keys + 2 * i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t lo = __hip_atomic_load(keys + 2 * i + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok &= (uint32_t)(hi >> 32) == ep && (uint32_t)(lo >> 32) == ep;
        const uint64_t k = (hi << 32) | (lo & 0xFFFFFFFFu);
        best = k > best ? k : best;
    }
    return best;
}
// The greedy loop's step advance (src/generate.rs:101-118 at -t 0): feed the
// next prompt id while any are left, else take the argmax (writing it to
// ids_out, if given); the position moves on by one.
__device__ __forceinline__ void lk_step_advance(uint32_t& token, uint32_t& pos, uint32_t& n_out, uint32_t& n_feed,
                                                uint32_t& fed, uint32_t best, const uint32_t* feed,
                                                uint32_t* ids_out, bool write_id) {
    if (n_feed > 0) {
        token = feed[fed];
        fed += 1;
        n_feed -= 1;
    } else {
        if (ids_out && write_id) ids_out[n_out] = best;
        n_out += 1;
        token = best;
    }
    pos += 1;
}
hipError_t lk_embed_step_launch(const LkDevW& table, const LkStepState* st_dev, float* x, hipStream_t st);
hipError_t lk_rope_kv_launch(float* qkv, uint32_t n_heads, uint32_t n_kv, const LkFreq& freq,
                             const LkStepState* st_dev, const uint32_t* pos_rows, uint32_t n_rows,
                             void* kcache, void* vcache, int kv_f32, uint32_t max_seq, uint64_t slot_stride,
                             const uint32_t* slots, hipStream_t st);
hipError_t lk_step_finish_launch(const uint64_t* keys, uint32_t n_keys, LkStepState* st_dev,
                                 const uint32_t* feed_ids, uint32_t* ids_out, hipStream_t st);

// End of a decode step in one launch (lmhead.hip): final RMSNorm, lm_head,
// argmax, step-state advance.
#define LK_HEAD_MAX_BLOCKS 1024u
struct LkHeadArgs {
    const float* x;      // residual stream before the final norm
    uint32_t x_stride;   // floats between elements (2: f32 halves of (f32 | epoch) words)
    const float* norm;
    float eps;
    LkDevW w;
    uint32_t h, vocab;
    float* logits;
    uint64_t* keys;      // 2 * LK_HEAD_MAX_BLOCKS words of (epoch | key half)
    uint32_t* epoch;     // launches so far (advanced by block 0)
    uint32_t* err;       // set to 2 if the key wait timed out
    LkStepState* st;
    const uint32_t* feed;
    uint32_t* ids_out;
    // 1: every block publishes its key and the launch ends there; the state
    // is left pending (the one-kernel step that follows folds the keys, or
    // lk_head_finish does).  0: block 0 collects the keys and advances the
    // state itself.
    uint32_t defer;
};
// lm_head rows of up to 256 16-byte chunks (Q8_0: h <= 4096, F16: 2048, Q4_K: 8192)
bool lk_lm_head_fits(uint32_t type, uint32_t h);
uint32_t lk_lm_head_rows(uint32_t type, uint32_t h);
uint32_t lk_lm_head_blocks(uint32_t vocab, uint32_t type, uint32_t h);
hipError_t lk_lm_head_launch(const LkHeadArgs& a, uint32_t blocks, hipStream_t st);
// The final norm and lm_head of 1..LK_HEAD_ROWS_MAX rows (rows of a.x h floats
// apart) into logits rows a.vocab floats apart; no argmax, nothing deferred
// (a.keys, a.epoch, a.st unused).
#define LK_HEAD_ROWS_MAX 2u
bool lk_lm_head_rows_fits(uint32_t type, uint32_t h, uint32_t nrows);
hipError_t lk_lm_head_rows_launch(const LkHeadArgs& a, uint32_t nrows, uint32_t blocks, hipStream_t st);
// Folds the keys of a deferred lm_head launch of `blocks` blocks into the
// state (if it is pending) and advances the key epoch: the end of a run of
// one-kernel steps.  One small launch.
hipError_t lk_head_finish_launch(const LkHeadArgs& a, uint32_t blocks, hipStream_t st);

// Attention (attention.hip).  q rows of n_heads*64, caches f16
// [seq][n_kv][max_seq][64]; ctx from ctx_len[seq] or, when null, st_dev->pos+1.
struct LkAttnArgs {
    const float* q;
    const void* k;          // f16 (uint16 bits) or f32 elements, see kv_f32
    const void* v;
    float* out;
    float* part;            // scratch: [seq][n_heads][max_chunks][2 + 64]
    uint32_t* cnt;          // [seq][n_kv] chunk arrival counters, zero between launches
    const uint32_t* ctx_len;
    const LkStepState* st;  // decode step state (single sequence, graph mode)
    const uint32_t* slots;  // optional row -> cache slot map
    uint32_t n_seq, n_heads, n_kv, max_seq;
    uint64_t seq_stride;    // elements between two slots of the cache
    uint64_t q_stride;      // floats between two sequences' q rows (out rows are n_heads * 64 apart)
    uint32_t kv_f32;        // 1: the cache holds f32, 0: f16
    uint32_t waves, tiles, cstride;  // set by lk_attn_launch: its chunk plan and partial slots per head
    // 1: rows i, i+1, ... are consecutive positions of one sequence (a
    // prefill chunk: one slot, ctx_len[i] + 1 == ctx_len[i + 1]), so an item
    // may take several rows at once (f16 cache, matrix-core kernel)
    uint32_t grouped;
    // rope != 0 (one row per item): q and each row's own k / v are not rotated
    // or appended yet.  The launch sums the QKV GEMM's split-K partials
    // (rope_part, [rope_ks][n_seq][q_stride]; rope_ks == 0: q already holds
    // the bias-added sums) plus bq / bk / bv, turns q and k by RoPE at the
    // row's position ctx_len - 1 (= pos_rows), and the block whose chunk holds
    // that position writes the row's k / v to the cache and uses them -- the
    // work of rows_rope_kv_kernel, which lk_attn_launch runs first instead
    // when its kernel for the call is not the one-row f16 matrix-core one.
    uint32_t rope, rope_ks;
    const float* rope_part;
    const float *bq, *bk, *bv;
    const uint32_t* pos_rows;
    LkFreq freq;
};
uint32_t lk_attn_chunk(uint32_t max_seq);
// Sets a's chunk plan (waves, tiles, cstride) for its n_seq, n_kv and
// max_seq, as lk_attn_launch does; returns the chunks per (sequence, kv head).
uint32_t lk_attn_set_plan(LkAttnArgs& a);
size_t lk_attn_part_floats(uint32_t n_seq, uint32_t n_heads, uint32_t max_seq);
// A launch's scratch buffer: a region of cnt_cap arrival counters (u32,
// one per (sequence, kv head), n_seq * n_kv <= cnt_cap) that must be zero
// before the buffer's first launch -- every launch leaves them zero -- then
// the partials.  The counters sit at a fixed place whatever the shape, so
// launches of different shapes on one buffer never see a partial as a count.
#ifndef LK_ATTN_CNT_STRIDE
#define LK_ATTN_CNT_STRIDE 64u  // words between two counters: each in its own 256-byte line
#endif
inline size_t lk_attn_cnt_region(size_t cnt_cap) { return cnt_cap * LK_ATTN_CNT_STRIDE; }
inline size_t lk_attn_scratch_floats(uint32_t n_seq, uint32_t n_heads, uint32_t max_seq, size_t cnt_cap) {
    return lk_attn_cnt_region(cnt_cap) + lk_attn_part_floats(n_seq, n_heads, max_seq);
}
inline void lk_attn_bind_scratch(LkAttnArgs& a, float* buf, size_t cnt_cap) {
    a.cnt = (uint32_t*)buf;
    a.part = buf + lk_attn_cnt_region(cnt_cap);
}
// Counter words reserved in the no-allocation entry point's fixed buffer.
#define LK_ATTN_SCRATCH_CNT 1024u
hipError_t lk_attn_launch(const LkAttnArgs& a, hipStream_t st);
// The fixed partial buffer of the no-allocation attention entry point:
// LK_ATTN_SCRATCH_FLOATS floats (8 MiB) per device; lk_attn_scratch gives
// the current device's address (looked up once per device).
#define LK_ATTN_SCRATCH_FLOATS (2u << 20)
hipError_t lk_attn_scratch(float** out);

// Multi-row dequant-fused GEMM (gemm.hip): Y[b][n] = sum_k X[b][k] W[n][k]
// for b < n_rows, the B-row form of the matvec (Linear::forward over a batch
// of tokens, src/model.rs:27-35).  Segments split N as in LkMvArgs (QKV); in
// LK_MV_SWIGLU mode seg[0] is gate and seg[1] up, both N rows, and seg[0].out
// receives silu(gate) * up.  Output row stride ldy (floats), input ldx.
struct LkGemmArgs {
    LkSeg seg[3];
    uint32_t nseg;
    uint32_t N;        // output units over all segments (SWIGLU: rows of one)
    uint32_t K;
    uint32_t n_rows;   // batch rows B
    const float* x;
    uint32_t ldx, ldy;
    float* part;       // split-K partials [ks][n_rows][N or 2N]
    uint32_t ks;       // K splits (1: the epilogue runs in the GEMM kernel)
};
// Plan: K splits for a launch and the partial floats it needs.
struct LkGemmPlan {
    uint32_t ks;
    uint32_t mb;       // 16-row batch tiles per wave (1 or 2)
    size_t part_floats;
};
LkGemmPlan lk_gemm_plan(uint32_t type, uint32_t N, uint32_t K, uint32_t n_rows, int mode);
// Checks the shape the GEMM assumes: N a multiple of 16 per segment, K of 32.
bool lk_gemm_shape_ok(uint32_t type, uint32_t N, uint32_t K);
// deferred_ks != null: a split launch leaves its partials [ks][n_rows][N] in
// a.part for the consumer to sum (*deferred_ks = ks, 0 when not split, in
// which case the epilogue already ran); the consumer applies bias / residual.
hipError_t lk_gemm_launch(LkGemmArgs a, int mode, hipStream_t st, uint32_t* deferred_ks = nullptr);
// Rows-path consumers of deferred split-K partials (layer.hip):
//  x[r] += sum_z part[z][r] (ks > 0), then y[r] = rmsnorm(x[r]) * w
hipError_t lk_rows_accnorm_launch(float* x, const float* part, uint32_t ks, uint32_t rows, uint32_t n,
                                  const float* w, float eps, float* y, hipStream_t st);
//  qkv[r] = sum_z part[z][r] + bias (ks > 0), then the rope_kv work of
//  lk_rope_kv_launch (rotated q back into qkv, k/v into the cache)
hipError_t lk_rows_rope_kv_launch(float* qkv, const float* part, uint32_t ks, const float* bq, const float* bk,
                                  const float* bv, uint32_t n_heads, uint32_t n_kv, const LkFreq& freq,
                                  const uint32_t* pos_rows, uint32_t n_rows, void* kcache, void* vcache, int kv_f32,
                                  uint32_t max_seq, uint64_t slot_stride, const uint32_t* slots, hipStream_t st);
//  greedy step of every row in two passes: per-slice argmax keys, then fold
hipError_t lk_rows_greedy2_launch(const float* logits, uint32_t n_rows, uint32_t n, uint64_t* keys, uint32_t* meta,
                                  uint32_t cap, uint32_t* out_ids, hipStream_t st);
#define LK_ARGMAX_SLICE 4096u
