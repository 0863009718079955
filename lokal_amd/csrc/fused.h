// fused.h -- arguments of the persistent one-kernel decode step (fused.hip).
#pragma once
#include "lkhip_common.h"

struct LkFusedLayer {
    LkDevW q, k, v, o, gate, up, down;
    const float* in_norm;
    const float* post_norm;
    const float* bq;  // null when the model has no q/k/v biases
    const float* bk;
    const float* bv;
};

struct LkFusedArgs {
    const LkFusedLayer* layers;  // device array, n_layers entries
    uint32_t n_layers;
    LkDevW embed;
    const float* norm;
    LkFreq freq;
    uint32_t h, I, nh, nkv, vocab;
    float eps;
    // session state
    void* kc;            // KV cache [layer][kv_head][max_seq][64], f16 or f32
    void* vc;
    uint64_t kv_layer;   // elements per layer of one cache
    uint32_t max_seq, max_chunks;
    LkStepState* st;
    // the session's deferred lm_head (lmhead.hip, LkHeadArgs::defer): when
    // st->pending, every workgroup folds the head_blocks argmax keys (epoch
    // *head_epoch + 1) into the step state at its start; block 0 writes the
    // advanced state back at the end (pending again: this step's lm_head
    // follows), the argmax to ids_out, and advances *head_epoch.  Null
    // head_keys: no fold (a Batcher row, meta set).
    const uint64_t* head_keys;
    uint32_t head_blocks;
    uint32_t* head_epoch;
    const uint32_t* feed;
    uint32_t* ids_out;
    uint32_t* epoch;     // token counter of the exchange epochs
    uint32_t* err;       // set when a bounded wait timed out
    uint32_t* xcd_cnt;   // fused.hip: per-XCD arrival counters (LK_XCDS words, LK_XCD_CNT_STRIDE apart), zeroed
                         // once; every launch adds gridDim / LK_XCDS to each
    // exchange buffers of (f32 | epoch) words, two copies by layer parity
    uint64_t* xb;   // [2][h]        layer input x
    uint64_t* qb;   // [2][qd+2kvd]  rotated q, this token's k and v
    uint64_t* pb;   // [2][nh][max_chunks][66] attention partials of each chunk (m, l, acc[64])
    uint64_t* ab;   // [2][qd]       attention output
    uint64_t* xpb;  // [2][h]        x after the attention residual
    uint64_t* ib;   // [2][I]        SwiGLU output
    // optional stage timestamps (s_memrealtime, 100 MHz), one row of
    // lk_fused_trace_len entries per workgroup: [0] start, [1] after the
    // embedding, [2 + 6L + s] after stage s of layer L, then at the end of
    // the block
    uint64_t* trace;
    uint32_t trace_block;
    // one-kernel step (fused.hip): copies of x, the attention output and x'
    // published (1..LK_FUSED_REP); each workgroup polls copy blockIdx % rep.
    // xb, ab and xpb hold [2][LK_FUSED_REP][n] words.
    uint32_t rep;
    // Batcher rows: meta = u32 [ids | pos | slots | ...], meta_cap apart;
    // nrows live rows; slot_elems = KV elements between two slots; x_out = the
    // final layer's f32 rows [nrows][h].  fused_rows.hip reads nrows rows;
    // fused.hip, when meta is set, serves row 0 from it (token, position and
    // KV slot) instead of st and writes x_out.
    const uint32_t* meta;
    uint32_t meta_cap, nrows;
    uint64_t slot_elems;
    float* x_out;
};
// ... followed by 8 sub-steps of layer 1's attention stage (when the traced
// block runs an attention unit there).
__host__ __device__ inline uint32_t lk_fused_trace_len(uint32_t n_layers) { return 2 + 6 * n_layers + 1 + 24; }
// Shape limits of the one-kernel step: hidden width (RMSNorm gains held by
// 4 per thread) and layers (stage timestamps kept in 256 LDS slots).
#define LK_FUSED_MAX_H 2048u
#define LK_FUSED_MAX_LAYERS 38u

// LDS of one workgroup for sessions of up to max_chunks 64-position tiles.
size_t lk_fused_lds_bytes(uint32_t h, uint32_t I, uint32_t nh, uint32_t nkv, uint32_t G, uint32_t max_chunks);
// Longest session (positions) the one-kernel step serves; longer ones run the
// per-stage kernels.  A head's attention is split into at most
// LK_FUSED_MAX_CH chunks of whole attention units (lk_fused_unit; one chunk
// per lane of the merge), each chunk one wave.
#define LK_FUSED_MAX_SEQ 32768u
#define LK_FUSED_MAX_CH 64u
// Positions of the one-kernel step's attention unit (a chunk is a run of
// whole units): a 64-position cache tile, half of one with an f32 cache.
__host__ __device__ constexpr uint32_t lk_fused_unit(bool kv_f32) { return kv_f32 ? 32u : 64u; }
// Longest session of the multi-row one-kernel step (one tile per wave).
#define LK_FUSED_ROWS_MAX_SEQ 4096u
// Exchange-vector copies the single-row step's buffers are laid out for.
#define LK_FUSED_REP 8u
// XCDs of the part (a launch's workgroups are dealt to them in turn, from an
// XCD that depends on earlier launches) and the hardware register holding a
// wave's XCD id (s_getreg_b32 HW_REG_XCC_ID, bits 3:0).
#define LK_XCDS 8u
#define LK_XCD_CNT_STRIDE 64u
#define LK_HWREG_XCC_ID (20 | (0 << 6) | ((4 - 1) << 11))
// Waves per workgroup.
#define LK_FUSED_WAVES 8u

int lk_fused_threads();
// Writes the XCD id (0..15) of each workgroup of a `blocks`-workgroup launch.
hipError_t lk_xcd_probe_launch(uint32_t* out, unsigned blocks, hipStream_t st);
// The multi-row one-kernel step (fused_rows.hip): 2-7 or LK_FUSED_ROWS
// Batcher rows per launch (fewer are padded), f16 KV.
#define LK_FUSED_ROWS 8u
size_t lk_fused_rows_lds_bytes(uint32_t h, uint32_t I, uint32_t nh, uint32_t nb);
hipError_t lk_fused_rows_launch(const LkFusedArgs& a, uint32_t wt, int nchh, int nchi, int G, uint32_t nb,
                                unsigned blocks, size_t lds, hipStream_t st, bool setup);
// setup=true checks the shape is instantiated, sets the LDS limit and checks
// one block fits per CU; setup=false launches `blocks` blocks.
hipError_t lk_fused_launch(const LkFusedArgs& a, uint32_t wt, int nchh, int nchi, int G, int kv_f32, unsigned blocks,
                           size_t lds, hipStream_t st, bool setup);
