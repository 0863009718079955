// batch_step.h -- arguments of the Batcher's persistent multi-row decode step
// (batch_step.hip).
#pragma once
#include "fused.h"

// Linear layers of one step, in the order a layer runs them.
enum LkBsGemm { LK_BS_QKV = 0, LK_BS_O = 1, LK_BS_GATEUP = 2, LK_BS_DOWN = 3 };

// Rows of a 128-column activation tile whose squares one linear layer's
// epilogue sums (the next RMSNorm's partial sums): h <= 128 * LK_BS_MAXT.
#define LK_BS_MAXT 16u
// Batch rows of one step (two 16-row MFMA column blocks per item).
#define LK_BS_MAX_ROWS 64u
// Arrival counters per linear layer (one per output tile), LK_ATTN_CNT_STRIDE apart.
#define LK_BS_CNT_PER_GEMM 1024u

struct LkBatchStepArgs {
    const LkFusedLayer* layers;  // device array, n_layers entries
    uint32_t n_layers;
    LkDevW embed;
    LkFreq freq;
    uint32_t h, I, nh, nkv;
    float eps;
    // the Batcher's row table: u32 [ids | pos | slots | ctx], meta_cap apart; nrows live rows
    const uint32_t* meta;
    uint32_t meta_cap, nrows;
    // the f16 KV pool: per layer [slot][kv_head][kv_seq][64]
    uint8_t* kc;
    uint8_t* vc;
    uint64_t layer_bytes;  // bytes of one layer of one cache
    uint64_t slot_elems;   // elements between two slots
    uint32_t kv_seq;
    // work buffers (f32): written and read inside the launch with agent-coherent
    // (write-through / L2-bypassing) accesses
    float* x;      // [nrows][h]: the residual stream; the final layer's rows at the end
    float* ss;     // [nrows][LK_BS_MAXT]: partial sums of squares of x per 128-column tile
    float* qkv;    // [nrows][qd + 2 kvd]: rotated q (k and v go to the cache)
    float* att;    // [nrows][qd]: attention output
    float* inner;  // [nrows][I]: SwiGLU output
    float* part;   // split-K partial tiles of the linear layers
    uint32_t* cnt; // 4 * LK_BS_CNT_PER_GEMM arrival counters, zero between uses
    uint32_t ks[4], per[4];  // per linear layer: K splits and 128-column chunks per split
    LkAttnArgs attn;  // scratch, plan and row maps of the attention phase (per-layer fields set in the kernel)
    uint64_t* bar;    // grid barrier: one tag word per workgroup (zero at first)
    uint32_t* epoch;  // launches so far (the barrier tags' high part)
    uint32_t* err;    // set when a barrier wait timed out
    // optional (null: off): block 0's s_memrealtime (100 MHz) at the start,
    // then after every barrier: 1 + 1 + 5 * n_layers entries (at most 255
    // barriers per launch: n_layers <= 50)
    uint64_t* trace;
};
inline uint32_t lk_batch_step_trace_len(uint32_t n_layers) { return 2 + 5 * n_layers; }

size_t lk_batch_step_lds_bytes();
// 16-row MFMA column blocks per linear-layer item for a step of n rows.
inline uint32_t lk_batch_step_mb(uint32_t n) { return n <= 16 ? 1u : 2u; }
// setup=true: checks the shape is instantiated, sets the LDS limit and checks one
// block per CU fits (both row-count instances); setup=false: launches.
hipError_t lk_batch_step_launch(const LkBatchStepArgs& a, uint32_t wt, int G, unsigned blocks, hipStream_t st,
                                bool setup);
