/*
 * lokal_hip.h -- C ABI of the MI355X (gfx950) decode backend for lokal.
 *
 * The boundary is lokal's backend seam, src/engine.rs:13-71 (Engine, Session,
 * Batcher, BatchRow) plus the quantized-GGUF constructor create_metal_quant
 * (src/engine.rs:150-162).  Every function returns 0 on success or a negative
 * LKHIP_E* code; lkhip_last_error() then holds a one-line, thread-local reason
 * in the reference's refusal style (src/engine.rs:105-109, src/main.rs:326-355).
 *
 * Ownership: the caller owns every host buffer passed in or out.  Sessions and
 * batches borrow their engine (Session<'_> in src/engine.rs:18) and must be
 * destroyed before it.  An engine is safe to share across threads for session
 * creation; a session or batch is single-threaded and owns its HIP stream.
 *
 * Pointer kinds: functions under "engine / session / batch" take HOST pointers.
 * The kernel-level functions under "kernels" take DEVICE pointers (from
 * lkhip_malloc) and a stream (NULL = the null stream) and do not synchronise.
 */
#ifndef LOKAL_HIP_H
#define LOKAL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    LKHIP_OK = 0,
    LKHIP_E_INVALID = -1,     /* bad argument / shape */
    LKHIP_E_UNSUPPORTED = -2, /* refused: type or shape this backend does not run */
    LKHIP_E_HIP = -3,         /* HIP runtime error */
    LKHIP_E_NOMEM = -4,       /* allocation failed */
    LKHIP_E_IO = -5           /* file could not be read / parsed */
};

/* GGUF tensor type ids (enum ggml_type), src/gguf/dequant.rs:21-40. */
enum {
    LKHIP_F32 = 0,
    LKHIP_F16 = 1,
    LKHIP_Q4_0 = 2,
    LKHIP_Q5_0 = 6,
    LKHIP_Q8_0 = 8,
    LKHIP_Q4_K = 12,
    LKHIP_Q5_K = 13,
    LKHIP_Q6_K = 14
};

/* ModelConfig, src/config.rs:10-30 (the fields the decode step reads).
 * head_dim 0 means hidden_size / num_attention_heads (config.rs:92-95). */
typedef struct lkhip_config {
    uint32_t hidden_size;
    uint32_t intermediate_size;
    uint32_t num_hidden_layers;
    uint32_t num_attention_heads;
    uint32_t num_key_value_heads;
    uint32_t vocab_size;
    uint32_t head_dim;
    uint32_t max_position_embeddings;
    float rms_norm_eps;
    float rope_theta;
} lkhip_config;

/* One named tensor as a TensorStore / GGUF tensor hands it over
 * (src/weights.rs:77-97, src/gguf/dequant.rs:129-133): HF name, GGUF type id,
 * row-major dims [rows, cols] (n_dims 1 => [cols]), raw little-endian bytes. */
typedef struct lkhip_tensor {
    const char* name;
    uint32_t ggml_type;
    uint32_t n_dims;
    uint64_t dims[2];
    const void* data;
    uint64_t nbytes;
} lkhip_tensor;

/* BatchRow, src/engine.rs:30-34. */
typedef struct lkhip_row {
    uint32_t token;
    uint32_t slot;
    uint64_t pos;
} lkhip_row;

/* Per-session kernel timing, summed over every forward since the last reset
 * (the HIP counterpart of LOKAL_GPU_TIMING's phase table, src/gpu/metal.rs:3856-3952). */
typedef struct lkhip_profile {
    uint64_t tokens;           /* forwards timed */
    uint64_t matvec_launches;  /* dequant-matvec kernel launches */
    double matvec_ms;          /* summed hipEvent time of those launches */
    double matvec_bytes;       /* algorithmic weight bytes they read */
    uint64_t lm_head_launches;
    double lm_head_ms;         /* the single largest matvec, lm_head */
    double lm_head_bytes;
    double attn_ms;            /* flash-decoding attention: one launch per layer, partials folded in-kernel */
    double other_ms;           /* norms, rope, gather, argmax */
} lkhip_profile;

typedef struct lkhip_engine lkhip_engine;
typedef struct lkhip_session lkhip_session;
typedef struct lkhip_batch lkhip_batch;
typedef struct lkhip_weight lkhip_weight;

/* ------------------------------------------------------------- general */

/* Thread-local reason for the last failure on this thread ("" if none). */
const char* lkhip_last_error(void);
/* Number of visible HIP devices (0 with no GPU; never fails). */
int lkhip_device_count(void);
/* Library version string. */
const char* lkhip_version(void);

/* ------------------------------------------------- engine / session */

/* Engine from named tensors (HF names as src/model.rs:160-186 reads them):
 * weights upload once and stay resident (src/gpu/mod.rs:9-10).  Linear
 * weights may be F16, Q8_0 or Q4_K; norms and biases F32 (or F16).  A missing
 * lm_head.weight ties it to model.embed_tokens.weight (src/model.rs:181-186).
 * llama_permuted != 0 undoes llama.cpp's q/k row permute at upload
 * (src/gguf/arch.rs:274-286, applied as in src/gguf/dequant.rs:548-553).
 * Replaces engine::create (src/engine.rs:76-111) for the "hip" backend. */
int lkhip_engine_create_tensors(const lkhip_config* cfg, const lkhip_tensor* tensors, size_t n_tensors,
                                int llama_permuted, lkhip_engine** out);
/* Engine straight from a GGUF v2/v3 file; weights stay quantized on device.
 * Replaces create_metal_quant (src/engine.rs:150-162) / MetalEngine::new_gguf_quant
 * (src/gpu/metal.rs:1667); config from GGUF metadata as gguf::model_config does
 * (src/gguf/arch.rs:164-223). */
int lkhip_engine_create_gguf(const char* path, lkhip_engine** out);
/* The --context-window contract of the "hip" arm.  engine::create and
 * create_metal_quant take win: Option<(window, sink)> (src/engine.rs:76-87,
 * :150-162, built in src/main.rs:159-162); this backend keeps every position's
 * K/V resident in HBM and has no sliding window, so, like the CPU arm
 * (src/engine.rs:84-87), it refuses one: window == 0 (None) returns LKHIP_OK,
 * any other value LKHIP_E_UNSUPPORTED with a one-line reason naming the
 * backends that window.  No device needed. */
int lkhip_context_window(size_t window, size_t sink);
/* Parses a GGUF file's header and tensor table only (no device needed): the
 * config lkhip_engine_create_gguf would build (gguf::model_config,
 * src/gguf/arch.rs:164-227), the number of tensors the decode step reads
 * (hf_name, src/gguf/arch.rs:229-270) and whether q/k rows carry the llama
 * converter's permutation (load_f32, src/gguf/dequant.rs:538-557).  Errors
 * as GgufFile::open reports them (src/gguf/container.rs:162-261). */
int lkhip_gguf_config(const char* path, lkhip_config* cfg_out, size_t* n_tensors_out, int* llama_permuted_out);
void lkhip_engine_destroy(lkhip_engine* e);
/* Engine::config (src/engine.rs:15). */
int lkhip_engine_config(const lkhip_engine* e, lkhip_config* out);
/* Algorithmic bytes of every weight one decode token reads (matvecs only). */
double lkhip_engine_matvec_bytes(const lkhip_engine* e);

/* Engine::session (src/engine.rs:17): KV cache (f16, on device) for max_seq positions. */
int lkhip_session_create(lkhip_engine* e, size_t max_seq, lkhip_session** out);
/* Same with the KV cache element type chosen: LKHIP_F16 (the GPU path's
 * format, src/gpu/metal.rs:3234-3235; what lkhip_session_create uses) or
 * LKHIP_F32 (the CPU path's format, src/model.rs:114-128). */
int lkhip_session_create_ex(lkhip_engine* e, size_t max_seq, uint32_t kv_type, lkhip_session** out);
void lkhip_session_destroy(lkhip_session* s);
/* Session::forward (src/engine.rs:51): one token at pos -> vocab logits (host). */
int lkhip_session_forward(lkhip_session* s, uint32_t token, size_t pos, float* logits_out);
/* Session::prefill (src/engine.rs:56-62): the chunked multi-row pass (up to
 * 512 positions per pass, each linear layer one GEMM reading its weights once),
 * within 1e-3 of lokal's token loop; LKHIP_PREFILL=loop runs the token loop
 * instead (bit-identical to forward).  Logits of the last position into
 * logits_out (may be NULL). */
int lkhip_session_prefill(lkhip_session* s, const uint32_t* ids, size_t n, float* logits_out);
/* Session::forward_batch (src/engine.rs:67-70): logits for every position,
 * n * vocab floats. */
int lkhip_session_forward_batch(lkhip_session* s, const uint32_t* ids, size_t n, size_t pos0, float* logits_out);
/* The greedy decode loop of generate.rs:101-118 at -t 0 (argmax, first max
 * wins, src/sampler.rs:67-75), run on the device: feeds `token` at `pos`, then
 * feeds each argmax back, n_steps times; writes the n_steps argmax ids.  No
 * host round trip per token.  logits_last (may be NULL) gets the final logits. */
int lkhip_session_decode_greedy(lkhip_session* s, uint32_t token, size_t pos, size_t n_steps, uint32_t* ids_out,
                                float* logits_last);
/* Read back one layer's KV cache row at pos as f32 (kv_dim values), from the
 * session's f16 or f32 cache (lkhip_session_create_ex's kv_type). */
int lkhip_session_read_kv(lkhip_session* s, uint32_t layer, size_t pos, int which_v, float* out);
/* Rows pos0..pos0+n-1 of the same cache, out[n][kv_dim] as f32.  A read-back
 * for tests and debugging, as read_kv; lokal's KvCache exposes its buffers the
 * same way (src/model.rs:114-128). */
int lkhip_session_read_kv_rows(lkhip_session* s, uint32_t layer, size_t pos0, size_t n, int which_v, float* out);
/* Kernel timing: on != 0 brackets every launch with hipEvents (eager launches,
 * no graph) until switched off; profile_get sums since the last reset. */
int lkhip_session_set_profiling(lkhip_session* s, int on);
int lkhip_session_profile(lkhip_session* s, lkhip_profile* out, int reset);
/* Stage timeline of the one-kernel decode step (the phase table of
 * LOKAL_GPU_TIMING, src/gpu/metal.rs:3994-4270): block >= 0 starts recording,
 * for EVERY workgroup, a 100 MHz timestamp at the start, after the embedding,
 * after each of the 6 stages of every layer and at the end, followed by 24
 * sub-step marks of layer 1 (2 + 6*layers + 1 + 24 entries per workgroup);
 * `block` names the workgroup stage_times-style summaries report; block < 0
 * stops recording.  lkhip_session_trace copies the last step's timestamps,
 * [workgroup][entries]; lkhip_session_trace_len gives their number (0 when
 * tracing is off). */
int lkhip_session_set_trace(lkhip_session* s, int block);
int lkhip_session_trace(lkhip_session* s, uint64_t* ticks, size_t n);
size_t lkhip_session_trace_len(const lkhip_session* s);

/* Engine::batcher (src/engine.rs:23-26): n_slots KV slots of max_seq positions,
 * pool laid out per layer as [slot][kv_head][max_seq][head_dim] f16. */
int lkhip_batch_create(lkhip_engine* e, size_t n_slots, size_t max_seq, lkhip_batch** out);
void lkhip_batch_destroy(lkhip_batch* b);
/* Batcher::prefill (src/engine.rs:44): fill one slot with a prompt. */
int lkhip_batch_prefill(lkhip_batch* b, uint32_t slot, const uint32_t* ids, size_t n, float* logits_out);
/* Batcher::decode_step (src/engine.rs:46): one token per row; one weight read
 * serves every row.  logits_out holds n_rows * vocab floats, in row order. */
int lkhip_batch_decode_step(lkhip_batch* b, const lkhip_row* rows, size_t n_rows, float* logits_out);
/* The serve loop's greedy decode over a batch (generate.rs:101-118 at -t 0 per
 * row, with Batcher::decode_step as the step, src/engine.rs:46): feeds each
 * row's token at its pos, then each row's argmax back, n_steps times, all on
 * the device; ids_out is n_steps * n_rows ids, step-major.  n_rows <= 64. */
int lkhip_batch_decode_greedy(lkhip_batch* b, const lkhip_row* rows, size_t n_rows, size_t n_steps,
                              uint32_t* ids_out);
/* Rows pos0..pos0+n-1 of one slot's f16 KV cache at one layer, out[n][kv_dim]
 * as f32: a read-back of MetalBatcher's per-slot pool for tests
 * (src/gpu/metal.rs:3557-3565). */
int lkhip_batch_read_kv_rows(lkhip_batch* b, uint32_t slot, uint32_t layer, size_t pos0, size_t n, int which_v,
                             float* out);
/* Phase timeline of the last persistent multi-row step (the Batcher's
 * one-launch step for several rows): s_memrealtime ticks (100 MHz) of its
 * first workgroup at the start and after each grid barrier (the embedding,
 * then q/k/v, attention, o_proj, gate/up, down of every layer).  Recorded
 * only when LKHIP_BSTEP_TRACE=1 was set when the batcher was created; the
 * counterpart of lkhip_session_trace, for the per-phase times of
 * LOKAL_GPU_TIMING's table (src/gpu/metal.rs:3856-3952). */
size_t lkhip_batch_trace_len(const lkhip_batch* b);
int lkhip_batch_trace(lkhip_batch* b, uint64_t* ticks, size_t n);

/* ------------------------------------------------------------ memory */

int lkhip_malloc(void** dptr, size_t bytes);
int lkhip_free(void* dptr);
int lkhip_memcpy_htod(void* dst, const void* src, size_t bytes);
int lkhip_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int lkhip_memcpy_dtod(void* dst, const void* src, size_t bytes);
int lkhip_memset(void* dptr, int value, size_t bytes);
int lkhip_synchronize(void);
/* Streams at default priority and events for timing kernel-level calls. */
int lkhip_stream_create(void** stream);
int lkhip_stream_destroy(void* stream);
int lkhip_stream_synchronize(void* stream);
int lkhip_event_create(void** ev);
int lkhip_event_destroy(void* ev);
int lkhip_event_record(void* ev, void* stream);
int lkhip_event_elapsed_ms(void* start, void* stop, float* ms);

/* ----------------------------------------------------------- kernels */

/* A weight matrix uploaded once in its GGUF type and repacked for the device
 * (values unchanged).  type F16, Q8_0, Q4_0, Q5_0, Q4_K, Q5_K or Q6_K; host
 * bytes are GGUF rows (src/gguf/dequant.rs:191-535 reads the same bytes).
 * Q4_0 / Q5_0 are stored as int8 + f16 scale, Q5_K / Q6_K as int8 + an f32
 * (scale, min) pair per 16 values: the same values at 1.06 / 1.5 device bytes
 * per weight. */
int lkhip_weight_create(uint32_t ggml_type, size_t rows, size_t cols, const void* host_bytes, size_t nbytes,
                        lkhip_weight** out);
void lkhip_weight_destroy(lkhip_weight* w);
/* Algorithmic bytes of the weight in its GGUF type. */
double lkhip_weight_bytes(const lkhip_weight* w);

/* dequant_row_ref (src/gguf/dequant.rs:191-535) for rows [row0, row0+n_rows):
 * out is n_rows * cols f32, bit-exact with the CPU dequant. */
int lkhip_dequant_rows(const lkhip_weight* w, size_t row0, size_t n_rows, float* out, void* stream);
/* Linear::forward (src/model.rs:27-35) with the weight dequantized in the load:
 * y[o] = dot(W[o,:], x) (+ bias[o]); accumulate != 0 adds into y instead
 * (the residual add of src/model.rs:235-237, :253-255).  fp32 accumulation. */
int lkhip_matvec(const lkhip_weight* w, const float* x, const float* bias, float* y, int accumulate, void* stream);
/* Typed forms of lkhip_matvec that refuse any other weight type. */
int lkhip_q8_0_matvec(const lkhip_weight* w, const float* x, const float* bias, float* y, int accumulate,
                      void* stream);
int lkhip_q4_k_matvec(const lkhip_weight* w, const float* x, const float* bias, float* y, int accumulate,
                      void* stream);
/* Linear::forward over n_rows activation rows (the multi-row GEMM of the
 * batched path; lokal's Metal backend runs this as matmul_pg,
 * src/gpu/kernels.metal:1749-1985): y[r*ldy + o] = dot(W[o,:], x[r*ldx ..])
 * (+ bias[o]), or += with accumulate.  fp32 accumulation on the matrix cores.
 * Needs cols % 32 == 0 (Q4_K: % 256), ldx % 4 == 0 and a 16-byte aligned x. */
int lkhip_matmul(const lkhip_weight* w, const float* x, size_t n_rows, size_t ldx, const float* bias, float* y,
                 size_t ldy, int accumulate, void* stream);
/* math::rmsnorm (src/math.rs:45-49) over n_rows rows of n: y = x*s*w. */
int lkhip_rmsnorm(const float* x, const float* w, size_t n_rows, size_t n, float eps, float* y, void* stream);
/* model::rope (src/model.rs:268-279) in place on n_rows rows of n floats
 * (n a multiple of head_dim); row r rotates at position pos[r] (device u32). */
int lkhip_rope_pairs(float* x, size_t n_rows, size_t n, size_t head_dim, const uint32_t* pos, float theta,
                     void* stream);
/* SwiGLU of src/model.rs:247-249 with math::silu (src/math.rs:68-70):
 * out[i] = silu(g[i]) * u[i], n elements. */
int lkhip_swiglu(const float* g, const float* u, size_t n, float* out, void* stream);
/* Embedding lookup, src/model.rs:200-202: out[r,:] = f32(table[ids[r],:]) for
 * n_ids ids (device u32); the table is a weight of any supported type. */
int lkhip_embed_gather(const lkhip_weight* table, const uint32_t* ids, size_t n_ids, float* out, void* stream);
/* model::attention (src/model.rs:286-318) by flash-decoding for n_seq
 * independent sequences, one query token each.  q: [n_seq][n_heads*head_dim]
 * f32; k_cache/v_cache: f16 [n_seq][n_kv_heads][max_seq][head_dim]; ctx_len
 * (device u32, n_seq) = positions 0..ctx_len-1 are live; out like q.
 * head_dim must be 64; n_heads a multiple of n_kv_heads, group <= 8.
 * One launch: chunk partials and the fold in the same kernel, with a scratch
 * buffer (arrival counters + partials) cached per calling thread and grown on
 * demand; calls from one thread on different streams share it, so such
 * calls must not overlap (order them on one stream or synchronise). */
int lkhip_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const uint32_t* ctx_len,
                      size_t n_seq, size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t max_seq, float* out,
                      void* stream);
/* lkhip_attn_decode without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot call hipMalloc (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).  Same
 * arguments, kernels and results as lkhip_attn_decode; the flash-decoding
 * arrival counters and partials go to a fixed 8 MiB device buffer (2^21
 * floats) that each device holds for the life of the process: 1024
 * counters 256 bytes apart (n_seq * n_kv_heads <= 1024), then
 * n_seq * n_heads * C * 66 partial floats, C = min(32, ceil(max_seq / 64)).
 * Larger calls fail with LKHIP_E_INVALID before any device work.  The
 * counters start at zero and every call leaves them zero.  All calls on one
 * device share the buffer: calls that overlap on a device (concurrent
 * streams or threads) race. */
int lkhip_attn_decode_noalloc(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                              const uint32_t* ctx_len, size_t n_seq, size_t n_heads, size_t n_kv_heads,
                              size_t head_dim, size_t max_seq, float* out, void* stream);
/* Greedy argmax (src/sampler.rs:67-75, first max wins) of n_rows rows of n. */
int lkhip_argmax(const float* x, size_t n_rows, size_t n, uint32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOKAL_HIP_H */
