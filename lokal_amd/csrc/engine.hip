// engine.hip -- host side of the HIP backend behind the C ABI of
// include/lokal_hip.h: weight upload/repack, Engine / Session / Batcher
// (src/engine.rs:13-71), the per-token launch sequence of Model::forward
// (src/model.rs:196-262), HIP-graph replay, and the kernel-level entry points.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/lokal_hip.h"
#include "lkhip_common.h"
#include "fused.h"
#include "batch_step.h"
#include "gguf.h"
#include "repack.h"

// ------------------------------------------------------------------ errors

static thread_local std::string g_err;

static int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_OR_FAIL(expr)                                                                                  \
    do {                                                                                                   \
        hipError_t _e = (expr);                                                                            \
        if (_e != hipSuccess) return fail(LKHIP_E_HIP, "%s failed: %s", #expr, hipGetErrorString(_e));     \
    } while (0)

extern "C" const char* lkhip_last_error(void) { return g_err.c_str(); }
extern "C" const char* lkhip_version(void) { return "lokal-hip 0.1 (gfx950)"; }
extern "C" int lkhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}


// ------------------------------------------------- co-resident launch gate
// The one-kernel steps (fused.hip, fused_rows.hip) and the lm_head launch
// (lmhead.hip) need every workgroup of their grid resident at once: their
// workgroups wait on words other workgroups publish.  Two such grids running
// together on one device (two sessions or batchers stepping from different
// threads, each on its own stream) can each hold part of the CUs, and their
// bounded waits then time out.  Every session and batcher launch therefore
// goes through this process-wide gate: a launch on a stream other than the
// last one that used the device is first ordered after everything that
// stream had enqueued (an event recorded there, waited on here), so the
// device runs the steps one at a time.  Launches on one stream are ordered
// by the stream itself and pay nothing extra.
struct CoopGate {
    std::mutex mu;
    hipStream_t last = nullptr;
    hipEvent_t ev = nullptr;
};
static CoopGate g_gate[16];

template <typename F>
static int gated_launch(int device, hipStream_t st, F&& launch) {
    CoopGate& g = g_gate[device & 15];
    std::lock_guard<std::mutex> lk(g.mu);
    if (g.last && g.last != st) {
        if (!g.ev) HIP_OR_FAIL(hipEventCreateWithFlags(&g.ev, hipEventDisableTiming));
        HIP_OR_FAIL(hipEventRecord(g.ev, g.last));
        HIP_OR_FAIL(hipStreamWaitEvent(st, g.ev, 0));
    }
    const int rc = launch();
    g.last = st;
    return rc;
}
// A stream about to be destroyed stops being the gate's reference point
// (its work is complete: the caller synchronised it).
static void gate_forget(int device, hipStream_t st) {
    CoopGate& g = g_gate[device & 15];
    std::lock_guard<std::mutex> lk(g.mu);
    if (g.last == st) g.last = nullptr;
}

// ------------------------------------------------------------------ weights

struct lkhip_weight {
    LkDevW dw{};
    void* data = nullptr;
    void* aux = nullptr;
    double bytes = 0;  // algorithmic bytes in the GGUF type
    uint32_t ggml_type = 0;  // the GGUF type (dw.type is the device form)
    ~lkhip_weight() {
        if (data) (void)hipFree(data);
        if (aux) (void)hipFree(aux);
    }
};

using lkr::blk_bytes;
using lkr::blk_elems;

static const char* type_name(uint32_t t) {
    switch (t) {
    case LKHIP_F32: return "F32";
    case LKHIP_F16: return "F16";
    case LKHIP_Q8_0: return "Q8_0";
    case LKHIP_Q4_K: return "Q4_K";
    case LK_Q8_SM: return "Q8_SM (device form of Q5_K / Q6_K)";
    case 2: return "Q4_0";
    case 6: return "Q5_0";
    case 13: return "Q5_K";
    case 14: return "Q6_K";
    default: return "unknown";
    }
}

// Row order of a llama.cpp-permuted q/k weight: device row j of head h reads
// source row h*hd + (j % (hd/2))*2 + j/(hd/2) (unpermute_llama_qk,
// src/gguf/arch.rs:274-286).
static size_t src_row(size_t r, size_t head_dim) {
    if (!head_dim) return r;
    const size_t h = r / head_dim, j = r % head_dim;
    return h * head_dim + (j % (head_dim / 2)) * 2 + j / (head_dim / 2);
}

// Repack GGUF rows into the device layout (values unchanged) and upload.
static int weight_create(uint32_t type, size_t rows, size_t cols, const void* host, size_t nbytes,
                         size_t unpermute_hd, lkhip_weight** out) {
    if (!host || !out || rows == 0 || cols == 0) return fail(LKHIP_E_INVALID, "weight: empty tensor or null pointer");
    if (blk_elems(type) == 0)
        return fail(LKHIP_E_UNSUPPORTED,
                    "tensor type %s is not supported by the hip backend — it takes F16, Q8_0, Q4_0, Q5_0, Q4_K, Q5_K and Q6_K",
                    type_name(type));
    if (cols % blk_elems(type))
        return fail(LKHIP_E_INVALID, "weight: %zu columns is not a whole number of %s blocks", cols, type_name(type));
    if (type == LKHIP_F16 && cols % 8)
        return fail(LKHIP_E_UNSUPPORTED, "F16 weight rows must hold a multiple of 8 values (got %zu)", cols);
    const size_t row_bytes = cols / blk_elems(type) * blk_bytes(type);
    if (nbytes != rows * row_bytes)
        return fail(LKHIP_E_INVALID, "weight: %zu bytes given, %zux%zu %s needs %zu", nbytes, rows, cols,
                    type_name(type), rows * row_bytes);
    if (rows > 0xFFFFFFFFull || cols > 0xFFFFFFFFull) return fail(LKHIP_E_INVALID, "weight too large");
    if (unpermute_hd && rows % unpermute_hd) return fail(LKHIP_E_INVALID, "unpermute: rows not a multiple of head_dim");

    auto w = std::make_unique<lkhip_weight>();
    const uint32_t dev = lkr::device_type(type);
    w->ggml_type = type;
    w->dw.type = dev;
    w->dw.rows = (uint32_t)rows;
    w->dw.cols = (uint32_t)cols;
    w->bytes = (double)nbytes;
    const uint8_t* src = (const uint8_t*)host;
    const size_t data_row = lkr::data_row_bytes(dev, cols), aux_row = lkr::aux_row_bytes(dev, cols);
    std::vector<uint8_t> hd(rows * data_row), ha(rows * aux_row);
    auto repack = [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; r++)
            lkr::repack_row(type, src + src_row(r, unpermute_hd) * row_bytes, cols, hd.data() + r * data_row,
                            ha.data() + r * aux_row);
    };
    const size_t nt = rows * row_bytes > (8u << 20) ? 8 : 1;
    std::vector<std::thread> th;
    for (size_t t = 0; t < nt; t++) th.emplace_back(repack, rows * t / nt, rows * (t + 1) / nt);
    for (auto& t : th) t.join();

    if (hipMalloc(&w->data, hd.size()) != hipSuccess)
        return fail(LKHIP_E_NOMEM, "hipMalloc of %zu bytes for a weight failed", hd.size());
    HIP_OR_FAIL(hipMemcpy(w->data, hd.data(), hd.size(), hipMemcpyHostToDevice));
    if (aux_row) {
        if (hipMalloc(&w->aux, ha.size()) != hipSuccess)
            return fail(LKHIP_E_NOMEM, "hipMalloc of %zu bytes for block scales failed", ha.size());
        HIP_OR_FAIL(hipMemcpy(w->aux, ha.data(), ha.size(), hipMemcpyHostToDevice));
    }
    w->dw.data = (const uint8_t*)w->data;
    w->dw.aux = (const uint8_t*)w->aux;
    *out = w.release();
    return LKHIP_OK;
}

extern "C" int lkhip_weight_create(uint32_t type, size_t rows, size_t cols, const void* host, size_t nbytes,
                                   lkhip_weight** out) {
    if (type == LKHIP_F32) return fail(LKHIP_E_UNSUPPORTED, "F32 matrices are not a matvec weight type here");
    return weight_create(type, rows, cols, host, nbytes, 0, out);
}
extern "C" void lkhip_weight_destroy(lkhip_weight* w) { delete w; }
extern "C" double lkhip_weight_bytes(const lkhip_weight* w) { return w ? w->bytes : 0.0; }

// --------------------------------------------------------------- the engine

struct DevBuf {
    void* p = nullptr;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p) { o.p = nullptr; }
    DevBuf& operator=(DevBuf&& o) noexcept {
        if (this != &o) {
            if (p) (void)hipFree(p);
            p = o.p;
            o.p = nullptr;
        }
        return *this;
    }
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    template <class T>
    T* as() const { return (T*)p; }
};

static int dev_alloc(DevBuf& b, size_t bytes) {
    if (hipMalloc(&b.p, bytes ? bytes : 4) != hipSuccess)
        return fail(LKHIP_E_NOMEM, "hipMalloc of %zu bytes failed", bytes);
    if (hipMemset(b.p, 0, bytes ? bytes : 4) != hipSuccess) return fail(LKHIP_E_HIP, "hipMemset failed");
    return LKHIP_OK;
}

struct Layer {
    std::unique_ptr<lkhip_weight> q, k, v, o, gate, up, down;
    DevBuf in_norm, post_norm, bq, bk, bv;
    bool has_bias = false;
};

// q, k and v stored in different device types: they cannot share one launch.
static bool qkv_mixed(const Layer& ly) {
    return ly.k->dw.type != ly.q->dw.type || ly.v->dw.type != ly.q->dw.type;
}

struct lkhip_engine {
    lkhip_config cfg{};
    uint32_t hd = 0, qd = 0, kvd = 0;
    std::vector<Layer> layers;
    std::unique_ptr<lkhip_weight> embed, lm_head_own;
    lkhip_weight* lm_head = nullptr;
    DevBuf norm;
    LkFreq freq{};
    double matvec_bytes = 0;
    int device = 0;
    // one-kernel decode step (fused.hip): per-layer descriptors on device and
    // the instantiated shape it runs; fused_ok = 0 when no instantiation fits
    DevBuf fused_layers;
    int fused_ok = 0, fused_nchh = 0, fused_nchi = 0, fused_g = 0;
    unsigned fused_blocks = 0;
    size_t fused_lds = 0;
    std::string fused_why;
};

struct Named {
    const lkhip_tensor* t = nullptr;
};

static int upload_vec(DevBuf& b, const lkhip_tensor* t, size_t n, const char* what) {
    if (!t) return fail(LKHIP_E_INVALID, "missing tensor %s", what);
    size_t cnt = t->n_dims == 2 ? t->dims[0] * t->dims[1] : t->dims[0];
    if (cnt != n) return fail(LKHIP_E_INVALID, "%s has %zu values but the config implies %zu", t->name, cnt, n);
    std::vector<float> h(n);
    if (t->ggml_type == LKHIP_F32) {
        if (t->nbytes != n * 4) return fail(LKHIP_E_INVALID, "%s: byte size mismatch", t->name);
        memcpy(h.data(), t->data, n * 4);
    } else if (t->ggml_type == LKHIP_F16) {
        if (t->nbytes != n * 2) return fail(LKHIP_E_INVALID, "%s: byte size mismatch", t->name);
        const uint8_t* s = (const uint8_t*)t->data;
        for (size_t i = 0; i < n; i++) h[i] = lkr::h2f(lkr::u16_at(s + 2 * i));
    } else {
        return fail(LKHIP_E_UNSUPPORTED, "%s: norm/bias tensors must be F32 or F16, got %s", t->name,
                    type_name(t->ggml_type));
    }
    int rc = dev_alloc(b, n * 4);
    if (rc) return rc;
    HIP_OR_FAIL(hipMemcpy(b.p, h.data(), n * 4, hipMemcpyHostToDevice));
    return LKHIP_OK;
}

static int upload_mat(std::unique_ptr<lkhip_weight>& w, const lkhip_tensor* t, size_t rows, size_t cols,
                      size_t unpermute_hd, const char* what) {
    if (!t) return fail(LKHIP_E_INVALID, "missing tensor %s", what);
    if (t->n_dims != 2 || t->dims[0] != rows || t->dims[1] != cols)
        return fail(LKHIP_E_INVALID, "%s is %llux%llu but the config implies %zux%zu", t->name,
                    (unsigned long long)t->dims[0], (unsigned long long)(t->n_dims == 2 ? t->dims[1] : 0), rows,
                    cols);
    lkhip_weight* p = nullptr;
    int rc = weight_create(t->ggml_type, rows, cols, t->data, t->nbytes, unpermute_hd, &p);
    if (rc) {
        std::string why = g_err;
        return fail(rc, "%s: %s", t->name, why.c_str());
    }
    w.reset(p);
    return LKHIP_OK;
}

// Decides whether the one-kernel decode step (fused.hip) can run this model
// and uploads its per-layer descriptors.  Models it cannot run keep the
// per-stage kernels; LKHIP_FUSED=0 forces those.
static int fused_setup(lkhip_engine* e) {
    const lkhip_config& c = e->cfg;
    e->fused_ok = 0;
    const char* env = getenv("LKHIP_FUSED");
    if (env && env[0] == '0') {
        e->fused_why = "disabled by LKHIP_FUSED=0";
        return LKHIP_OK;
    }
    const uint32_t wt = e->layers[0].q->dw.type;
    for (const Layer& ly : e->layers)
        for (auto* w : {ly.q.get(), ly.k.get(), ly.v.get(), ly.o.get(), ly.gate.get(), ly.up.get(), ly.down.get()})
            if (w->dw.type != wt) {
                e->fused_why = "mixed weight types";
                return LKHIP_OK;
            }
    if (e->lm_head->dw.type != wt) {
        e->fused_why = "lm_head type differs from the layer weights";
        return LKHIP_OK;
    }
    const uint32_t ce = (wt == LKHIP_Q8_0 || wt == LK_Q8_SM) ? 16 : wt == LKHIP_F16 ? 8 : 32;
    const uint32_t h = c.hidden_size, I = c.intermediate_size;
    if (e->qd != h) {
        e->fused_why = "q width differs from hidden size";
        return LKHIP_OK;
    }
    e->fused_nchh = (int)((h / ce + 63) / 64);
    e->fused_nchi = (int)((I / ce + 63) / 64);
    e->fused_g = (int)(c.num_attention_heads / c.num_key_value_heads);
    int cus = 0;
    HIP_OR_FAIL(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, e->device));
    e->fused_blocks = (unsigned)cus;
    if (const char* fb = getenv("LKHIP_FUSED_BLOCKS")) {  // measurement: fewer workgroups than CUs
        const int v = atoi(fb);
        if (v > 0 && v <= cus) e->fused_blocks = (unsigned)v;
    }
    const uint32_t nw = e->fused_blocks * (uint32_t)(lk_fused_threads() / 64);
    if ((c.num_attention_heads + 2 * c.num_key_value_heads) * 32 > nw || h > nw) {
        e->fused_why = "more rows per stage than waves";
        return LKHIP_OK;
    }
    if (h > LK_FUSED_MAX_H || c.num_hidden_layers > LK_FUSED_MAX_LAYERS) {
        e->fused_why = "wider or deeper than the one-kernel step takes";
        return LKHIP_OK;
    }
    if (c.num_attention_heads * LK_FUSED_MAX_CH > nw) {
        e->fused_why = "more attention tiles than waves";
        return LKHIP_OK;
    }
    // the q/k/v rows, attention chunks and merges of an XCD's query heads run
    // on that XCD's waves (fused.hip)
    {
        const uint32_t nh = c.num_attention_heads, G = nh / c.num_key_value_heads;
        const uint32_t wx = nw / LK_XCDS;
        bool fits = e->fused_blocks % LK_XCDS == 0;
        for (uint32_t x = 0; x < LK_XCDS && fits; x++) {
            const uint32_t h0 = (x * nh + LK_XCDS - 1) / LK_XCDS, h1 = ((x + 1) * nh + LK_XCDS - 1) / LK_XCDS;
            const uint32_t nq = h1 - h0, nj = nq ? (h1 - 1) / G - h0 / G + 1 : 0;
            fits = (nq + 2 * nj) * 32 <= wx && nq * LK_FUSED_MAX_CH <= wx;
        }
        if (!fits) {
            e->fused_why = "more q/k/v rows or attention chunks per XCD than its waves";
            return LKHIP_OK;
        }
        // the step's workgroups must land evenly on XCDs 0..LK_XCDS-1 (it
        // numbers them per XCD by the hardware id)
        DevBuf ids;
        int rc = dev_alloc(ids, (size_t)e->fused_blocks * 4);
        if (rc) return rc;
        HIP_OR_FAIL(lk_xcd_probe_launch(ids.as<uint32_t>(), e->fused_blocks, nullptr));
        std::vector<uint32_t> h_ids(e->fused_blocks);
        HIP_OR_FAIL(hipMemcpy(h_ids.data(), ids.p, h_ids.size() * 4, hipMemcpyDeviceToHost));
        uint32_t per[16] = {};
        for (uint32_t id : h_ids) per[id & 15]++;
        for (uint32_t x = 0; x < 16; x++)
            if (per[x] != (x < LK_XCDS ? e->fused_blocks / LK_XCDS : 0)) fits = false;
        if (!fits) {
            e->fused_why = "the device does not spread a launch's workgroups evenly over 8 XCDs";
            return LKHIP_OK;
        }
    }
    // LDS limit for the longest session the one-kernel step serves
    e->fused_lds = lk_fused_lds_bytes(h, I, c.num_attention_heads, c.num_key_value_heads, (uint32_t)e->fused_g,
                                      LK_FUSED_MAX_CH);
    LkFusedArgs probe{};
    hipError_t st = hipSuccess;
    for (int kv32 = 0; kv32 < 2 && st == hipSuccess; kv32++)  // both KV cache types
        st = lk_fused_launch(probe, wt, e->fused_nchh, e->fused_nchi, e->fused_g, kv32, e->fused_blocks, e->fused_lds,
                             nullptr, true);
    if (st != hipSuccess) {
        (void)hipGetLastError();
        e->fused_why = "no fused instantiation for this shape";
        return LKHIP_OK;
    }
    std::vector<LkFusedLayer> hl(c.num_hidden_layers);
    for (uint32_t L = 0; L < c.num_hidden_layers; L++) {
        Layer& ly = e->layers[L];
        hl[L] = LkFusedLayer{ly.q->dw, ly.k->dw, ly.v->dw, ly.o->dw, ly.gate->dw, ly.up->dw, ly.down->dw,
                             ly.in_norm.as<float>(), ly.post_norm.as<float>(),
                             ly.has_bias ? ly.bq.as<float>() : nullptr, ly.has_bias ? ly.bk.as<float>() : nullptr,
                             ly.has_bias ? ly.bv.as<float>() : nullptr};
    }
    int rc = dev_alloc(e->fused_layers, hl.size() * sizeof(LkFusedLayer));
    if (rc) return rc;
    HIP_OR_FAIL(hipMemcpy(e->fused_layers.p, hl.data(), hl.size() * sizeof(LkFusedLayer), hipMemcpyHostToDevice));
    e->fused_ok = 1;
    return LKHIP_OK;
}

extern "C" int lkhip_engine_create_tensors(const lkhip_config* cfg, const lkhip_tensor* tensors, size_t n_tensors,
                                           int llama_permuted, lkhip_engine** out) {
    if (!cfg || !out || (!tensors && n_tensors)) return fail(LKHIP_E_INVALID, "engine: null argument");
    *out = nullptr;
    auto e = std::make_unique<lkhip_engine>();
    e->cfg = *cfg;
    if (!cfg->num_attention_heads || !cfg->num_key_value_heads || !cfg->hidden_size || !cfg->num_hidden_layers ||
        !cfg->vocab_size || !cfg->intermediate_size)
        return fail(LKHIP_E_INVALID, "engine: config has a zero dimension");
    e->hd = cfg->head_dim ? cfg->head_dim : cfg->hidden_size / cfg->num_attention_heads;
    if (e->hd != 64)
        return fail(LKHIP_E_UNSUPPORTED, "head_dim %u is not supported by the hip backend — 64 only", e->hd);
    if (cfg->num_attention_heads % cfg->num_key_value_heads ||
        cfg->num_attention_heads / cfg->num_key_value_heads > 8)
        return fail(LKHIP_E_UNSUPPORTED, "GQA group %u/%u is not supported — query heads per kv head must be 1..8",
                    cfg->num_attention_heads, cfg->num_key_value_heads);
    // Per-head q/k RMSNorm (Qwen3-style self_attn.q_norm / k_norm, applied
    // before RoPE at src/model.rs:213-222) is not computed by these kernels:
    // refuse rather than run the layer without it.
    for (size_t i = 0; i < n_tensors; i++) {
        const char* nm = tensors[i].name;
        if (nm && (strstr(nm, "self_attn.q_norm") || strstr(nm, "self_attn.k_norm")))
            return fail(LKHIP_E_UNSUPPORTED,
                        "%s: per-head q/k RMSNorm is not supported by the hip backend — use -b cpu", nm);
    }
    if (lkhip_device_count() == 0) return fail(LKHIP_E_HIP, "no HIP device visible — the hip backend needs an AMD GPU");
    e->qd = cfg->num_attention_heads * e->hd;
    e->kvd = cfg->num_key_value_heads * e->hd;
    (void)hipGetDevice(&e->device);
    // RoPE inverse frequencies with the CPU path's own f32 powf (src/model.rs:273).
    for (uint32_t i = 0; i < e->hd / 2; i++)
        e->freq.f[i] = powf(cfg->rope_theta, -(2.0f * (float)i) / (float)e->hd);

    auto find = [&](const std::string& name) -> const lkhip_tensor* {
        for (size_t i = 0; i < n_tensors; i++)
            if (tensors[i].name && name == tensors[i].name) return &tensors[i];
        return nullptr;
    };
    const size_t h = cfg->hidden_size, I = cfg->intermediate_size;
    const size_t uhd = llama_permuted ? e->hd : 0;
    e->layers.resize(cfg->num_hidden_layers);
    int rc;
    for (uint32_t L = 0; L < cfg->num_hidden_layers; L++) {
        Layer& ly = e->layers[L];
        std::string p = "model.layers." + std::to_string(L) + ".";
        if ((rc = upload_vec(ly.in_norm, find(p + "input_layernorm.weight"), h, (p + "input_layernorm.weight").c_str())))
            return rc;
        if ((rc = upload_vec(ly.post_norm, find(p + "post_attention_layernorm.weight"), h,
                             (p + "post_attention_layernorm.weight").c_str())))
            return rc;
        if ((rc = upload_mat(ly.q, find(p + "self_attn.q_proj.weight"), e->qd, h, uhd, "q_proj"))) return rc;
        if ((rc = upload_mat(ly.k, find(p + "self_attn.k_proj.weight"), e->kvd, h, uhd, "k_proj"))) return rc;
        if ((rc = upload_mat(ly.v, find(p + "self_attn.v_proj.weight"), e->kvd, h, 0, "v_proj"))) return rc;
        if ((rc = upload_mat(ly.o, find(p + "self_attn.o_proj.weight"), h, e->qd, 0, "o_proj"))) return rc;
        if ((rc = upload_mat(ly.gate, find(p + "mlp.gate_proj.weight"), I, h, 0, "gate_proj"))) return rc;
        if ((rc = upload_mat(ly.up, find(p + "mlp.up_proj.weight"), I, h, 0, "up_proj"))) return rc;
        if ((rc = upload_mat(ly.down, find(p + "mlp.down_proj.weight"), h, I, 0, "down_proj"))) return rc;
        const lkhip_tensor* bq = find(p + "self_attn.q_proj.bias");
        const lkhip_tensor* bk = find(p + "self_attn.k_proj.bias");
        const lkhip_tensor* bv = find(p + "self_attn.v_proj.bias");
        if (bq || bk || bv) {
            // Qwen2 carries all three (model.rs reads each independently; a
            // missing one is zero here, which is what no-bias means).
            std::vector<float> zero(std::max(e->qd, e->kvd), 0.f);
            lkhip_tensor zq{"zero", LKHIP_F32, 1, {e->qd, 0}, zero.data(), (uint64_t)e->qd * 4};
            lkhip_tensor zk{"zero", LKHIP_F32, 1, {e->kvd, 0}, zero.data(), (uint64_t)e->kvd * 4};
            if ((rc = upload_vec(ly.bq, bq ? bq : &zq, e->qd, "q bias"))) return rc;
            if ((rc = upload_vec(ly.bk, bk ? bk : &zk, e->kvd, "k bias"))) return rc;
            if ((rc = upload_vec(ly.bv, bv ? bv : &zk, e->kvd, "v bias"))) return rc;
            ly.has_bias = true;
        }
        // q/k/v of different types (Q4_K_M files store some v in Q6_K) run
        // as one launch per projection; gate and up share the SwiGLU launch
        if (ly.gate->dw.type != ly.up->dw.type)
            return fail(LKHIP_E_UNSUPPORTED, "layer %u: gate/up weights must share one type for the fused SwiGLU matvec",
                        L);
        for (auto* w : {ly.q.get(), ly.k.get(), ly.v.get(), ly.o.get(), ly.gate.get(), ly.up.get(), ly.down.get()})
            e->matvec_bytes += w->bytes;
    }
    if ((rc = upload_mat(e->embed, find("model.embed_tokens.weight"), cfg->vocab_size, h, 0, "embed_tokens")))
        return rc;
    if ((rc = upload_vec(e->norm, find("model.norm.weight"), h, "model.norm.weight"))) return rc;
    if (const lkhip_tensor* lm = find("lm_head.weight")) {
        if ((rc = upload_mat(e->lm_head_own, lm, cfg->vocab_size, h, 0, "lm_head"))) return rc;
        e->lm_head = e->lm_head_own.get();
    } else {
        e->lm_head = e->embed.get();  // tied (src/model.rs:181-186)
    }
    if (e->lm_head->dw.type == LKHIP_F32)
        return fail(LKHIP_E_UNSUPPORTED, "lm_head must be F16, Q8_0 or Q4_K on the hip backend");
    if (!lk_lm_head_fits(e->lm_head->dw.type, cfg->hidden_size))
        return fail(LKHIP_E_UNSUPPORTED, "hidden_size %u is wider than the lm_head kernel takes for type %s",
                    cfg->hidden_size, type_name(e->lm_head->dw.type));
    e->matvec_bytes += e->lm_head->bytes;
    if ((rc = fused_setup(e.get()))) return rc;
    *out = e.release();
    return LKHIP_OK;
}

extern "C" void lkhip_engine_destroy(lkhip_engine* e) { delete e; }
extern "C" int lkhip_engine_config(const lkhip_engine* e, lkhip_config* out) {
    if (!e || !out) return fail(LKHIP_E_INVALID, "null argument");
    *out = e->cfg;
    out->head_dim = e->hd;
    return LKHIP_OK;
}
extern "C" double lkhip_engine_matvec_bytes(const lkhip_engine* e) { return e ? e->matvec_bytes : 0.0; }

// -------------------------------------------------------------- sessions

// KV cache seen by the rows path: per layer [slot][n_kv][kv_seq][64].
struct KvDesc {
    uint8_t* kc = nullptr;
    uint8_t* vc = nullptr;
    size_t layer_bytes = 0;    // one layer of one cache, all slots
    uint64_t slot_elems = 0;   // elements between two slots
    uint32_t kv_seq = 0;       // cache rows per kv head
    uint32_t max_seq = 0;      // positions a slot holds
    int kv_f32 = 0;
};

enum HeadMode { HEAD_NONE = 0, HEAD_LAST = 1, HEAD_ALL = 2 };
#define LK_ROWS_LOGITS 64u   // rows whose logits one pass can return
#define LK_PREFILL_CHUNK 512u  // prompt positions per prefill pass (PREFILL_CHUNK, src/gpu/metal.rs:30)

struct Rows {
    uint32_t cap = 0;
    DevBuf meta;   // u32 [ids | pos | slots | ctx | steps], cap each
    DevBuf x, xn, qkv, att, inner, logits, gpart, apart, out_ids, keys;
    size_t out_ids_cap = 0;
    uint32_t* h_meta = nullptr;  // pinned, 5 * cap
    ~Rows() {
        if (h_meta) (void)hipHostFree(h_meta);
    }
};

enum Cat { C_MATVEC = 0, C_LMHEAD = 1, C_ATTN = 2, C_OTHER = 3 };

struct lkhip_session {
    lkhip_engine* e = nullptr;
    size_t max_seq = 0;
    hipStream_t stream = nullptr;
    DevBuf kc, vc;  // [layer][n_kv][kv_seq][64], f16 or f32 (kv_f32)
    size_t kv_seq = 0;  // cache rows per kv head: max_seq rounded up to whole 64-position tiles
    int kv_f32 = 0;
    DevBuf x, xn, qkv, att, inner, logits, part, keys, head_epoch, err, state, feed, ids_out;
    LkStepState* h_state = nullptr;  // pinned
    float* h_logits = nullptr;       // pinned; max(vocab, max_seq) words: logits or greedy ids
    uint32_t head_blocks = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // one-kernel decode step: exchange buffers, epoch counter, error flag
    bool use_fused = false;
    uint32_t fused_rep = LK_FUSED_REP;  // exchange-vector copies (LKHIP_FUSED_REP)
    uint32_t max_chunks = 0;
    size_t fused_lds = 0;
    DevBuf xb, qb, pb, ab, xpb, ib, epoch, xcd_cnt;
    std::unique_ptr<Rows> rows;  // multi-row buffers (prefill, forward_batch), on first use
    DevBuf trace;          // stage timestamps of one block (lkhip_session_set_trace)
    int trace_block = -1;
    // profiling
    bool profiling = false;
    std::vector<hipEvent_t> ev;
    std::vector<int> ev_cat;
    std::vector<double> ev_bytes;
    lkhip_profile prof{};
    ~lkhip_session() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        for (auto v : ev) (void)hipEventDestroy(v);
        if (h_state) (void)hipHostFree(h_state);
        if (h_logits) (void)hipHostFree(h_logits);
        if (stream) {
            (void)hipStreamSynchronize(stream);
            gate_forget(e ? e->device : 0, stream);
            (void)hipStreamDestroy(stream);
        }
    }
};

static size_t kv_layer_elems(const lkhip_session* s) {
    return (size_t)s->e->cfg.num_key_value_heads * s->kv_seq * 64;
}

// Records one launch for profiling: an event after every launch.
struct Rec {
    lkhip_session* s;
    int idx = 0;
    explicit Rec(lkhip_session* s_) : s(s_) {}
    hipError_t mark(int cat, double bytes) {
        if (!s->profiling) return hipSuccess;
        if ((size_t)idx + 1 >= s->ev.size()) return hipErrorInvalidValue;
        s->ev_cat[idx] = cat;
        s->ev_bytes[idx] = bytes;
        idx++;
        return hipEventRecord(s->ev[idx], s->stream);
    }
};

static LkMvArgs mv_args(const float* x, uint32_t cols) {
    LkMvArgs a{};
    a.x = x;
    a.cols = cols;
    return a;
}

// Final RMSNorm + lm_head + argmax + step advance (lmhead.hip).
static LkHeadArgs head_args(lkhip_session* s, const float* x, uint32_t x_stride, bool defer) {
    const lkhip_engine* e = s->e;
    LkHeadArgs a{};
    a.x = x;
    a.x_stride = x_stride;
    a.norm = e->norm.as<float>();
    a.eps = e->cfg.rms_norm_eps;
    a.w = e->lm_head->dw;
    a.h = e->cfg.hidden_size;
    a.vocab = e->cfg.vocab_size;
    a.logits = s->logits.as<float>();
    a.keys = s->keys.as<uint64_t>();
    a.epoch = s->head_epoch.as<uint32_t>();
    a.err = s->err.as<uint32_t>();
    a.st = s->state.as<LkStepState>();
    a.feed = s->feed.as<uint32_t>();
    a.ids_out = s->ids_out.as<uint32_t>();
    a.defer = defer ? 1u : 0u;
    return a;
}
// Whether the one-kernel step path defers the lm_head's argmax fold to the
// next step's start (LKHIP_HEAD_DEFER=0: the lm_head's block 0 collects the
// keys itself, as on the per-stage path).
static bool head_deferred() {
    const char* d = getenv("LKHIP_HEAD_DEFER");
    return !(d && d[0] == '0');
}
// defer: the one-kernel step path, whose next step (or head_finish) folds the keys
static hipError_t enqueue_head(lkhip_session* s, const float* x, uint32_t x_stride, bool defer, hipStream_t st) {
    return lk_lm_head_launch(head_args(s, x, x_stride, defer), s->head_blocks, st);
}
// Folds a deferred lm_head's keys into the step state, if still pending: after
// the last step of a device-side loop, so the state and ids are final.
static hipError_t enqueue_head_finish(lkhip_session* s, hipStream_t st) {
    return lk_head_finish_launch(head_args(s, nullptr, 1, true), s->head_blocks, st);
}

// The whole decode step of one token (Model::forward, src/model.rs:196-262)
// enqueued on the session stream; reads token/pos from the device state.
static hipError_t enqueue_step(lkhip_session* s, Rec& rec) {
    lkhip_engine* e = s->e;
    const lkhip_config& c = e->cfg;
    hipStream_t st = s->stream;
    const uint32_t h = c.hidden_size, I = c.intermediate_size;
    float* x = s->x.as<float>();
    float* xn = s->xn.as<float>();
    float* qkv = s->qkv.as<float>();
    LkStepState* state = s->state.as<LkStepState>();
    hipError_t err;
#define STEP(call, cat, bytes)                   \
    do {                                         \
        if ((err = (call)) != hipSuccess) return err; \
        if ((err = rec.mark(cat, bytes)) != hipSuccess) return err; \
    } while (0)

    if (s->use_fused) {
        LkFusedArgs a{};
        a.layers = e->fused_layers.as<LkFusedLayer>();
        a.n_layers = c.num_hidden_layers;
        a.embed = e->embed->dw;
        a.norm = e->norm.as<float>();
        a.freq = e->freq;
        a.h = h;
        a.I = I;
        a.nh = c.num_attention_heads;
        a.nkv = c.num_key_value_heads;
        a.vocab = c.vocab_size;
        a.eps = c.rms_norm_eps;
        a.kc = s->kc.p;
        a.vc = s->vc.p;
        a.kv_layer = kv_layer_elems(s);
        a.max_seq = (uint32_t)s->kv_seq;
        a.max_chunks = s->max_chunks;
        a.st = state;
        a.head_keys = head_deferred() ? s->keys.as<uint64_t>() : nullptr;
        a.head_blocks = s->head_blocks;
        a.head_epoch = s->head_epoch.as<uint32_t>();
        a.feed = s->feed.as<uint32_t>();
        a.ids_out = s->ids_out.as<uint32_t>();
        a.epoch = s->epoch.as<uint32_t>();
        a.err = s->err.as<uint32_t>();
        a.xcd_cnt = s->xcd_cnt.as<uint32_t>();
        a.xb = s->xb.as<uint64_t>();
        a.qb = s->qb.as<uint64_t>();
        a.pb = s->pb.as<uint64_t>();
        a.ab = s->ab.as<uint64_t>();
        a.xpb = s->xpb.as<uint64_t>();
        a.ib = s->ib.as<uint64_t>();
        a.trace = s->trace_block >= 0 ? s->trace.as<uint64_t>() : nullptr;
        a.trace_block = (uint32_t)(s->trace_block >= 0 ? s->trace_block : 0);
        a.rep = s->fused_rep;
        // The one kernel streams every layer weight of the step: its time is
        // the dequant-matvec time of the layers.
        STEP(lk_fused_launch(a, e->layers[0].q->dw.type, e->fused_nchh, e->fused_nchi, e->fused_g, s->kv_f32,
                             e->fused_blocks, s->fused_lds, st, false),
             C_MATVEC, e->matvec_bytes - e->lm_head->bytes);
        // the last layer's output: f32 halves of the (f32 | epoch) words
        STEP(enqueue_head(s, (const float*)(s->xb.as<uint64_t>() + (size_t)(c.num_hidden_layers & 1) * LK_FUSED_REP * h),
                          2, head_deferred(), st),
             C_LMHEAD, e->lm_head->bytes);
        return hipSuccess;
    }

    STEP(lk_embed_step_launch(e->embed->dw, state, x, st), C_OTHER, 0);
    for (uint32_t L = 0; L < c.num_hidden_layers; L++) {
        Layer& ly = e->layers[L];
        STEP(lk_rmsnorm_launch(x, ly.in_norm.as<float>(), 1, h, c.rms_norm_eps, xn, st), C_OTHER, 0);
        {
            const LkSeg sq{ly.q->dw, ly.has_bias ? ly.bq.as<float>() : nullptr, qkv};
            const LkSeg sk{ly.k->dw, ly.has_bias ? ly.bk.as<float>() : nullptr, qkv + e->qd};
            const LkSeg sv{ly.v->dw, ly.has_bias ? ly.bv.as<float>() : nullptr, qkv + e->qd + e->kvd};
            if (!qkv_mixed(ly)) {
                LkMvArgs a = mv_args(xn, h);
                a.nseg = 3;
                a.seg[0] = sq;
                a.seg[1] = sk;
                a.seg[2] = sv;
                a.total_rows = e->qd + 2 * e->kvd;
                STEP(lk_matvec_launch(a, LK_MV_STORE, st), C_MATVEC, ly.q->bytes + ly.k->bytes + ly.v->bytes);
            } else {
                const LkSeg segs[3] = {sq, sk, sv};
                const lkhip_weight* ws[3] = {ly.q.get(), ly.k.get(), ly.v.get()};
                for (int i = 0; i < 3; i++) {
                    LkMvArgs a = mv_args(xn, h);
                    a.nseg = 1;
                    a.seg[0] = segs[i];
                    a.total_rows = segs[i].w.rows;
                    STEP(lk_matvec_launch(a, LK_MV_STORE, st), C_MATVEC, ws[i]->bytes);
                }
            }
        }
        const size_t kv_el = s->kv_f32 ? 4 : 2;
        uint8_t* kc = s->kc.as<uint8_t>() + (size_t)L * kv_layer_elems(s) * kv_el;
        uint8_t* vc = s->vc.as<uint8_t>() + (size_t)L * kv_layer_elems(s) * kv_el;
        STEP(lk_rope_kv_launch(qkv, c.num_attention_heads, c.num_key_value_heads, e->freq, state, nullptr, 1, kc, vc,
                               s->kv_f32,
                               (uint32_t)s->kv_seq, 0, nullptr, st),
             C_OTHER, 0);
        {
            LkAttnArgs a{};
            a.q = qkv;
            a.k = kc;
            a.v = vc;
            a.kv_f32 = (uint32_t)s->kv_f32;
            a.out = s->att.as<float>();
            a.st = state;
            a.n_seq = 1;
            a.n_heads = c.num_attention_heads;
            a.n_kv = c.num_key_value_heads;
            a.max_seq = (uint32_t)s->kv_seq;
            lk_attn_bind_scratch(a, s->part.as<float>(), c.num_key_value_heads);
            a.seq_stride = 0;
            a.q_stride = e->qd;
            STEP(lk_attn_launch(a, st), C_ATTN, 0);
        }
        {
            LkMvArgs a = mv_args(s->att.as<float>(), e->qd);
            a.nseg = 1;
            a.seg[0] = {ly.o->dw, nullptr, x};
            a.total_rows = h;
            STEP(lk_matvec_launch(a, LK_MV_ACC, st), C_MATVEC, ly.o->bytes);
        }
        STEP(lk_rmsnorm_launch(x, ly.post_norm.as<float>(), 1, h, c.rms_norm_eps, xn, st), C_OTHER, 0);
        {
            LkMvArgs a = mv_args(xn, h);
            a.nseg = 2;
            a.seg[0] = {ly.gate->dw, nullptr, s->inner.as<float>()};
            a.seg[1] = {ly.up->dw, nullptr, nullptr};
            a.total_rows = I;
            STEP(lk_matvec_launch(a, LK_MV_SWIGLU, st), C_MATVEC, ly.gate->bytes + ly.up->bytes);
        }
        {
            LkMvArgs a = mv_args(s->inner.as<float>(), I);
            a.nseg = 1;
            a.seg[0] = {ly.down->dw, nullptr, x};
            a.total_rows = h;
            STEP(lk_matvec_launch(a, LK_MV_ACC, st), C_MATVEC, ly.down->bytes);
        }
    }
    STEP(enqueue_head(s, x, 1, false, st), C_LMHEAD, e->lm_head->bytes);
#undef STEP
    return hipSuccess;
}

// Whether the session replays its step as a HIP graph (LKHIP_GRAPH=1).  By
// default it launches the step directly: measured on MI355X at the Qwen2.5
// shape, the one-kernel step's two launches ran faster that way (2590 against
// 2555 tok/s) and the per-stage step's ~220 as fast (1177 against 1172).
static bool want_graph(const lkhip_session*) {
    const char* g = getenv("LKHIP_GRAPH");
    return g && g[0] == '1';
}

static int build_graph(lkhip_session* s) {
    Rec rec(s);
    HIP_OR_FAIL(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal));
    hipError_t e1 = enqueue_step(s, rec);
    hipGraph_t g = nullptr;
    hipError_t e2 = hipStreamEndCapture(s->stream, &g);
    if (e1 != hipSuccess || e2 != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return fail(LKHIP_E_HIP, "capturing the decode step failed: %s",
                    hipGetErrorString(e1 != hipSuccess ? e1 : e2));
    }
    s->graph = g;
    HIP_OR_FAIL(hipGraphInstantiate(&s->exec, g, nullptr, nullptr, 0));
    return LKHIP_OK;
}

extern "C" int lkhip_session_create(lkhip_engine* e, size_t max_seq, lkhip_session** out) {
    return lkhip_session_create_ex(e, max_seq, LKHIP_F16, out);
}

extern "C" int lkhip_session_create_ex(lkhip_engine* e, size_t max_seq, uint32_t kv_type, lkhip_session** out) {
    if (!e || !out) return fail(LKHIP_E_INVALID, "session: null argument");
    *out = nullptr;
    if (kv_type != LKHIP_F16 && kv_type != LKHIP_F32)
        return fail(LKHIP_E_UNSUPPORTED, "session: the KV cache is F16 or F32, not %s", type_name(kv_type));
    if (max_seq == 0 || max_seq > 0x7FFFFFFF) return fail(LKHIP_E_INVALID, "session: max_seq must be in 1..2^31");
    (void)hipSetDevice(e->device);
    auto s = std::make_unique<lkhip_session>();
    s->e = e;
    s->max_seq = max_seq;
    s->kv_seq = (max_seq + 63) / 64 * 64;
    const lkhip_config& c = e->cfg;
    HIP_OR_FAIL(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    int rc;
    s->kv_f32 = kv_type == LKHIP_F32;
    const size_t kv = (size_t)c.num_hidden_layers * kv_layer_elems(s.get()) * (s->kv_f32 ? 4 : 2);
    if ((rc = dev_alloc(s->kc, kv)) || (rc = dev_alloc(s->vc, kv))) return rc;
    if ((rc = dev_alloc(s->x, c.hidden_size * 4)) || (rc = dev_alloc(s->xn, c.hidden_size * 4)) ||
        (rc = dev_alloc(s->qkv, (e->qd + 2 * e->kvd) * 4)) || (rc = dev_alloc(s->att, e->qd * 4)) ||
        (rc = dev_alloc(s->inner, (size_t)c.intermediate_size * 4)) ||
        (rc = dev_alloc(s->logits, (size_t)c.vocab_size * 4)))
        return rc;
    if ((rc = dev_alloc(s->part, lk_attn_scratch_floats(1, c.num_attention_heads, (uint32_t)s->kv_seq,
                                                           c.num_key_value_heads) * 4))) return rc;
    s->head_blocks = lk_lm_head_blocks(c.vocab_size, e->lm_head->dw.type, c.hidden_size);
    if ((rc = dev_alloc(s->keys, (size_t)LK_HEAD_MAX_BLOCKS * 2 * 8)) || (rc = dev_alloc(s->head_epoch, 4)) ||
        (rc = dev_alloc(s->err, 4)))
        return rc;
    if ((rc = dev_alloc(s->state, sizeof(LkStepState)))) return rc;
    if ((rc = dev_alloc(s->feed, max_seq * 4)) || (rc = dev_alloc(s->ids_out, max_seq * 4))) return rc;
    if (e->fused_ok && max_seq <= LK_FUSED_MAX_SEQ) {
        const size_t h = c.hidden_size, I = c.intermediate_size;
        const size_t qkvd = e->qd + 2 * e->kvd;
        const size_t unit = lk_fused_unit(s->kv_f32 != 0);
        s->max_chunks = (uint32_t)std::min<size_t>((max_seq + unit - 1) / unit, LK_FUSED_MAX_CH);
        if ((rc = dev_alloc(s->xb, 2 * h * 8 * LK_FUSED_REP)) || (rc = dev_alloc(s->qb, 2 * LK_XCDS * qkvd * 8)) ||
            (rc = dev_alloc(s->pb, 2 * (size_t)c.num_attention_heads * s->max_chunks * 66 * 8)) ||
            (rc = dev_alloc(s->ab, 2 * (size_t)e->qd * 8 * LK_FUSED_REP)) ||
            (rc = dev_alloc(s->xpb, 2 * h * 8 * LK_FUSED_REP)) ||
            (rc = dev_alloc(s->ib, 2 * I * 8)) ||
            (rc = dev_alloc(s->epoch, 4)) || (rc = dev_alloc(s->xcd_cnt, LK_XCDS * LK_XCD_CNT_STRIDE * 4)))
            return rc;
        HIP_OR_FAIL(hipMemset(s->xcd_cnt.p, 0, LK_XCDS * LK_XCD_CNT_STRIDE * 4));
        const uint32_t one = 1;
        HIP_OR_FAIL(hipMemcpy(s->epoch.p, &one, 4, hipMemcpyHostToDevice));
        s->fused_lds = lk_fused_lds_bytes(c.hidden_size, c.intermediate_size, c.num_attention_heads,
                                          c.num_key_value_heads, (uint32_t)e->fused_g, s->max_chunks);
        s->use_fused = true;
        const char* rp = getenv("LKHIP_FUSED_REP");
        if (rp) s->fused_rep = std::min<uint32_t>(LK_FUSED_REP, std::max<uint32_t>(1, (uint32_t)atoi(rp)));
    }
    HIP_OR_FAIL(hipHostMalloc((void**)&s->h_state, sizeof(LkStepState), hipHostMallocDefault));
    // The staging buffer carries either one row of logits or up to max_seq greedy ids.
    HIP_OR_FAIL(hipHostMalloc((void**)&s->h_logits, std::max<size_t>(c.vocab_size, max_seq) * 4,
                              hipHostMallocDefault));
    if (want_graph(s.get()) && (rc = build_graph(s.get()))) return rc;
    *out = s.release();
    return LKHIP_OK;
}

extern "C" void lkhip_session_destroy(lkhip_session* s) {
    if (s && s->stream) (void)hipStreamSynchronize(s->stream);
    delete s;
}

static int set_state(lkhip_session* s, uint32_t token, size_t pos, uint32_t n_feed) {
    memset(s->h_state, 0, sizeof(LkStepState));
    s->h_state->token = token;
    s->h_state->pos = (uint32_t)pos;
    s->h_state->n_feed = n_feed;
    HIP_OR_FAIL(hipMemcpyAsync(s->state.p, s->h_state, sizeof(LkStepState), hipMemcpyHostToDevice, s->stream));
    return LKHIP_OK;
}

// Runs one step: graph replay, or eager with events when profiling.
static int run_step(lkhip_session* s) {
    if (!s->profiling) {
        return gated_launch(s->e->device, s->stream, [&]() -> int {
            if (s->exec) {
                HIP_OR_FAIL(hipGraphLaunch(s->exec, s->stream));
            } else {
                Rec rec(s);
                hipError_t err = enqueue_step(s, rec);
                if (err != hipSuccess)
                    return fail(LKHIP_E_HIP, "decode step launch failed: %s", hipGetErrorString(err));
            }
            return LKHIP_OK;
        });
    }
    Rec rec(s);
    int rc = gated_launch(s->e->device, s->stream, [&]() -> int {
        HIP_OR_FAIL(hipEventRecord(s->ev[0], s->stream));
        hipError_t err = enqueue_step(s, rec);
        if (err != hipSuccess) return fail(LKHIP_E_HIP, "decode step launch failed: %s", hipGetErrorString(err));
        return LKHIP_OK;
    });
    if (rc) return rc;
    HIP_OR_FAIL(hipEventSynchronize(s->ev[rec.idx]));
    for (int i = 0; i < rec.idx; i++) {
        float ms = 0.f;
        HIP_OR_FAIL(hipEventElapsedTime(&ms, s->ev[i], s->ev[i + 1]));
        switch (s->ev_cat[i]) {
        case C_MATVEC:
            s->prof.matvec_launches++;
            s->prof.matvec_ms += ms;
            s->prof.matvec_bytes += s->ev_bytes[i];
            break;
        case C_LMHEAD:
            s->prof.lm_head_launches++;
            s->prof.lm_head_ms += ms;
            s->prof.lm_head_bytes += s->ev_bytes[i];
            s->prof.matvec_launches++;
            s->prof.matvec_ms += ms;
            s->prof.matvec_bytes += s->ev_bytes[i];
            break;
        case C_ATTN: s->prof.attn_ms += ms; break;
        default: s->prof.other_ms += ms; break;
        }
    }
    s->prof.tokens++;
    return LKHIP_OK;
}

// After a run of steps: the one-kernel path leaves the last lm_head's keys
// pending (the next step would fold them); fold them now so the state and
// the ids are final.
static int finish_steps(lkhip_session* s) {
    if (!s->use_fused || !head_deferred()) return LKHIP_OK;
    hipError_t err = enqueue_head_finish(s, s->stream);
    if (err != hipSuccess) return fail(LKHIP_E_HIP, "decode step finish launch failed: %s", hipGetErrorString(err));
    return LKHIP_OK;
}

static int check_tok(lkhip_session* s, uint32_t token, size_t pos) {
    if (token >= s->e->cfg.vocab_size)
        return fail(LKHIP_E_INVALID, "token id %u is outside the vocabulary (%u)", token, s->e->cfg.vocab_size);
    if (pos >= s->max_seq)
        return fail(LKHIP_E_INVALID, "position %zu exceeds the session's KV cache (%zu positions)", pos, s->max_seq);
    return LKHIP_OK;
}

// Waits for the session stream; if a bounded wait inside the one-kernel step
// timed out, the session drops to the per-stage kernels and the call fails.
static int sync_check(lkhip_session* s) {
    HIP_OR_FAIL(hipStreamSynchronize(s->stream));
    uint32_t flag = 0;
    HIP_OR_FAIL(hipMemcpy(&flag, s->err.p, 4, hipMemcpyDeviceToHost));
    if (!flag) return LKHIP_OK;
    HIP_OR_FAIL(hipMemset(s->err.p, 0, 4));
    if (!(flag & 1)) {
        return fail(LKHIP_E_HIP, "the lm_head's argmax keys were incomplete when folded (a collection timed out: is "
                                 "every CU free?) — the token and state of that step are invalid; restart from a known "
                                 "position");
    }
    // bit 0: a wait inside the one-kernel step timed out (bit 1 may be set too)
    s->use_fused = false;
    if (s->exec) {
        (void)hipGraphExecDestroy(s->exec);
        s->exec = nullptr;
    }
    if (s->graph) {
        (void)hipGraphDestroy(s->graph);
        s->graph = nullptr;
    }
    if (want_graph(s)) {  // the per-stage step from now on
        int rc = build_graph(s);
        if (rc) return rc;
    }
    return fail(LKHIP_E_HIP, "the one-kernel decode step%s timed out waiting on another workgroup (is every CU "
                             "free?) — this session now runs the per-stage kernels; repeat the call",
                flag & 2 ? " and the lm_head launch" : "");
}

static int copy_logits(lkhip_session* s, float* out) {
    const size_t n = s->e->cfg.vocab_size;
    HIP_OR_FAIL(hipMemcpyAsync(s->h_logits, s->logits.p, n * 4, hipMemcpyDeviceToHost, s->stream));
    int rc = sync_check(s);
    if (rc) return rc;
    memcpy(out, s->h_logits, n * 4);
    return LKHIP_OK;
}

extern "C" int lkhip_session_forward(lkhip_session* s, uint32_t token, size_t pos, float* logits_out) {
    if (!s || !logits_out) return fail(LKHIP_E_INVALID, "forward: null argument");
    int rc;
    if ((rc = check_tok(s, token, pos)) || (rc = set_state(s, token, pos, 0)) || (rc = run_step(s))) return rc;
    return copy_logits(s, logits_out);
}

extern "C" int lkhip_session_decode_greedy(lkhip_session* s, uint32_t token, size_t pos, size_t n_steps,
                                           uint32_t* ids_out, float* logits_last) {
    if (!s || (!ids_out && n_steps)) return fail(LKHIP_E_INVALID, "decode_greedy: null argument");
    if (n_steps == 0) return LKHIP_OK;
    int rc;
    if ((rc = check_tok(s, token, pos))) return rc;
    if (pos + n_steps > s->max_seq)
        return fail(LKHIP_E_INVALID, "decode of %zu steps from position %zu exceeds the session's context (%zu)",
                    n_steps, pos, s->max_seq);
    if ((rc = set_state(s, token, pos, 0))) return rc;
    for (size_t i = 0; i < n_steps; i++)
        if ((rc = run_step(s))) return rc;
    if ((rc = finish_steps(s))) return rc;
    HIP_OR_FAIL(hipMemcpyAsync(s->h_logits, s->ids_out.p, n_steps * 4, hipMemcpyDeviceToHost, s->stream));
    if ((rc = sync_check(s))) return rc;
    memcpy(ids_out, s->h_logits, n_steps * 4);
    if (logits_last) return copy_logits(s, logits_last);
    return LKHIP_OK;
}

static float half_bits_to_f32(uint16_t hb16) {
    uint32_t hb = hb16, sign = (hb >> 15) << 31, ex = (hb >> 10) & 31, m = hb & 1023, bits;
    if (ex == 0) {
        if (m == 0) bits = sign;
        else {
            int k = -1;
            do { m <<= 1; k++; } while (!(m & 1024));
            bits = sign | ((uint32_t)(112 - k) << 23) | ((m & 1023) << 13);
        }
    } else if (ex == 31) bits = sign | 0x7f800000u | (m << 13);
    else bits = sign | ((ex + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// Rows pos0..pos0+n-1 of one layer's cache, laid out [kv_head][kv_seq][64]
// from `base`, into out[n][n_kv * 64] as f32.
static int read_kv_rows(const uint8_t* base, uint32_t n_kv, size_t kv_seq, bool f32, size_t pos0, size_t n,
                        float* out) {
    const size_t el = f32 ? 4 : 2;
    std::vector<uint8_t> h(n * 64 * el);
    for (uint32_t kh = 0; kh < n_kv; kh++) {
        HIP_OR_FAIL(hipMemcpy(h.data(), base + ((size_t)kh * kv_seq + pos0) * 64 * el, n * 64 * el,
                              hipMemcpyDeviceToHost));
        for (size_t r = 0; r < n; r++) {
            float* o = out + r * n_kv * 64 + kh * 64;
            if (f32) {
                memcpy(o, h.data() + r * 256, 256);
                continue;
            }
            for (int d = 0; d < 64; d++) {
                const uint8_t* b = h.data() + (r * 64 + d) * 2;
                o[d] = half_bits_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            }
        }
    }
    return LKHIP_OK;
}

extern "C" int lkhip_session_read_kv_rows(lkhip_session* s, uint32_t layer, size_t pos0, size_t n, int which_v,
                                          float* out) {
    if (!s || (!out && n)) return fail(LKHIP_E_INVALID, "read_kv: null argument");
    const lkhip_config& c = s->e->cfg;
    if (layer >= c.num_hidden_layers || pos0 > s->max_seq || n > s->max_seq - pos0)
        return fail(LKHIP_E_INVALID, "read_kv: out of range");
    if (n == 0) return LKHIP_OK;
    HIP_OR_FAIL(hipStreamSynchronize(s->stream));
    const size_t el = s->kv_f32 ? 4 : 2;
    const uint8_t* base = (which_v ? s->vc : s->kc).as<uint8_t>() + (size_t)layer * kv_layer_elems(s) * el;
    return read_kv_rows(base, c.num_key_value_heads, s->kv_seq, s->kv_f32 != 0, pos0, n, out);
}

extern "C" int lkhip_session_read_kv(lkhip_session* s, uint32_t layer, size_t pos, int which_v, float* out) {
    if (!s || !out) return fail(LKHIP_E_INVALID, "read_kv: null argument");
    if (pos >= s->max_seq) return fail(LKHIP_E_INVALID, "read_kv: out of range");
    return lkhip_session_read_kv_rows(s, layer, pos, 1, which_v, out);
}

extern "C" int lkhip_session_set_profiling(lkhip_session* s, int on) {
    if (!s) return fail(LKHIP_E_INVALID, "null session");
    s->profiling = on != 0;
    if (s->profiling && s->ev.empty()) {
        const size_t n = 16 + (size_t)s->e->cfg.num_hidden_layers * 12;
        s->ev.resize(n);
        s->ev_cat.resize(n);
        s->ev_bytes.resize(n);
        for (auto& v : s->ev) HIP_OR_FAIL(hipEventCreate(&v));
    }
    return LKHIP_OK;
}

extern "C" int lkhip_session_profile(lkhip_session* s, lkhip_profile* out, int reset) {
    if (!s || !out) return fail(LKHIP_E_INVALID, "null argument");
    *out = s->prof;
    if (reset) s->prof = lkhip_profile{};
    return LKHIP_OK;
}

static int rebuild_graph(lkhip_session* s) {
    HIP_OR_FAIL(hipStreamSynchronize(s->stream));
    if (s->exec) {
        (void)hipGraphExecDestroy(s->exec);
        s->exec = nullptr;
    }
    if (s->graph) {
        (void)hipGraphDestroy(s->graph);
        s->graph = nullptr;
    }
    return want_graph(s) ? build_graph(s) : LKHIP_OK;
}

extern "C" int lkhip_session_set_trace(lkhip_session* s, int block) {
    if (!s) return fail(LKHIP_E_INVALID, "null session");
    if (!s->use_fused) return fail(LKHIP_E_UNSUPPORTED, "stage tracing needs the one-kernel decode step");
    if (block >= (int)s->e->fused_blocks) return fail(LKHIP_E_INVALID, "trace block %d out of range", block);
    if (block >= 0 && !s->trace.p) {
        int rc = dev_alloc(s->trace, (size_t)s->e->fused_blocks * lk_fused_trace_len(s->e->cfg.num_hidden_layers) * 8);
        if (rc) return rc;
    }
    s->trace_block = block < 0 ? -1 : block;
    return rebuild_graph(s);
}

static size_t trace_len(const lkhip_session* s) {
    if (s->trace_block < 0) return 0;
    return (size_t)s->e->fused_blocks * lk_fused_trace_len(s->e->cfg.num_hidden_layers);
}

extern "C" size_t lkhip_session_trace_len(const lkhip_session* s) { return s ? trace_len(s) : 0; }

extern "C" int lkhip_session_trace(lkhip_session* s, uint64_t* ticks, size_t n) {
    if (!s || !ticks) return fail(LKHIP_E_INVALID, "null argument");
    const size_t len = trace_len(s);
    if (s->trace_block < 0) return fail(LKHIP_E_INVALID, "stage tracing is off");
    if (n < len) return fail(LKHIP_E_INVALID, "trace needs %zu entries", len);
    HIP_OR_FAIL(hipStreamSynchronize(s->stream));
    HIP_OR_FAIL(hipMemcpy(ticks, s->trace.p, len * 8, hipMemcpyDeviceToHost));
    return LKHIP_OK;
}

// ------------------------------------------------------------ rows path
// Model::forward (src/model.rs:196-262) for B tokens in one pass: every
// linear layer is one multi-row GEMM (gemm.hip) that reads each weight once
// for all rows.  A row is (token, position, KV slot); rows of one slot at
// consecutive positions are a prefill chunk (each row attends to the
// positions up to its own: its K/V are written before attention runs), rows
// of different slots are a Batcher decode step (src/engine.rs:42-47).

// Split-K workspace the rows path needs for up to `cap` rows.
static size_t rows_gemm_part(const lkhip_engine* e, uint32_t cap) {
    const lkhip_config& c = e->cfg;
    const uint32_t h = c.hidden_size, I = c.intermediate_size;
    size_t need = 0;
    for (uint32_t n = 1; n <= cap; n++)
    for (const Layer& l0 : e->layers) {
        const LkGemmPlan p[5] = {
            lk_gemm_plan(l0.q->dw.type, e->qd + 2 * e->kvd, h, n, LK_MV_STORE),
            lk_gemm_plan(l0.o->dw.type, h, e->qd, n, LK_MV_ACC), lk_gemm_plan(l0.gate->dw.type, I, h, n, LK_MV_SWIGLU),
            lk_gemm_plan(l0.down->dw.type, h, I, n, LK_MV_ACC),
            lk_gemm_plan(e->lm_head->dw.type, c.vocab_size, h, n < LK_ROWS_LOGITS ? n : LK_ROWS_LOGITS, LK_MV_STORE)};
        for (const auto& q : p) need = std::max(need, q.part_floats);
        if (qkv_mixed(l0))
            for (const lkhip_weight* w : {l0.q.get(), l0.k.get(), l0.v.get()})
                need = std::max(need, lk_gemm_plan(w->dw.type, w->dw.rows, h, n, LK_MV_STORE).part_floats);
    }
    return need;
}

static int rows_check_engine(const lkhip_engine* e) {
    const lkhip_config& c = e->cfg;
    const uint32_t h = c.hidden_size, I = c.intermediate_size;
    for (const Layer& ly : e->layers) {
        if (!lk_gemm_shape_ok(ly.q->dw.type, e->qd + 2 * e->kvd, h) || !lk_gemm_shape_ok(ly.k->dw.type, e->kvd, h) ||
            !lk_gemm_shape_ok(ly.v->dw.type, e->kvd, h) || !lk_gemm_shape_ok(ly.o->dw.type, h, e->qd) ||
            !lk_gemm_shape_ok(ly.gate->dw.type, I, h) || !lk_gemm_shape_ok(ly.down->dw.type, h, I))
            return fail(LKHIP_E_UNSUPPORTED,
                        "the batched path needs hidden and intermediate widths that are multiples of 32 (256 for "
                        "Q4_K) — hidden %u, intermediate %u do not fit",
                        h, I);
    }
    return LKHIP_OK;
}

static int rows_alloc(const lkhip_engine* e, Rows& R, uint32_t cap, uint32_t max_seq) {
    const lkhip_config& c = e->cfg;
    int rc = rows_check_engine(e);
    if (rc) return rc;
    R.cap = cap;
    const size_t h = c.hidden_size, I = c.intermediate_size, qkvd = e->qd + 2 * e->kvd;
    const size_t lrows = std::min<uint32_t>(cap, LK_ROWS_LOGITS);
    if ((rc = dev_alloc(R.meta, 5 * (size_t)cap * 4)) || (rc = dev_alloc(R.x, cap * h * 4)) ||
        (rc = dev_alloc(R.xn, cap * h * 4)) || (rc = dev_alloc(R.qkv, cap * qkvd * 4)) ||
        (rc = dev_alloc(R.att, cap * (size_t)e->qd * 4)) || (rc = dev_alloc(R.inner, cap * I * 4)) ||
        (rc = dev_alloc(R.logits, lrows * c.vocab_size * 4)) ||
        (rc = dev_alloc(R.keys, lrows * ((c.vocab_size + LK_ARGMAX_SLICE - 1) / LK_ARGMAX_SLICE) * 8)) ||
        (rc = dev_alloc(R.gpart, rows_gemm_part(e, cap) * 4)) ||
        (rc = dev_alloc(R.apart, lk_attn_scratch_floats(cap, c.num_attention_heads, max_seq, (size_t)cap * c.num_key_value_heads) * 4)))
        return rc;
    HIP_OR_FAIL(hipHostMalloc((void**)&R.h_meta, 5 * (size_t)cap * 4, hipHostMallocDefault));
    return LKHIP_OK;
}

static hipError_t rows_gemm(Rows& R, LkGemmArgs a, int mode, hipStream_t st) {
    a.part = R.gpart.as<float>();
    a.ks = 0;  // the planned split
    return lk_gemm_launch(a, mode, st);
}

// One pass over n rows whose meta is already on the device; logits of the
// last row (HEAD_LAST) or of every row (HEAD_ALL, n <= LK_ROWS_LOGITS).
// The final RMSNorm (with `pend` split-K partials still to add to x) and the
// lm_head GEMM of every row (HEAD_ALL) or of the last one (HEAD_LAST).
static hipError_t enqueue_rows_head(const lkhip_engine* e, Rows& R, uint32_t n, const float* part, uint32_t pend,
                                    int head, hipStream_t st) {
    const lkhip_config& c = e->cfg;
    const uint32_t h = c.hidden_size;
    float *x = R.x.as<float>(), *xn = R.xn.as<float>();
    hipError_t err = lk_rows_accnorm_launch(x, part, pend, n, h, e->norm.as<float>(), c.rms_norm_eps, xn, st);
    if (err != hipSuccess) return err;
    LkGemmArgs a{};
    a.nseg = 1;
    a.seg[0] = {e->lm_head->dw, nullptr, R.logits.as<float>()};
    a.N = c.vocab_size;
    a.K = h;
    a.n_rows = head == HEAD_ALL ? n : 1;
    a.x = head == HEAD_ALL ? xn : xn + (size_t)(n - 1) * h;
    a.ldx = h;
    a.ldy = c.vocab_size;
    return rows_gemm(R, a, LK_MV_STORE, st);
}

// one_seq: the rows are consecutive positions of one sequence (a prefill
// chunk), which lets the attention read each K/V tile once for several rows.
static hipError_t enqueue_rows(const lkhip_engine* e, Rows& R, uint32_t n, const KvDesc& kv, int head,
                               hipStream_t st, bool one_seq) {
    const lkhip_config& c = e->cfg;
    const uint32_t h = c.hidden_size, I = c.intermediate_size, qd = e->qd, kvd = e->kvd;
    const uint32_t qkvd = qd + 2 * kvd, cap = R.cap;
    uint32_t* meta = R.meta.as<uint32_t>();
    const uint32_t *ids = meta, *pos = meta + cap, *slots = meta + 2 * cap, *ctx = meta + 3 * cap;
    float *x = R.x.as<float>(), *xn = R.xn.as<float>(), *qkv = R.qkv.as<float>();
    float *att = R.att.as<float>(), *inner = R.inner.as<float>();
    hipError_t err;
#define RSTEP(call)                                   \
    do {                                              \
        if ((err = (call)) != hipSuccess) return err; \
    } while (0)
    RSTEP(lk_gather_launch(e->embed->dw, ids, n, x, st));
    // Split-K partials of the QKV, o_proj and down GEMMs are summed by the
    // kernel that consumes them (RoPE + KV append, residual add + RMSNorm)
    // rather than by a reduce launch of their own.
    float* part = R.gpart.as<float>();
    uint32_t pend = 0;  // down partials of the previous layer not yet added to x
    for (uint32_t L = 0; L < c.num_hidden_layers; L++) {
        const Layer& ly = e->layers[L];
        if (L == 0) RSTEP(lk_rmsnorm_launch(x, ly.in_norm.as<float>(), n, h, c.rms_norm_eps, xn, st));
        else RSTEP(lk_rows_accnorm_launch(x, part, pend, n, h, ly.in_norm.as<float>(), c.rms_norm_eps, xn, st));
        uint32_t ks = 0;
        {
            LkGemmArgs a{};
            a.nseg = 3;
            a.seg[0] = {ly.q->dw, ly.has_bias ? ly.bq.as<float>() : nullptr, qkv};
            a.seg[1] = {ly.k->dw, ly.has_bias ? ly.bk.as<float>() : nullptr, qkv + qd};
            a.seg[2] = {ly.v->dw, ly.has_bias ? ly.bv.as<float>() : nullptr, qkv + qd + kvd};
            a.N = qkvd;
            a.K = h;
            a.n_rows = n;
            a.x = xn;
            a.ldx = h;
            a.ldy = qkvd;
            a.part = part;
            if (!qkv_mixed(ly)) {
                RSTEP(lk_gemm_launch(a, LK_MV_STORE, st, &ks));
            } else {
                // one GEMM per projection, each reduced (bias included) into
                // qkv, so the RoPE pass reads finished rows (ks = 0)
                const LkSeg segs[3] = {a.seg[0], a.seg[1], a.seg[2]};
                for (int i = 0; i < 3; i++) {
                    a.nseg = 1;
                    a.seg[0] = segs[i];
                    a.N = segs[i].w.rows;
                    RSTEP(lk_gemm_launch(a, LK_MV_STORE, st));
                }
            }
        }
        uint8_t* kc = kv.kc + L * kv.layer_bytes;
        uint8_t* vc = kv.vc + L * kv.layer_bytes;
        const float* bq = ly.has_bias ? ly.bq.as<float>() : nullptr;
        const float* bk = ly.has_bias ? ly.bk.as<float>() : nullptr;
        const float* bv = ly.has_bias ? ly.bv.as<float>() : nullptr;
        // Batcher rows (sequences that never read each other's K/V): the
        // attention launch rotates q and appends each row's own k / v itself
        // (LkAttnArgs::rope).  A prompt chunk's rows read each other's K/V,
        // so every row is appended first.
        const bool rope_in_attn = !one_seq && !(head == HEAD_NONE && L + 1 == c.num_hidden_layers);
        if (!rope_in_attn)
            RSTEP(lk_rows_rope_kv_launch(qkv, part, ks, bq, bk, bv, c.num_attention_heads, c.num_key_value_heads,
                                         e->freq, pos, n, kc, vc, kv.kv_f32, kv.kv_seq, kv.slot_elems, slots, st));
        // without logits only the last layer's K/V are needed from it
        if (head == HEAD_NONE && L + 1 == c.num_hidden_layers) break;
        {
            LkAttnArgs a{};
            a.q = qkv;
            a.k = kc;
            a.v = vc;
            a.kv_f32 = (uint32_t)kv.kv_f32;
            a.out = att;
            a.ctx_len = ctx;
            a.slots = slots;
            a.n_seq = n;
            a.n_heads = c.num_attention_heads;
            a.n_kv = c.num_key_value_heads;
            a.max_seq = kv.kv_seq;
            lk_attn_bind_scratch(a, R.apart.as<float>(), (size_t)R.cap * c.num_key_value_heads);
            a.seq_stride = kv.slot_elems;
            a.q_stride = qkvd;
            a.grouped = one_seq ? 1u : 0u;
            if (rope_in_attn) {
                a.rope = 1;
                a.rope_ks = ks;
                a.rope_part = part;
                a.bq = bq;
                a.bk = bk;
                a.bv = bv;
                a.pos_rows = pos;
                a.freq = e->freq;
            }
            RSTEP(lk_attn_launch(a, st));
        }
        {
            LkGemmArgs a{};
            a.nseg = 1;
            a.seg[0] = {ly.o->dw, nullptr, x};
            a.N = h;
            a.K = qd;
            a.n_rows = n;
            a.x = att;
            a.ldx = qd;
            a.ldy = h;
            a.part = part;
            RSTEP(lk_gemm_launch(a, LK_MV_ACC, st, &ks));
        }
        RSTEP(lk_rows_accnorm_launch(x, part, ks, n, h, ly.post_norm.as<float>(), c.rms_norm_eps, xn, st));
        {
            LkGemmArgs a{};
            a.nseg = 2;
            a.seg[0] = {ly.gate->dw, nullptr, inner};
            a.seg[1] = {ly.up->dw, nullptr, nullptr};
            a.N = I;
            a.K = h;
            a.n_rows = n;
            a.x = xn;
            a.ldx = h;
            a.ldy = I;
            RSTEP(rows_gemm(R, a, LK_MV_SWIGLU, st));
        }
        {
            LkGemmArgs a{};
            a.nseg = 1;
            a.seg[0] = {ly.down->dw, nullptr, x};
            a.N = h;
            a.K = I;
            a.n_rows = n;
            a.x = inner;
            a.ldx = I;
            a.ldy = h;
            a.part = part;
            RSTEP(lk_gemm_launch(a, LK_MV_ACC, st, &pend));
        }
    }
    if (head != HEAD_NONE) RSTEP(enqueue_rows_head(e, R, n, part, pend, head, st));
#undef RSTEP
    return hipSuccess;
}

// Uploads n rows of (token, pos, slot) (ctx = pos + 1, steps = 0).
static int rows_upload(Rows& R, const uint32_t* tok, const size_t* pos, const uint32_t* slot, uint32_t n,
                       hipStream_t st) {
    const uint32_t cap = R.cap;
    // the pinned buffer may still feed an earlier async copy
    HIP_OR_FAIL(hipStreamSynchronize(st));
    for (uint32_t i = 0; i < n; i++) {
        R.h_meta[i] = tok[i];
        R.h_meta[cap + i] = (uint32_t)pos[i];
        R.h_meta[2 * cap + i] = slot[i];
        R.h_meta[3 * cap + i] = (uint32_t)pos[i] + 1;
        R.h_meta[4 * cap + i] = 0;
    }
    for (int a = 0; a < 5; a++)
        HIP_OR_FAIL(hipMemcpyAsync(R.meta.as<uint32_t>() + (size_t)a * cap, R.h_meta + (size_t)a * cap, n * 4,
                                   hipMemcpyHostToDevice, st));
    return LKHIP_OK;
}

// Prefill of ids at positions pos0.. into one slot, in chunks; the logits of
// the last position into logits_out (device -> host), if given.
static int rows_prefill(const lkhip_engine* e, Rows& R, const KvDesc& kv, uint32_t slot, const uint32_t* ids,
                        size_t n, size_t pos0, float* logits_out, hipStream_t st) {
    const uint32_t chunk = std::min<uint32_t>(R.cap, LK_PREFILL_CHUNK);
    std::vector<size_t> pos(chunk);
    std::vector<uint32_t> slots(chunk, slot);
    for (size_t off = 0; off < n; off += chunk) {
        const uint32_t m = (uint32_t)std::min<size_t>(chunk, n - off);
        for (uint32_t i = 0; i < m; i++) pos[i] = pos0 + off + i;
        int rc = rows_upload(R, ids + off, pos.data(), slots.data(), m, st);
        if (rc) return rc;
        const bool last = off + m == n;
        // Through the gate: a long prefill on this stream must not hold CUs while
        // another stream's one-kernel step needs every workgroup resident.
        rc = gated_launch(e->device, st, [&]() -> int {
            hipError_t err = enqueue_rows(e, R, m, kv, last && logits_out ? HEAD_LAST : HEAD_NONE, st, true);
            if (err != hipSuccess)
                return fail(LKHIP_E_HIP, "batched prefill launch failed: %s", hipGetErrorString(err));
            return LKHIP_OK;
        });
        if (rc) return rc;
    }
    if (logits_out)
        HIP_OR_FAIL(hipMemcpyAsync(logits_out, R.logits.p, (size_t)e->cfg.vocab_size * 4, hipMemcpyDeviceToHost, st));
    HIP_OR_FAIL(hipStreamSynchronize(st));
    return LKHIP_OK;
}

static KvDesc session_kv(lkhip_session* s) {
    KvDesc d;
    const size_t el = s->kv_f32 ? 4 : 2;
    d.kc = s->kc.as<uint8_t>();
    d.vc = s->vc.as<uint8_t>();
    d.layer_bytes = kv_layer_elems(s) * el;
    d.slot_elems = 0;
    d.kv_seq = (uint32_t)s->kv_seq;
    d.max_seq = (uint32_t)s->max_seq;
    d.kv_f32 = s->kv_f32;
    return d;
}

// The session's rows buffers, allocated on first use.
static int session_rows(lkhip_session* s) {
    if (s->rows) return LKHIP_OK;
    auto r = std::make_unique<Rows>();
    const uint32_t cap = (uint32_t)std::min<size_t>(s->max_seq, LK_PREFILL_CHUNK);
    int rc = rows_alloc(s->e, *r, cap, (uint32_t)s->kv_seq);
    if (rc) return rc;
    s->rows = std::move(r);
    return LKHIP_OK;
}

// LKHIP_PREFILL=loop runs prefill as the per-token decode step instead.
static bool prefill_batched() {
    const char* p = getenv("LKHIP_PREFILL");
    return !(p && strcmp(p, "loop") == 0);
}

extern "C" int lkhip_session_prefill(lkhip_session* s, const uint32_t* ids, size_t n, float* logits_out) {
    if (!s || (!ids && n)) return fail(LKHIP_E_INVALID, "prefill: null argument");
    if (n == 0) return fail(LKHIP_E_INVALID, "empty prompt");
    if (n > s->max_seq)
        return fail(LKHIP_E_INVALID, "prompt (%zu tokens) exceeds the session's context (%zu)", n, s->max_seq);
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= s->e->cfg.vocab_size)
            return fail(LKHIP_E_INVALID, "token id %u is outside the vocabulary (%u)", ids[i], s->e->cfg.vocab_size);
    int rc;
    if (prefill_batched() && rows_check_engine(s->e) == LKHIP_OK) {
        if ((rc = session_rows(s))) return rc;
        return rows_prefill(s->e, *s->rows, session_kv(s), 0, ids, n, 0, logits_out, s->stream);
    }
    if (n > 1) HIP_OR_FAIL(hipMemcpyAsync(s->feed.p, ids + 1, (n - 1) * 4, hipMemcpyHostToDevice, s->stream));
    if ((rc = set_state(s, ids[0], 0, (uint32_t)(n - 1)))) return rc;
    for (size_t i = 0; i < n; i++)
        if ((rc = run_step(s))) return rc;
    if ((rc = finish_steps(s))) return rc;
    if (logits_out) return copy_logits(s, logits_out);
    return sync_check(s);
}

extern "C" int lkhip_session_forward_batch(lkhip_session* s, const uint32_t* ids, size_t n, size_t pos0,
                                           float* logits_out) {
    if (!s || (!ids && n) || (!logits_out && n)) return fail(LKHIP_E_INVALID, "forward_batch: null argument");
    if (n == 0) return LKHIP_OK;
    if (pos0 + n > s->max_seq)
        return fail(LKHIP_E_INVALID, "positions %zu..%zu exceed the session's KV cache (%zu positions)", pos0,
                    pos0 + n - 1, s->max_seq);
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= s->e->cfg.vocab_size)
            return fail(LKHIP_E_INVALID, "token id %u is outside the vocabulary (%u)", ids[i], s->e->cfg.vocab_size);
    int rc = rows_check_engine(s->e);
    if (rc) {  // widths the GEMM does not take: the token loop
        for (size_t i = 0; i < n; i++)
            if ((rc = lkhip_session_forward(s, ids[i], pos0 + i, logits_out + i * (size_t)s->e->cfg.vocab_size)))
                return rc;
        return LKHIP_OK;
    }
    if ((rc = session_rows(s))) return rc;
    Rows& R = *s->rows;
    const size_t V = s->e->cfg.vocab_size;
    const uint32_t chunk = std::min<uint32_t>(R.cap, LK_ROWS_LOGITS);
    std::vector<size_t> pos(chunk);
    std::vector<uint32_t> slots(chunk, 0);
    const KvDesc kv = session_kv(s);
    for (size_t off = 0; off < n; off += chunk) {
        const uint32_t m = (uint32_t)std::min<size_t>(chunk, n - off);
        for (uint32_t i = 0; i < m; i++) pos[i] = pos0 + off + i;
        if ((rc = rows_upload(R, ids + off, pos.data(), slots.data(), m, s->stream))) return rc;
        rc = gated_launch(s->e->device, s->stream, [&]() -> int {
            hipError_t err = enqueue_rows(s->e, R, m, kv, HEAD_ALL, s->stream, true);
            if (err != hipSuccess) return fail(LKHIP_E_HIP, "forward_batch launch failed: %s", hipGetErrorString(err));
            return LKHIP_OK;
        });
        if (rc) return rc;
        HIP_OR_FAIL(hipMemcpyAsync(logits_out + off * V, R.logits.p, m * V * 4, hipMemcpyDeviceToHost, s->stream));
    }
    HIP_OR_FAIL(hipStreamSynchronize(s->stream));
    return LKHIP_OK;
}

// ------------------------------------------------------------------ batcher
// Continuous batching (src/engine.rs:36-47): a KV pool of n_slots slots,
// per layer [slot][n_kv][kv_seq][64] f16; a decode step is one rows pass over
// the step's rows (one weight read for all of them).  Decode steps of a given
// row count are captured once as a HIP graph and replayed.

struct lkhip_batch {
    lkhip_engine* e = nullptr;
    size_t n_slots = 0, max_seq = 0;
    hipStream_t stream = nullptr;
    DevBuf kc, vc;
    KvDesc kv;
    Rows rows;
    std::vector<hipGraphExec_t> step_graph;    // by row count: logits of every row
    std::vector<hipGraphExec_t> greedy_graph;  // by row count: + argmax fed back
    // the multi-row one-kernel step (fused_rows.hip) for up to LK_FUSED_ROWS rows
    bool fused_ok = false;            // any of the three kernels below runs here
    bool fused_k_ok[7] = {false, false, false, false, false, false, false};
    size_t fused_lds[7] = {0, 0, 0, 0, 0, 0, 0};  // 2- to 7- and LK_FUSED_ROWS-row kernels
    uint32_t fused_chunks = 0;
    DevBuf fxb, fqb, fpb, fab, fxpb, fib, fepoch, ferr;
    // a step of one row: the single-row one-kernel step (fused.hip) on the
    // row's cache slot, its own exchange buffers and epoch
    bool single_ok = false;
    size_t single_lds = 0;
    uint32_t single_chunks = 0;
    DevBuf sxb, sqb, spb, sab, sxpb, sib, sepoch, sxcd;
    // its final norm + lm_head: lm_head_kernel (the session's one-launch head)
    // in its deferred mode, whose block keys go to hkeys unread (the greedy
    // fold reads the logits)
    DevBuf hkeys, hepoch;
    uint32_t head_blocks = 0;
    // 2-row one-kernel steps: the final norm + lm_head of both rows as one
    // lm_head_rows_kernel launch instead of the norm launch and the GEMM
    // (LKHIP_HEAD_ROWS=0 keeps the GEMM)
    bool head_rows = false;
    std::vector<hipGraphExec_t> fused_graph[2];  // [greedy] by row count
    // the persistent multi-row step (batch_step.hip) for bstep_min..64 rows
    bool bstep_ok = false;
    uint32_t bstep_min = 0;
    DevBuf bs_ss, bs_part, bs_cnt, bs_bar, bs_epoch, bs_trace;
    std::vector<hipGraphExec_t> bstep_graph[2];  // [greedy] by row count
    void drop_fused_graphs() {
        for (auto* vv : {&fused_graph[0], &fused_graph[1], &bstep_graph[0], &bstep_graph[1]}) {
            for (auto g : *vv)
                if (g) (void)hipGraphExecDestroy(g);
            vv->clear();
        }
    }
    ~lkhip_batch() {
        for (auto g : step_graph)
            if (g) (void)hipGraphExecDestroy(g);
        for (auto g : greedy_graph)
            if (g) (void)hipGraphExecDestroy(g);
        drop_fused_graphs();
        if (stream) {
            (void)hipStreamSynchronize(stream);
            gate_forget(e ? e->device : 0, stream);
            (void)hipStreamDestroy(stream);
        }
    }
};

// Whether the Batcher replays its steps as HIP graphs (LKHIP_GRAPH=1).  By
// default it launches them directly: measured on MI355X at the Qwen2.5
// shape, that is as fast or faster at every row count (1 row 0.429 against
// 0.435 ms per step, 16 rows 1.481 against 1.491, 64 rows 2.165 against
// 2.185).
static bool graphs_on() {
    const char* g = getenv("LKHIP_GRAPH");
    return g && g[0] == '1';
}

// The multi-row one-kernel step over the rows whose meta is on the device,
// leaving the final x rows in rows.x.
// Rows of the multi-row one-kernel step's instances, and the one that serves
// n rows (fewer are padded).
static constexpr uint32_t kRowsNb[7] = {2, 3, 4, 5, 6, 7, LK_FUSED_ROWS};
static int rows_kernel(size_t n) { return n <= 2 ? 0 : n <= 7 ? (int)n - 2 : 6; }

static hipError_t batch_enqueue_fused(lkhip_batch* b, uint32_t n, hipStream_t st) {
    const lkhip_engine* e = b->e;
    const lkhip_config& c = e->cfg;
    LkFusedArgs a{};
    a.layers = e->fused_layers.as<LkFusedLayer>();
    a.n_layers = c.num_hidden_layers;
    a.embed = e->embed->dw;
    a.norm = e->norm.as<float>();
    a.freq = e->freq;
    a.h = c.hidden_size;
    a.I = c.intermediate_size;
    a.nh = c.num_attention_heads;
    a.nkv = c.num_key_value_heads;
    a.vocab = c.vocab_size;
    a.eps = c.rms_norm_eps;
    a.kc = b->kv.kc;
    a.vc = b->kv.vc;
    a.kv_layer = b->kv.layer_bytes / 2;
    a.max_seq = b->kv.kv_seq;
    a.max_chunks = b->fused_chunks;
    a.epoch = b->fepoch.as<uint32_t>();
    a.err = b->ferr.as<uint32_t>();
    a.xb = b->fxb.as<uint64_t>();
    a.qb = b->fqb.as<uint64_t>();
    a.pb = b->fpb.as<uint64_t>();
    a.ab = b->fab.as<uint64_t>();
    a.xpb = b->fxpb.as<uint64_t>();
    a.ib = b->fib.as<uint64_t>();
    a.meta = b->rows.meta.as<uint32_t>();
    a.meta_cap = b->rows.cap;
    a.nrows = n;
    a.slot_elems = b->kv.slot_elems;
    a.x_out = b->rows.x.as<float>();
    const int k = rows_kernel(n);
    return lk_fused_rows_launch(a, e->layers[0].q->dw.type, e->fused_nchh, e->fused_nchi, e->fused_g,
                                kRowsNb[k], e->fused_blocks, b->fused_lds[k], st, false);
}

// One row's decode step on the single-row one-kernel step: token, position and
// cache slot from row 0 of the row table on the device, the final x into
// rows.x for the rows' lm_head.
static hipError_t batch_enqueue_single(lkhip_batch* b, hipStream_t st) {
    const lkhip_engine* e = b->e;
    const lkhip_config& c = e->cfg;
    LkFusedArgs a{};
    a.layers = e->fused_layers.as<LkFusedLayer>();
    a.n_layers = c.num_hidden_layers;
    a.embed = e->embed->dw;
    a.norm = e->norm.as<float>();
    a.freq = e->freq;
    a.h = c.hidden_size;
    a.I = c.intermediate_size;
    a.nh = c.num_attention_heads;
    a.nkv = c.num_key_value_heads;
    a.vocab = c.vocab_size;
    a.eps = c.rms_norm_eps;
    a.kc = b->kv.kc;
    a.vc = b->kv.vc;
    a.kv_layer = b->kv.layer_bytes / sizeof(uint16_t);  // a Batcher's cache is f16
    a.max_seq = b->kv.kv_seq;
    a.max_chunks = b->single_chunks;
    a.epoch = b->sepoch.as<uint32_t>();
    a.err = b->ferr.as<uint32_t>();
    a.xcd_cnt = b->sxcd.as<uint32_t>();
    a.xb = b->sxb.as<uint64_t>();
    a.qb = b->sqb.as<uint64_t>();
    a.pb = b->spb.as<uint64_t>();
    a.ab = b->sab.as<uint64_t>();
    a.xpb = b->sxpb.as<uint64_t>();
    a.ib = b->sib.as<uint64_t>();
    a.rep = LK_XCDS;
    a.meta = b->rows.meta.as<uint32_t>();
    a.meta_cap = b->rows.cap;
    a.nrows = 1;
    a.slot_elems = b->kv.slot_elems;
    a.x_out = b->rows.x.as<float>();
    return lk_fused_launch(a, e->layers[0].q->dw.type, e->fused_nchh, e->fused_nchi, e->fused_g, 0, e->fused_blocks,
                           b->single_lds, st, false);
}

// Fewest rows a step takes on the persistent multi-row step by default: none
// (LK_BS_MAX_ROWS + 1).  Measured on MI355X at the Qwen2.5-0.5B Q8_0 shape it
// is slower than the paths it would replace at every row count (4 rows 1.46
// ms per step against 0.75 on fused_rows_kernel, 16 rows 1.59 against 1.50 on
// the per-layer launches, 64 rows 2.33 against 2.04): its five grid barriers
// and split-K round trips per layer cost 8-17 us a phase.
// LKHIP_BATCH_STEP_MIN=n turns it on from n rows.
#ifndef LK_BSTEP_MIN_ROWS
#define LK_BSTEP_MIN_ROWS (LK_BS_MAX_ROWS + 1)
#endif
// Shapes the persistent multi-row step takes: one weight type across the
// layers (fused_setup checked it), an instantiated GQA group, hidden and
// intermediate widths in whole 32-column blocks (Q4_K: 256), q/k/v segments in
// whole 16-row tiles, at most LK_BS_MAXT 128-column tiles of hidden.
static bool bstep_shape_ok(const lkhip_engine* e) {
    const lkhip_config& c = e->cfg;
    const uint32_t wt = e->layers[0].q->dw.type, G = (uint32_t)e->fused_g;
    if (wt != LKHIP_Q8_0 && wt != LKHIP_F16 && wt != LKHIP_Q4_K) return false;
    if (G != 3 && G != 4 && G != 7 && G != 8) return false;
    const uint32_t blk = wt == LKHIP_Q4_K ? 256 : 32;
    if (c.hidden_size % blk || c.intermediate_size % blk || e->qd % blk) return false;
    if (c.hidden_size > 128 * LK_BS_MAXT || c.num_hidden_layers > 50) return false;
    return e->qd % 16 == 0 && e->kvd % 16 == 0;
}

// Split-K plan of the persistent multi-row step's linear layers for n rows:
// enough (output tile, K split) items for every CU, each split at least one
// 128-column chunk.
struct BsPlan {
    uint32_t ks[4], per[4];
    size_t part_floats;
};
static BsPlan bstep_plan(const lkhip_engine* e, uint32_t n) {
    const lkhip_config& c = e->cfg;
    const uint32_t h = c.hidden_size, I = c.intermediate_size, qd = e->qd, kvd = e->kvd;
    const uint32_t NK[4][3] = {{qd + 2 * kvd, h, 1}, {h, qd, 1}, {I, h, 2}, {h, I, 1}};  // N, K, outputs
    BsPlan p{};
    const uint32_t rb = 16 * lk_batch_step_mb(n), bt = (n + rb - 1) / rb;
    for (int g = 0; g < 4; g++) {
        const uint32_t nt = (NK[g][0] + 127) / 128, nck = (NK[g][1] + 127) / 128;
        // the split whose busiest workgroup runs the fewest chunks (items per
        // workgroup x chunks per item); a tie goes to fewer splits
        uint32_t best = ~0u;
        for (uint32_t ks = 1; ks <= nck; ks++) {
            const uint32_t per = (nck + ks - 1) / ks, ks2 = (nck + per - 1) / per;
            const uint32_t rounds = (nt * bt * ks2 + e->fused_blocks - 1) / e->fused_blocks;
            const uint32_t cost = rounds * per;
            if (cost < best) {
                best = cost;
                p.per[g] = per;
                p.ks[g] = ks2;
            }
        }
        if (p.ks[g] > 1)
            p.part_floats = std::max<size_t>(p.part_floats, (size_t)p.ks[g] * n * NK[g][0] * NK[g][2]);
    }
    return p;
}

// The persistent multi-row step over the rows whose meta is on the device,
// leaving the final x rows in rows.x.
static hipError_t batch_enqueue_bstep(lkhip_batch* b, uint32_t n, hipStream_t st) {
    const lkhip_engine* e = b->e;
    const lkhip_config& c = e->cfg;
    Rows& R = b->rows;
    LkBatchStepArgs a{};
    a.layers = e->fused_layers.as<LkFusedLayer>();
    a.n_layers = c.num_hidden_layers;
    a.embed = e->embed->dw;
    a.freq = e->freq;
    a.h = c.hidden_size;
    a.I = c.intermediate_size;
    a.nh = c.num_attention_heads;
    a.nkv = c.num_key_value_heads;
    a.eps = c.rms_norm_eps;
    a.meta = R.meta.as<uint32_t>();
    a.meta_cap = R.cap;
    a.nrows = n;
    a.kc = b->kv.kc;
    a.vc = b->kv.vc;
    a.layer_bytes = b->kv.layer_bytes;
    a.slot_elems = b->kv.slot_elems;
    a.kv_seq = b->kv.kv_seq;
    a.x = R.x.as<float>();
    a.ss = b->bs_ss.as<float>();
    a.qkv = R.qkv.as<float>();
    a.att = R.att.as<float>();
    a.inner = R.inner.as<float>();
    a.part = b->bs_part.as<float>();
    a.cnt = b->bs_cnt.as<uint32_t>();
    const BsPlan p = bstep_plan(e, n);
    for (int g = 0; g < 4; g++) {
        a.ks[g] = p.ks[g];
        a.per[g] = p.per[g];
    }
    LkAttnArgs& at = a.attn;
    at.ctx_len = a.meta + 3 * R.cap;
    at.slots = a.meta + 2 * R.cap;
    at.n_seq = n;
    at.n_heads = c.num_attention_heads;
    at.n_kv = c.num_key_value_heads;
    at.max_seq = b->kv.kv_seq;
    at.seq_stride = b->kv.slot_elems;
    at.q_stride = e->qd + 2 * e->kvd;
    at.kv_f32 = 0;
    lk_attn_bind_scratch(at, R.apart.as<float>(), (size_t)R.cap * c.num_key_value_heads);
    (void)lk_attn_set_plan(at);
    a.bar = b->bs_bar.as<uint64_t>();
    a.epoch = b->bs_epoch.as<uint32_t>();
    a.err = b->ferr.as<uint32_t>();
    a.trace = b->bs_trace.p ? b->bs_trace.as<uint64_t>() : nullptr;
    return lk_batch_step_launch(a, e->layers[0].q->dw.type, e->fused_g, e->fused_blocks, st, false);
}

// Whether the one-kernel step takes rows at these positions (the largest of
// each row over the call): one wave per (row, head, 64-position tile).
static bool batch_fused_fits(const lkhip_batch* b, const std::vector<size_t>& last_pos) {
    if (last_pos.size() == 1 && b->single_ok) return true;  // the single-row step (any position)
    if (!b->fused_ok || last_pos.size() > LK_FUSED_ROWS || !b->fused_k_ok[rows_kernel(last_pos.size())]) return false;
    const lkhip_config& c = b->e->cfg;
    const size_t nb = kRowsNb[rows_kernel(last_pos.size())];
    size_t items = (nb - last_pos.size()) * c.num_attention_heads;  // padding rows
    for (size_t p : last_pos) {
        if (p / 64 + 1 > b->fused_chunks) return false;
        items += (size_t)c.num_attention_heads * (p / 64 + 1);
    }
    return items <= (size_t)b->e->fused_blocks * (lk_fused_threads() / 64);
}

// The device path of a step of these rows: 2 the persistent multi-row step
// (bstep_min rows and up), 1 the one-kernel steps (one row, or a few rows
// that fit fused_rows_kernel), 0 the per-layer launches.
enum { PATH_LAYERS = 0, PATH_FUSED = 1, PATH_BSTEP = 2 };
static int batch_path(const lkhip_batch* b, const std::vector<size_t>& last_pos) {
    const size_t n = last_pos.size();
    if (n == 1 && b->single_ok) return PATH_FUSED;
    if (b->bstep_ok && n >= b->bstep_min && n <= LK_BS_MAX_ROWS) return PATH_BSTEP;
    return batch_fused_fits(b, last_pos) ? PATH_FUSED : PATH_LAYERS;
}

// The final norm and lm_head of a one-row step (the row's final x, written by
// the single-row one-kernel step, in rows.x) into rows.logits: one
// lm_head_kernel launch in its deferred mode, instead of the norm launch and
// the GEMM's 16-row tile for one row.
static hipError_t batch_head_single(lkhip_batch* b, hipStream_t st) {
    const lkhip_engine* e = b->e;
    LkHeadArgs a{};
    a.x = b->rows.x.as<float>();
    a.x_stride = 1;
    a.norm = e->norm.as<float>();
    a.eps = e->cfg.rms_norm_eps;
    a.w = e->lm_head->dw;
    a.h = e->cfg.hidden_size;
    a.vocab = e->cfg.vocab_size;
    a.logits = b->rows.logits.as<float>();
    a.keys = b->hkeys.as<uint64_t>();
    a.epoch = b->hepoch.as<uint32_t>();
    a.err = b->ferr.as<uint32_t>();
    a.defer = 1;
    return lk_lm_head_launch(a, b->head_blocks, st);
}

// The final norm and lm_head of a 2-row one-kernel step (the rows' final x
// in rows.x) into rows.logits: one lm_head_rows_kernel launch.
static bool batch_head_rows_ok(const lkhip_batch* b, uint32_t n) {
    const lkhip_engine* e = b->e;
    return b->head_rows && n >= 2 && lk_lm_head_rows_fits(e->lm_head->dw.type, e->cfg.hidden_size, n);
}
static hipError_t batch_head_rows(lkhip_batch* b, uint32_t n, hipStream_t st) {
    const lkhip_engine* e = b->e;
    LkHeadArgs a{};
    a.x = b->rows.x.as<float>();
    a.x_stride = 1;
    a.norm = e->norm.as<float>();
    a.eps = e->cfg.rms_norm_eps;
    a.w = e->lm_head->dw;
    a.h = e->cfg.hidden_size;
    a.vocab = e->cfg.vocab_size;
    a.logits = b->rows.logits.as<float>();
    return lk_lm_head_rows_launch(a, n, b->head_blocks, st);
}

// Enqueues a decode step of n rows (meta on the device); greedy adds the
// argmax feedback.  Replays a captured graph when graphs are on.  fused: the
// multi-row one-kernel step instead of the per-layer launches.
static int batch_enqueue_step(lkhip_batch* b, uint32_t n, bool greedy, int path = PATH_LAYERS) {
    std::vector<hipGraphExec_t>& cache =
        path == PATH_BSTEP ? b->bstep_graph[greedy ? 1 : 0]
                           : (path == PATH_FUSED ? b->fused_graph[greedy ? 1 : 0]
                                                 : (greedy ? b->greedy_graph : b->step_graph));
    auto body = [&](hipStream_t st) -> hipError_t {
        hipError_t err;
        if (path == PATH_BSTEP) err = batch_enqueue_bstep(b, n, st);
        else if (path == PATH_FUSED) err = n == 1 && b->single_ok ? batch_enqueue_single(b, st) : batch_enqueue_fused(b, n, st);
        else err = enqueue_rows(b->e, b->rows, n, b->kv, HEAD_ALL, st, false);
        if (err == hipSuccess && path != PATH_LAYERS) {
            if (path == PATH_FUSED && n == 1 && b->single_ok) err = batch_head_single(b, st);
            else if (path == PATH_FUSED && batch_head_rows_ok(b, n)) err = batch_head_rows(b, n, st);
            else err = enqueue_rows_head(b->e, b->rows, n, nullptr, 0, HEAD_ALL, st);
        }
        if (err != hipSuccess || !greedy) return err;
        return lk_rows_greedy2_launch(b->rows.logits.as<float>(), n, b->e->cfg.vocab_size, b->rows.keys.as<uint64_t>(),
                                      b->rows.meta.as<uint32_t>(), b->rows.cap, b->rows.out_ids.as<uint32_t>(), st);
    };
    if (!graphs_on()) {
        return gated_launch(b->e->device, b->stream, [&]() -> int {
            hipError_t err = body(b->stream);
            if (err != hipSuccess) return fail(LKHIP_E_HIP, "decode_step launch failed: %s", hipGetErrorString(err));
            return LKHIP_OK;
        });
    }
    if (cache.size() <= n) cache.resize(n + 1, nullptr);
    if (!cache[n]) {
        HIP_OR_FAIL(hipStreamBeginCapture(b->stream, hipStreamCaptureModeThreadLocal));
        hipError_t e1 = body(b->stream);
        hipGraph_t g = nullptr;
        hipError_t e2 = hipStreamEndCapture(b->stream, &g);
        if (e1 != hipSuccess || e2 != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return fail(LKHIP_E_HIP, "capturing the batched decode step failed: %s",
                        hipGetErrorString(e1 != hipSuccess ? e1 : e2));
        }
        hipError_t e3 = hipGraphInstantiate(&cache[n], g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e3 != hipSuccess) {
            cache[n] = nullptr;
            return fail(LKHIP_E_HIP, "instantiating the batched decode step failed: %s", hipGetErrorString(e3));
        }
    }
    return gated_launch(b->e->device, b->stream, [&]() -> int {
        HIP_OR_FAIL(hipGraphLaunch(cache[n], b->stream));
        return LKHIP_OK;
    });
}

extern "C" int lkhip_batch_create(lkhip_engine* e, size_t n_slots, size_t max_seq, lkhip_batch** out) {
    if (!e || !out || n_slots == 0 || max_seq == 0) return fail(LKHIP_E_INVALID, "batch: bad argument");
    if (max_seq > 0x7FFFFFFF || n_slots > 4096) return fail(LKHIP_E_INVALID, "batch: max_seq or n_slots too large");
    *out = nullptr;
    (void)hipSetDevice(e->device);
    auto b = std::make_unique<lkhip_batch>();
    b->e = e;
    b->n_slots = n_slots;
    b->max_seq = max_seq;
    const lkhip_config& c = e->cfg;
    const size_t kv_seq = (max_seq + 63) / 64 * 64;
    const uint64_t slot_elems = (uint64_t)c.num_key_value_heads * kv_seq * 64;
    const size_t layer_bytes = n_slots * slot_elems * 2;
    int rc;
    HIP_OR_FAIL(hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking));
    if ((rc = dev_alloc(b->kc, c.num_hidden_layers * layer_bytes)) ||
        (rc = dev_alloc(b->vc, c.num_hidden_layers * layer_bytes)))
        return rc;
    b->kv.kc = b->kc.as<uint8_t>();
    b->kv.vc = b->vc.as<uint8_t>();
    b->kv.layer_bytes = layer_bytes;
    b->kv.slot_elems = slot_elems;
    b->kv.kv_seq = (uint32_t)kv_seq;
    b->kv.max_seq = (uint32_t)max_seq;
    b->kv.kv_f32 = 0;
    const uint32_t cap = (uint32_t)std::max<size_t>(n_slots, std::min<size_t>(max_seq, LK_PREFILL_CHUNK));
    if ((rc = rows_alloc(e, b->rows, cap, (uint32_t)kv_seq))) return rc;
    // the multi-row one-kernel step, where the model's shape has one
    // (LKHIP_BATCH_FUSED=0 keeps every step on the per-layer launches)
    const char* fe = getenv("LKHIP_BATCH_FUSED");
    if (e->fused_ok && !(fe && fe[0] == '0') && kv_seq <= LK_FUSED_ROWS_MAX_SEQ) {
        const size_t h = c.hidden_size, I = c.intermediate_size, nb = LK_FUSED_ROWS;
        const size_t qkvd = e->qd + 2 * e->kvd;
        b->fused_chunks = (uint32_t)(kv_seq / 64);
        // each row count's kernel on its own: the 8-row one's LDS can exceed
        // a CU's where the 2- and 4-row ones fit (TinyLlama's widths)
        LkFusedArgs probe{};
        bool ok = false;
        for (int k = 0; k < 7; k++) {
            const uint32_t kb = kRowsNb[k];
            b->fused_lds[k] = lk_fused_rows_lds_bytes(c.hidden_size, c.intermediate_size, c.num_attention_heads, kb);
            b->fused_k_ok[k] = lk_fused_rows_launch(probe, e->layers[0].q->dw.type, e->fused_nchh, e->fused_nchi,
                                                    e->fused_g, kb, e->fused_blocks, b->fused_lds[k], nullptr,
                                                    true) == hipSuccess;
            if (!b->fused_k_ok[k]) (void)hipGetLastError();
            ok |= b->fused_k_ok[k];
        }
        if (ok) {
            if ((rc = dev_alloc(b->fxb, 2 * nb * h * 8)) || (rc = dev_alloc(b->fqb, 2 * nb * qkvd * 8)) ||
                (rc = dev_alloc(b->fpb, 2 * nb * c.num_attention_heads * b->fused_chunks * 66 * 8)) ||
                (rc = dev_alloc(b->fab, 2 * nb * e->qd * 8)) || (rc = dev_alloc(b->fxpb, 2 * nb * h * 8)) ||
                (rc = dev_alloc(b->fib, 2 * nb * I * 8)) || (rc = dev_alloc(b->fepoch, 4)) ||
                (rc = dev_alloc(b->ferr, 4)))
                return rc;
            const uint32_t one = 1;
            HIP_OR_FAIL(hipMemcpy(b->fepoch.p, &one, 4, hipMemcpyHostToDevice));
            b->fused_ok = true;
        } else {
            (void)hipGetLastError();
        }
    }
    {
        const char* hr = getenv("LKHIP_HEAD_ROWS");
        b->head_rows = b->fused_ok && !(hr && hr[0] == '0');
        b->head_blocks = lk_lm_head_blocks(c.vocab_size, e->lm_head->dw.type, c.hidden_size);
    }
    // steps of one row: the single-row one-kernel step, for any cache length
    // it takes (LKHIP_BATCH_FUSED=0 keeps these on the per-layer launches too)
    if (e->fused_ok && !(fe && fe[0] == '0') && kv_seq <= LK_FUSED_MAX_SEQ) {
        const size_t h = c.hidden_size, I = c.intermediate_size;
        const size_t qkvd = e->qd + 2 * e->kvd;
        b->single_chunks = (uint32_t)std::min<size_t>(kv_seq / 64, LK_FUSED_MAX_CH);
        b->single_lds = lk_fused_lds_bytes(c.hidden_size, c.intermediate_size, c.num_attention_heads,
                                           c.num_key_value_heads, (uint32_t)e->fused_g, b->single_chunks);
        if ((rc = dev_alloc(b->sxb, 2 * h * 8 * LK_FUSED_REP)) || (rc = dev_alloc(b->sqb, 2 * LK_XCDS * qkvd * 8)) ||
            (rc = dev_alloc(b->spb, 2 * (size_t)c.num_attention_heads * b->single_chunks * 66 * 8)) ||
            (rc = dev_alloc(b->sab, 2 * (size_t)e->qd * 8 * LK_FUSED_REP)) ||
            (rc = dev_alloc(b->sxpb, 2 * h * 8 * LK_FUSED_REP)) || (rc = dev_alloc(b->sib, 2 * I * 8)) ||
            (rc = dev_alloc(b->sepoch, 4)) || (rc = dev_alloc(b->sxcd, LK_XCDS * LK_XCD_CNT_STRIDE * 4)) ||
            (rc = dev_alloc(b->hkeys, (size_t)LK_HEAD_MAX_BLOCKS * 2 * 8)) || (rc = dev_alloc(b->hepoch, 4)))
            return rc;
        HIP_OR_FAIL(hipMemset(b->hepoch.p, 0, 4));
        b->head_blocks = lk_lm_head_blocks(c.vocab_size, e->lm_head->dw.type, c.hidden_size);
        if (!b->ferr.p && (rc = dev_alloc(b->ferr, 4))) return rc;
        HIP_OR_FAIL(hipMemset(b->sxcd.p, 0, LK_XCDS * LK_XCD_CNT_STRIDE * 4));
        HIP_OR_FAIL(hipMemset(b->ferr.p, 0, 4));
        const uint32_t one = 1;
        HIP_OR_FAIL(hipMemcpy(b->sepoch.p, &one, 4, hipMemcpyHostToDevice));
        b->single_ok = true;
    }
    // the persistent multi-row step (LKHIP_BATCH_STEP=0 leaves it off;
    // LKHIP_BATCH_STEP_MIN sets the fewest rows it takes)
    const char* bse = getenv("LKHIP_BATCH_STEP");
    if (e->fused_ok && !(bse && bse[0] == '0') && !(fe && fe[0] == '0') && bstep_shape_ok(e)) {
        LkBatchStepArgs probe{};
        if (lk_batch_step_launch(probe, e->layers[0].q->dw.type, e->fused_g, e->fused_blocks, nullptr, true) ==
            hipSuccess) {
            size_t part = 0;
            for (uint32_t n = 2; n <= LK_BS_MAX_ROWS; n++) part = std::max(part, bstep_plan(e, n).part_floats);
            if ((rc = dev_alloc(b->bs_ss, (size_t)LK_BS_MAX_ROWS * LK_BS_MAXT * 4)) ||
                (rc = dev_alloc(b->bs_part, std::max<size_t>(part, 1) * 4)) ||
                (rc = dev_alloc(b->bs_cnt, (size_t)4 * LK_BS_CNT_PER_GEMM * LK_ATTN_CNT_STRIDE * 4)) ||
                (rc = dev_alloc(b->bs_bar, (size_t)e->fused_blocks * 8)) || (rc = dev_alloc(b->bs_epoch, 4)))
                return rc;
            if (!b->ferr.p && (rc = dev_alloc(b->ferr, 4))) return rc;
            const char* bt = getenv("LKHIP_BSTEP_TRACE");
            if (bt && bt[0] == '1' &&
                (rc = dev_alloc(b->bs_trace, (size_t)lk_batch_step_trace_len(c.num_hidden_layers) * 8)))
                return rc;
            const char* bm = getenv("LKHIP_BATCH_STEP_MIN");
            b->bstep_min = bm ? (uint32_t)std::max(2, atoi(bm)) : (uint32_t)LK_BSTEP_MIN_ROWS;
            b->bstep_ok = true;
        } else {
            (void)hipGetLastError();
        }
    }
    *out = b.release();
    return LKHIP_OK;
}

// Waits for the batch stream; if a bounded wait inside a one-kernel step
// (single- or multi-row) timed out, the batcher drops to the per-layer
// launches and the call fails (repeating it recomputes the same positions).
static int batch_sync_check(lkhip_batch* b, bool fused) {
    HIP_OR_FAIL(hipStreamSynchronize(b->stream));
    if (!fused) return LKHIP_OK;
    uint32_t flag = 0;
    HIP_OR_FAIL(hipMemcpy(&flag, b->ferr.p, 4, hipMemcpyDeviceToHost));
    if (!flag) return LKHIP_OK;
    HIP_OR_FAIL(hipMemset(b->ferr.p, 0, 4));
    b->fused_ok = false;
    b->single_ok = false;
    b->bstep_ok = false;
    b->drop_fused_graphs();
    return fail(LKHIP_E_HIP, "the batcher's one-kernel step timed out waiting on another workgroup (is every CU "
                             "free?) — this batcher now runs the per-layer kernels; repeat the call");
}
extern "C" void lkhip_batch_destroy(lkhip_batch* b) { delete b; }

extern "C" int lkhip_batch_prefill(lkhip_batch* b, uint32_t slot, const uint32_t* ids, size_t n, float* logits_out) {
    if (!b || (!ids && n)) return fail(LKHIP_E_INVALID, "batch prefill: null argument");
    if (slot >= b->n_slots) return fail(LKHIP_E_INVALID, "batch prefill: slot %u out of range", slot);
    if (n == 0) return fail(LKHIP_E_INVALID, "empty prompt");
    if (n > b->max_seq)
        return fail(LKHIP_E_INVALID, "prompt (%zu tokens) exceeds the slot's context (%zu)", n, b->max_seq);
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= b->e->cfg.vocab_size)
            return fail(LKHIP_E_INVALID, "token id %u is outside the vocabulary (%u)", ids[i], b->e->cfg.vocab_size);
    return rows_prefill(b->e, b->rows, b->kv, slot, ids, n, 0, logits_out, b->stream);
}

static int batch_check_rows(lkhip_batch* b, const lkhip_row* rows, size_t n_rows, size_t extra_steps) {
    if (n_rows > b->n_slots) return fail(LKHIP_E_INVALID, "decode_step: %zu rows for %zu slots", n_rows, b->n_slots);
    for (size_t i = 0; i < n_rows; i++) {
        if (rows[i].slot >= b->n_slots)
            return fail(LKHIP_E_INVALID, "decode_step: slot %u out of range", rows[i].slot);
        if (rows[i].token >= b->e->cfg.vocab_size)
            return fail(LKHIP_E_INVALID, "token id %u is outside the vocabulary (%u)", rows[i].token,
                        b->e->cfg.vocab_size);
        if (rows[i].pos + extra_steps >= b->max_seq)
            return fail(LKHIP_E_INVALID, "position %llu exceeds the slot's KV cache (%zu positions)",
                        (unsigned long long)(rows[i].pos + extra_steps), b->max_seq);
        for (size_t j = 0; j < i; j++)
            if (rows[j].slot == rows[i].slot)
                return fail(LKHIP_E_INVALID, "decode_step: slot %u appears twice in one step", rows[i].slot);
    }
    return LKHIP_OK;
}

static int batch_upload_rows(lkhip_batch* b, const lkhip_row* rows, uint32_t n) {
    std::vector<uint32_t> tok(n), slot(n);
    std::vector<size_t> pos(n);
    for (uint32_t i = 0; i < n; i++) {
        tok[i] = rows[i].token;
        slot[i] = rows[i].slot;
        pos[i] = (size_t)rows[i].pos;
    }
    return rows_upload(b->rows, tok.data(), pos.data(), slot.data(), n, b->stream);
}

extern "C" int lkhip_batch_decode_step(lkhip_batch* b, const lkhip_row* rows, size_t n_rows, float* logits_out) {
    if (!b || (!rows && n_rows) || (!logits_out && n_rows)) return fail(LKHIP_E_INVALID, "decode_step: null argument");
    if (n_rows == 0) return LKHIP_OK;
    int rc = batch_check_rows(b, rows, n_rows, 0);
    if (rc) return rc;
    const size_t V = b->e->cfg.vocab_size;
    bool any_fused = false;
    for (size_t off = 0; off < n_rows; off += LK_ROWS_LOGITS) {  // logits of up to 64 rows per pass
        const uint32_t m = (uint32_t)std::min<size_t>(LK_ROWS_LOGITS, n_rows - off);
        std::vector<size_t> last(m);
        for (uint32_t i = 0; i < m; i++) last[i] = (size_t)rows[off + i].pos;
        const int path = batch_path(b, last);
        any_fused |= path != PATH_LAYERS;
        if ((rc = batch_upload_rows(b, rows + off, m)) || (rc = batch_enqueue_step(b, m, false, path))) return rc;
        HIP_OR_FAIL(hipMemcpyAsync(logits_out + off * V, b->rows.logits.p, m * V * 4, hipMemcpyDeviceToHost, b->stream));
    }
    return batch_sync_check(b, any_fused);
}

extern "C" int lkhip_batch_decode_greedy(lkhip_batch* b, const lkhip_row* rows, size_t n_rows, size_t n_steps,
                                         uint32_t* ids_out) {
    if (!b || (!rows && n_rows) || (!ids_out && n_rows && n_steps))
        return fail(LKHIP_E_INVALID, "decode_greedy: null argument");
    if (n_rows == 0 || n_steps == 0) return LKHIP_OK;
    if (n_rows > LK_ROWS_LOGITS)
        return fail(LKHIP_E_INVALID, "decode_greedy: %zu rows — one call takes at most %u", n_rows, LK_ROWS_LOGITS);
    int rc = batch_check_rows(b, rows, n_rows, n_steps - 1);
    if (rc) return rc;
    const uint32_t n = (uint32_t)n_rows;
    const size_t need = n_steps * n_rows;
    if (need > b->rows.out_ids_cap) {  // the greedy graphs hold the buffer's address
        HIP_OR_FAIL(hipStreamSynchronize(b->stream));
        for (auto& g : b->greedy_graph)
            if (g) {
                (void)hipGraphExecDestroy(g);
                g = nullptr;
            }
        for (auto* vv : {&b->fused_graph[1], &b->bstep_graph[1]})
            for (auto& g : *vv)
                if (g) {
                    (void)hipGraphExecDestroy(g);
                    g = nullptr;
                }
        b->rows.out_ids = DevBuf();
        if ((rc = dev_alloc(b->rows.out_ids, need * 4))) return rc;
        b->rows.out_ids_cap = need;
    }
    std::vector<size_t> last(n);
    for (uint32_t i = 0; i < n; i++) last[i] = (size_t)rows[i].pos + n_steps - 1;
    const int path = batch_path(b, last);
    if ((rc = batch_upload_rows(b, rows, n))) return rc;
    for (size_t s = 0; s < n_steps; s++)
        if ((rc = batch_enqueue_step(b, n, true, path))) return rc;
    HIP_OR_FAIL(hipMemcpyAsync(ids_out, b->rows.out_ids.p, need * 4, hipMemcpyDeviceToHost, b->stream));
    return batch_sync_check(b, path != PATH_LAYERS);
}

extern "C" size_t lkhip_batch_trace_len(const lkhip_batch* b) {
    return b && b->bs_trace.p ? lk_batch_step_trace_len(b->e->cfg.num_hidden_layers) : 0;
}
extern "C" int lkhip_batch_trace(lkhip_batch* b, uint64_t* ticks, size_t n) {
    if (!b || (!ticks && n)) return fail(LKHIP_E_INVALID, "batch trace: null argument");
    const size_t len = lkhip_batch_trace_len(b);
    if (!len) return fail(LKHIP_E_UNSUPPORTED, "batch trace: set LKHIP_BSTEP_TRACE=1 before creating the batcher");
    HIP_OR_FAIL(hipStreamSynchronize(b->stream));
    HIP_OR_FAIL(hipMemcpy(ticks, b->bs_trace.p, std::min(n, len) * 8, hipMemcpyDeviceToHost));
    return LKHIP_OK;
}

extern "C" int lkhip_batch_read_kv_rows(lkhip_batch* b, uint32_t slot, uint32_t layer, size_t pos0, size_t n,
                                        int which_v, float* out) {
    if (!b || (!out && n)) return fail(LKHIP_E_INVALID, "read_kv: null argument");
    const lkhip_config& c = b->e->cfg;
    if (slot >= b->n_slots || layer >= c.num_hidden_layers || pos0 > b->max_seq || n > b->max_seq - pos0)
        return fail(LKHIP_E_INVALID, "read_kv: out of range");
    if (n == 0) return LKHIP_OK;
    HIP_OR_FAIL(hipStreamSynchronize(b->stream));
    const uint8_t* base = (which_v ? b->kv.vc : b->kv.kc) + (size_t)layer * b->kv.layer_bytes +
                          (size_t)slot * b->kv.slot_elems * 2;
    return read_kv_rows(base, c.num_key_value_heads, b->kv.kv_seq, false, pos0, n, out);
}

// ------------------------------------------------------------------ memory

extern "C" int lkhip_malloc(void** p, size_t bytes) {
    if (!p) return fail(LKHIP_E_INVALID, "null argument");
    if (hipMalloc(p, bytes ? bytes : 4) != hipSuccess) return fail(LKHIP_E_NOMEM, "hipMalloc of %zu bytes failed", bytes);
    return LKHIP_OK;
}
extern "C" int lkhip_free(void* p) {
    HIP_OR_FAIL(hipFree(p));
    return LKHIP_OK;
}
extern "C" int lkhip_memcpy_htod(void* dst, const void* src, size_t bytes) {
    HIP_OR_FAIL(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return LKHIP_OK;
}
extern "C" int lkhip_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    HIP_OR_FAIL(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return LKHIP_OK;
}
extern "C" int lkhip_memcpy_dtod(void* dst, const void* src, size_t bytes) {
    HIP_OR_FAIL(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return LKHIP_OK;
}
extern "C" int lkhip_memset(void* p, int v, size_t bytes) {
    HIP_OR_FAIL(hipMemset(p, v, bytes));
    return LKHIP_OK;
}
extern "C" int lkhip_synchronize(void) {
    HIP_OR_FAIL(hipDeviceSynchronize());
    return LKHIP_OK;
}
extern "C" int lkhip_stream_create(void** s) {
    if (!s) return fail(LKHIP_E_INVALID, "null argument");
    HIP_OR_FAIL(hipStreamCreateWithFlags((hipStream_t*)s, hipStreamNonBlocking));
    return LKHIP_OK;
}
extern "C" int lkhip_stream_destroy(void* s) {
    HIP_OR_FAIL(hipStreamDestroy((hipStream_t)s));
    return LKHIP_OK;
}
extern "C" int lkhip_stream_synchronize(void* s) {
    HIP_OR_FAIL(hipStreamSynchronize((hipStream_t)s));
    return LKHIP_OK;
}
extern "C" int lkhip_event_create(void** ev) {
    if (!ev) return fail(LKHIP_E_INVALID, "null argument");
    HIP_OR_FAIL(hipEventCreate((hipEvent_t*)ev));
    return LKHIP_OK;
}
extern "C" int lkhip_event_destroy(void* ev) {
    HIP_OR_FAIL(hipEventDestroy((hipEvent_t)ev));
    return LKHIP_OK;
}
extern "C" int lkhip_event_record(void* ev, void* st) {
    HIP_OR_FAIL(hipEventRecord((hipEvent_t)ev, (hipStream_t)st));
    return LKHIP_OK;
}
extern "C" int lkhip_event_elapsed_ms(void* a, void* b, float* ms) {
    if (!ms) return fail(LKHIP_E_INVALID, "null argument");
    HIP_OR_FAIL(hipEventSynchronize((hipEvent_t)b));
    HIP_OR_FAIL(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return LKHIP_OK;
}

// ------------------------------------------------------------------ kernels

#define LAUNCH_OR_FAIL(expr)                                                                                  \
    do {                                                                                                      \
        hipError_t _e = (expr);                                                                               \
        if (_e != hipSuccess) return fail(LKHIP_E_HIP, "kernel launch failed: %s", hipGetErrorString(_e));   \
    } while (0)

extern "C" int lkhip_dequant_rows(const lkhip_weight* w, size_t row0, size_t n_rows, float* out, void* stream) {
    if (!w || (!out && n_rows)) return fail(LKHIP_E_INVALID, "dequant_rows: null argument");
    if (row0 + n_rows > w->dw.rows) return fail(LKHIP_E_INVALID, "dequant_rows: rows out of range");
    LAUNCH_OR_FAIL(lk_dequant_launch(w->dw, (uint32_t)row0, (uint32_t)n_rows, out, (hipStream_t)stream));
    return LKHIP_OK;
}

extern "C" int lkhip_matvec(const lkhip_weight* w, const float* x, const float* bias, float* y, int accumulate,
                            void* stream) {
    if (!w || !x || !y) return fail(LKHIP_E_INVALID, "matvec: null argument");
    LkMvArgs a = mv_args(x, w->dw.cols);
    a.nseg = 1;
    a.seg[0] = {w->dw, bias, y};
    a.total_rows = w->dw.rows;
    LAUNCH_OR_FAIL(lk_matvec_launch(a, accumulate ? LK_MV_ACC : LK_MV_STORE, (hipStream_t)stream));
    return LKHIP_OK;
}
extern "C" int lkhip_q8_0_matvec(const lkhip_weight* w, const float* x, const float* bias, float* y, int accumulate,
                                 void* stream) {
    if (w && w->ggml_type != LKHIP_Q8_0) return fail(LKHIP_E_INVALID, "q8_0_matvec: weight is %s", type_name(w->ggml_type));
    return lkhip_matvec(w, x, bias, y, accumulate, stream);
}
extern "C" int lkhip_q4_k_matvec(const lkhip_weight* w, const float* x, const float* bias, float* y, int accumulate,
                                 void* stream) {
    if (w && w->ggml_type != LKHIP_Q4_K) return fail(LKHIP_E_INVALID, "q4_k_matvec: weight is %s", type_name(w->ggml_type));
    return lkhip_matvec(w, x, bias, y, accumulate, stream);
}

extern "C" int lkhip_matmul(const lkhip_weight* w, const float* x, size_t n_rows, size_t ldx, const float* bias,
                            float* y, size_t ldy, int accumulate, void* stream) {
    if (!w || ((!x || !y) && n_rows)) return fail(LKHIP_E_INVALID, "matmul: null argument");
    if (n_rows == 0) return LKHIP_OK;
    if (n_rows > 0xFFFF) return fail(LKHIP_E_INVALID, "matmul: at most 65535 rows per call");
    const LkDevW& d = w->dw;
    if (!lk_gemm_shape_ok(d.type, d.rows, d.cols))
        return fail(LKHIP_E_UNSUPPORTED, "matmul: a %ux%u %s weight does not fit the GEMM (cols %% %u)", d.rows,
                    d.cols, type_name(d.type), d.type == LKHIP_Q4_K ? 256u : 32u);
    if (ldx < d.cols || ldy < d.rows || ldx % 4 || (uintptr_t)x % 16)
        return fail(LKHIP_E_INVALID, "matmul: ldx must be >= cols and a multiple of 4, x 16-byte aligned, ldy >= rows");
    const int mode = accumulate ? LK_MV_ACC : LK_MV_STORE;
    const LkGemmPlan p = lk_gemm_plan(d.type, d.rows, d.cols, (uint32_t)n_rows, mode);
    hipStream_t st = (hipStream_t)stream;
    void* part = nullptr;
    if (p.part_floats) HIP_OR_FAIL(hipMallocAsync(&part, p.part_floats * 4, st));
    LkGemmArgs a{};
    a.nseg = 1;
    a.seg[0] = {d, bias, y};
    a.N = d.rows;
    a.K = d.cols;
    a.n_rows = (uint32_t)n_rows;
    a.x = x;
    a.ldx = (uint32_t)ldx;
    a.ldy = (uint32_t)ldy;
    a.part = (float*)part;
    a.ks = p.ks;
    hipError_t e = lk_gemm_launch(a, mode, st);
    if (part) (void)hipFreeAsync(part, st);
    if (e != hipSuccess) return fail(LKHIP_E_HIP, "kernel launch failed: %s", hipGetErrorString(e));
    return LKHIP_OK;
}

extern "C" int lkhip_rmsnorm(const float* x, const float* w, size_t n_rows, size_t n, float eps, float* y,
                             void* stream) {
    if ((!x || !w || !y) && n_rows) return fail(LKHIP_E_INVALID, "rmsnorm: null argument");
    if (n == 0) return fail(LKHIP_E_INVALID, "rmsnorm: empty row");
    LAUNCH_OR_FAIL(lk_rmsnorm_launch(x, w, (uint32_t)n_rows, (uint32_t)n, eps, y, (hipStream_t)stream));
    return LKHIP_OK;
}

extern "C" int lkhip_rope_pairs(float* x, size_t n_rows, size_t n, size_t head_dim, const uint32_t* pos, float theta,
                                void* stream) {
    if ((!x || !pos) && n_rows) return fail(LKHIP_E_INVALID, "rope: null argument");
    if (head_dim == 0 || head_dim % 2 || head_dim > 128 || n % head_dim)
        return fail(LKHIP_E_INVALID, "rope: n (%zu) must be a multiple of an even head_dim <= 128 (%zu)", n, head_dim);
    LkFreq f{};
    for (size_t i = 0; i < head_dim / 2; i++) f.f[i] = powf(theta, -(2.0f * (float)i) / (float)head_dim);
    LAUNCH_OR_FAIL(lk_rope_launch(x, (uint32_t)n_rows, (uint32_t)n, (uint32_t)head_dim, pos, f, (hipStream_t)stream));
    return LKHIP_OK;
}

extern "C" int lkhip_swiglu(const float* g, const float* u, size_t n, float* out, void* stream) {
    if ((!g || !u || !out) && n) return fail(LKHIP_E_INVALID, "swiglu: null argument");
    LAUNCH_OR_FAIL(lk_swiglu_launch(g, u, (uint32_t)n, out, (hipStream_t)stream));
    return LKHIP_OK;
}

extern "C" int lkhip_embed_gather(const lkhip_weight* table, const uint32_t* ids, size_t n_ids, float* out,
                                  void* stream) {
    if (!table || ((!ids || !out) && n_ids)) return fail(LKHIP_E_INVALID, "embed_gather: null argument");
    LAUNCH_OR_FAIL(lk_gather_launch(table->dw, ids, (uint32_t)n_ids, out, (hipStream_t)stream));
    return LKHIP_OK;
}

// Shape checks shared by both attention entry points.
static int attn_decode_check(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const uint32_t* ctx_len,
                             size_t n_heads, size_t n_kv_heads, size_t head_dim, float* out, const char* who) {
    if (!q || !k_cache || !v_cache || !ctx_len || !out) return fail(LKHIP_E_INVALID, "%s: null argument", who);
    if (head_dim != 64) return fail(LKHIP_E_UNSUPPORTED, "%s: head_dim %zu — 64 only", who, head_dim);
    if (n_kv_heads == 0 || n_heads % n_kv_heads || n_heads / n_kv_heads > 8)
        return fail(LKHIP_E_UNSUPPORTED, "%s: GQA group %zu/%zu not supported (1..8)", who, n_heads, n_kv_heads);
    return LKHIP_OK;
}

static int attn_decode_launch(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const uint32_t* ctx_len,
                              size_t n_seq, size_t n_heads, size_t n_kv_heads, size_t max_seq, float* out, float* buf,
                              size_t cnt_cap, void* stream) {
    LkAttnArgs a{};
    a.q = q;
    a.k = k_cache;
    a.v = v_cache;
    a.out = out;
    a.ctx_len = ctx_len;
    a.n_seq = (uint32_t)n_seq;
    a.n_heads = (uint32_t)n_heads;
    a.n_kv = (uint32_t)n_kv_heads;
    a.max_seq = (uint32_t)max_seq;
    lk_attn_bind_scratch(a, buf, cnt_cap);
    a.seq_stride = (uint64_t)n_kv_heads * max_seq * 64;
    a.q_stride = n_heads * 64;
    LAUNCH_OR_FAIL(lk_attn_launch(a, (hipStream_t)stream));
    return LKHIP_OK;
}

extern "C" int lkhip_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                 const uint32_t* ctx_len, size_t n_seq, size_t n_heads, size_t n_kv_heads,
                                 size_t head_dim, size_t max_seq, float* out, void* stream) {
    int rc = attn_decode_check(q, k_cache, v_cache, ctx_len, n_heads, n_kv_heads, head_dim, out, "attn_decode");
    if (rc) return rc;
    if (n_seq == 0 || max_seq == 0) return LKHIP_OK;
    if (n_seq > 0xFFFFFFFFu || max_seq > 0x7FFFFFFFu)
        return fail(LKHIP_E_INVALID, "attn_decode: n_seq or max_seq out of range");
    // Scratch for this call (arrival counters + partials), cached per thread
    // and grown on demand; a new buffer starts zeroed.  (Deliberately never
    // freed at thread exit: the HIP runtime may already be torn down by then.)
    static thread_local void* buf = nullptr;
    static thread_local size_t buf_bytes = 0, cnt_cap = 0;
    const size_t cnt_need = n_seq * n_kv_heads;
    const size_t part_need = lk_attn_part_floats((uint32_t)n_seq, (uint32_t)n_heads, (uint32_t)max_seq);
    if (cnt_need > cnt_cap || (lk_attn_cnt_region(cnt_cap) + part_need) * 4 > buf_bytes) {
        const size_t cap = std::max<size_t>({cnt_cap, cnt_need, 256});
        const size_t need = (lk_attn_cnt_region(cap) + part_need) * 4;
        HIP_OR_FAIL(hipStreamSynchronize((hipStream_t)stream));
        if (buf) (void)hipFree(buf);
        buf = nullptr;
        buf_bytes = cnt_cap = 0;
        if (hipMalloc(&buf, need) != hipSuccess) {
            buf = nullptr;
            return fail(LKHIP_E_NOMEM, "hipMalloc of %zu bytes failed", need);
        }
        HIP_OR_FAIL(hipMemset(buf, 0, need));
        buf_bytes = need;
        cnt_cap = cap;
    }
    return attn_decode_launch(q, k_cache, v_cache, ctx_len, n_seq, n_heads, n_kv_heads, max_seq, out, (float*)buf,
                              cnt_cap, stream);
}

extern "C" int lkhip_attn_decode_noalloc(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                         const uint32_t* ctx_len, size_t n_seq, size_t n_heads, size_t n_kv_heads,
                                         size_t head_dim, size_t max_seq, float* out, void* stream) {
    int rc = attn_decode_check(q, k_cache, v_cache, ctx_len, n_heads, n_kv_heads, head_dim, out,
                               "attn_decode_noalloc");
    if (rc) return rc;
    if (n_seq == 0 || max_seq == 0) return LKHIP_OK;
    if (n_seq > 0xFFFFFFFFu || max_seq > 0x7FFFFFFFu)
        return fail(LKHIP_E_INVALID, "attn_decode_noalloc: n_seq or max_seq out of range");
    if (n_seq * n_kv_heads > LK_ATTN_SCRATCH_CNT)
        return fail(LKHIP_E_INVALID,
                    "attn_decode_noalloc: %zu sequences x %zu kv heads exceed its %u arrival counters — use "
                    "lkhip_attn_decode",
                    n_seq, n_kv_heads, LK_ATTN_SCRATCH_CNT);
    const size_t need = lk_attn_scratch_floats((uint32_t)n_seq, (uint32_t)n_heads, (uint32_t)max_seq,
                                               LK_ATTN_SCRATCH_CNT);
    if (need > LK_ATTN_SCRATCH_FLOATS)
        return fail(LKHIP_E_INVALID,
                    "attn_decode_noalloc: %zu sequences x %zu heads x %zu positions need %zu scratch floats, more "
                    "than its fixed %u-float (8 MiB) device buffer — use lkhip_attn_decode",
                    n_seq, n_heads, max_seq, need, LK_ATTN_SCRATCH_FLOATS);
    float* buf = nullptr;
    HIP_OR_FAIL(lk_attn_scratch(&buf));
    return attn_decode_launch(q, k_cache, v_cache, ctx_len, n_seq, n_heads, n_kv_heads, max_seq, out, buf,
                              LK_ATTN_SCRATCH_CNT, stream);
}

extern "C" int lkhip_argmax(const float* x, size_t n_rows, size_t n, uint32_t* out, void* stream) {
    if ((!x || !out) && n_rows) return fail(LKHIP_E_INVALID, "argmax: null argument");
    LAUNCH_OR_FAIL(lk_argmax_rows_launch(x, (uint32_t)n_rows, (uint32_t)n, out, (hipStream_t)stream));
    return LKHIP_OK;
}

extern "C" int lkhip_context_window(size_t window, size_t sink) {
    if (window == 0) return LKHIP_OK;
    return fail(LKHIP_E_UNSUPPORTED,
                "--context-window needs a GPU-windowed backend — -b hip keeps the whole KV cache resident (window %zu, "
                "sink %zu refused); drop the flag or use -b metal, -b hybrid, or -b lowmem",
                window, sink);
}

extern "C" int lkhip_gguf_config(const char* path, lkhip_config* cfg_out, size_t* n_tensors_out,
                                 int* llama_permuted_out) {
    if (!path || !cfg_out) return fail(LKHIP_E_INVALID, "gguf_config: null argument");
    LkGguf g;
    std::string why;
    const int rc = lk_gguf_open(path, &g, &why);
    if (rc) return fail(rc, "%s", why.c_str());
    *cfg_out = g.cfg;
    if (n_tensors_out) *n_tensors_out = g.tensors.size();
    if (llama_permuted_out) *llama_permuted_out = g.llama_permuted;
    lk_gguf_close(&g);
    return LKHIP_OK;
}

extern "C" int lkhip_engine_create_gguf(const char* path, lkhip_engine** out) {
    if (!path || !out) return fail(LKHIP_E_INVALID, "engine: null argument");
    *out = nullptr;
    LkGguf g;
    std::string why;
    int rc = lk_gguf_open(path, &g, &why);
    if (rc) return fail(rc, "%s", why.c_str());
    // weights stay quantized: the engine repacks the mapped bytes onto the
    // device (the create_metal_quant path, src/engine.rs:150-162)
    std::vector<lkhip_tensor> ts(g.tensors.size());
    for (size_t i = 0; i < g.tensors.size(); i++) {
        const LkGgufTensor& t = g.tensors[i];
        ts[i] = lkhip_tensor{t.name.c_str(), t.type, t.n_dims, {t.dims[0], t.dims[1]}, t.data, t.nbytes};
    }
    rc = lkhip_engine_create_tensors(&g.cfg, ts.data(), ts.size(), g.llama_permuted ? 1 : 0, out);
    lk_gguf_close(&g);
    return rc;
}
