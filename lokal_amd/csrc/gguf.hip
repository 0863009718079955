// gguf.hip -- GGUF v2/v3 container reader (host code): the file lokal's
// quantized path runs (GgufFile::open, src/gguf/container.rs:162-261), its
// config (model_config, src/gguf/arch.rs:164-227) and the GGUF -> HF tensor
// names (hf_name, src/gguf/arch.rs:229-270).  The file is memory-mapped and
// read in place; weights are handed to lkhip_engine_create_tensors, which
// repacks them onto the device.  Little-endian files only.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <map>

namespace {

// Elements per block and bytes per block of the GGUF type ids this reader
// sizes (ggml_type; src/gguf/dequant.rs:21-120).  {0, 0} = unknown.
struct TypeSize {
    uint32_t blk, bytes;
    const char* name;
};
TypeSize type_size(uint32_t t) {
    switch (t) {
    case 0: return {1, 4, "F32"};
    case 1: return {1, 2, "F16"};
    case 2: return {32, 18, "Q4_0"};
    case 3: return {32, 20, "Q4_1"};
    case 6: return {32, 22, "Q5_0"};
    case 7: return {32, 24, "Q5_1"};
    case 8: return {32, 34, "Q8_0"};
    case 9: return {32, 36, "Q8_1"};
    case 10: return {256, 84, "Q2_K"};
    case 11: return {256, 110, "Q3_K"};
    case 12: return {256, 144, "Q4_K"};
    case 13: return {256, 176, "Q5_K"};
    case 14: return {256, 210, "Q6_K"};
    case 15: return {256, 292, "Q8_K"};
    case 30: return {1, 2, "BF16"};
    default: return {0, 0, nullptr};
    }
}
// Types the hip backend uploads: matrices F16 / Q8_0 / Q4_0 / Q5_0 / Q4_K /
// Q5_K / Q6_K, vectors F32 / F16.
bool runs(uint32_t t) { return t == 0 || t == 1 || t == 2 || t == 6 || t == 8 || (t >= 12 && t <= 14); }

struct Value {
    enum Kind { U, I, F, B, S, ARR } kind = U;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
    uint64_t arr_len = 0;
};

struct Cursor {
    const uint8_t* b;
    size_t n, p = 0;
    std::string* err;
    bool ok = true;
    const uint8_t* take(size_t k) {
        if (!ok) return nullptr;
        if (k > n || p > n - k) {
            char m[160];
            snprintf(m, sizeof m, "GGUF truncated: need %zu bytes at offset %zu, file has %zu", k, p, n);
            *err = m;
            ok = false;
            return nullptr;
        }
        const uint8_t* r = b + p;
        p += k;
        return r;
    }
    template <typename T>
    T get() {
        T v{};
        if (const uint8_t* q = take(sizeof(T))) memcpy(&v, q, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t k = get<uint64_t>();
        if (!ok) return {};
        if (k > (1u << 24)) {
            char m[128];
            snprintf(m, sizeof m, "GGUF string of %llu bytes at offset %zu — corrupt length", (unsigned long long)k, p);
            *err = m;
            ok = false;
            return {};
        }
        const uint8_t* q = take((size_t)k);
        return q ? std::string((const char*)q, (size_t)k) : std::string();
    }
    // One metadata value of type id ty (enum gguf_type); scalars widen.
    Value value(uint32_t ty, const std::string& key) {
        Value v;
        switch (ty) {
        case 0: v.kind = Value::U; v.u = get<uint8_t>(); break;
        case 1: v.kind = Value::I; v.i = get<int8_t>(); break;
        case 2: v.kind = Value::U; v.u = get<uint16_t>(); break;
        case 3: v.kind = Value::I; v.i = get<int16_t>(); break;
        case 4: v.kind = Value::U; v.u = get<uint32_t>(); break;
        case 5: v.kind = Value::I; v.i = get<int32_t>(); break;
        case 6: v.kind = Value::F; v.f = get<float>(); break;
        case 7: v.kind = Value::B; v.u = get<uint8_t>() != 0; break;
        case 8: v.kind = Value::S; v.s = str(); break;
        case 10: v.kind = Value::U; v.u = get<uint64_t>(); break;
        case 11: v.kind = Value::I; v.i = get<int64_t>(); break;
        case 12: v.kind = Value::F; v.f = get<double>(); break;
        case 9: {
            const uint32_t et = get<uint32_t>();
            const uint64_t cnt = get<uint64_t>();
            if (!ok) break;
            if (cnt > (1u << 26)) {
                *err = "GGUF array " + key + ": corrupt length";
                ok = false;
                break;
            }
            if (et == 9) {
                *err = "GGUF array " + key + ": nested arrays are not supported";
                ok = false;
                break;
            }
            v.kind = Value::ARR;
            v.arr_len = cnt;
            // walk the elements (the tokenizer's strings, per-layer arrays)
            for (uint64_t k = 0; k < cnt && ok; k++) (void)value(et, key);
            break;
        }
        default:
            *err = "GGUF key " + key + ": value type " + std::to_string(ty) + " unsupported";
            ok = false;
        }
        return v;
    }
};

// GGUF tensor name -> HF name (src/gguf/arch.rs:229-270); empty = not read
// by the forward pass (e.g. rope_freqs.weight).
std::string hf_name(const std::string& g) {
    if (g == "token_embd.weight") return "model.embed_tokens.weight";
    if (g == "output_norm.weight") return "model.norm.weight";
    if (g == "output.weight") return "lm_head.weight";
    if (g.compare(0, 4, "blk.") != 0) return {};
    const size_t dot = g.find('.', 4);
    if (dot == std::string::npos) return {};
    const std::string idx = g.substr(4, dot - 4);
    if (idx.empty() || idx.find_first_not_of("0123456789") != std::string::npos) return {};
    const std::string rest = g.substr(dot + 1);
    const size_t d2 = rest.rfind('.');
    if (d2 == std::string::npos) return {};
    const std::string part = rest.substr(0, d2), kind = rest.substr(d2 + 1);
    if (kind != "weight" && kind != "bias") return {};
    static const std::map<std::string, std::string> m = {
        {"attn_norm", "input_layernorm"},      {"ffn_norm", "post_attention_layernorm"},
        {"attn_q", "self_attn.q_proj"},        {"attn_k", "self_attn.k_proj"},
        {"attn_v", "self_attn.v_proj"},        {"attn_output", "self_attn.o_proj"},
        {"attn_q_norm", "self_attn.q_norm"},   {"attn_k_norm", "self_attn.k_norm"},
        {"ffn_gate", "mlp.gate_proj"},         {"ffn_up", "mlp.up_proj"},
        {"ffn_down", "mlp.down_proj"},
    };
    auto it = m.find(part);
    if (it == m.end()) return {};
    return "model.layers." + idx + "." + it->second + "." + kind;
}

}  // namespace

int lk_gguf_open(const char* path, LkGguf* g, std::string* err) {
    *g = LkGguf{};
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        *err = std::string("cannot open ") + path + ": " + strerror(errno);
        return LKHIP_E_IO;
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 4) {
        close(fd);
        *err = std::string(path) + " is not a GGUF file (too short)";
        return LKHIP_E_IO;
    }
    void* map = mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) {
        *err = std::string("cannot map ") + path + ": " + strerror(errno);
        return LKHIP_E_IO;
    }
    g->map = map;
    g->map_len = (size_t)sb.st_size;
    auto fail = [&](int code) {
        lk_gguf_close(g);
        return code;
    };
    Cursor rd{(const uint8_t*)map, (size_t)sb.st_size, 0, err};
    const uint8_t* magic = rd.take(4);
    if (!magic || memcmp(magic, "GGUF", 4) != 0) {
        *err = std::string(path) + " is not a GGUF file (bad magic)";
        return fail(LKHIP_E_IO);
    }
    const uint32_t version = rd.get<uint32_t>();
    if (version == 0x02000000u || version == 0x03000000u) {
        *err = "big-endian GGUF files are not supported — re-export little-endian";
        return fail(LKHIP_E_UNSUPPORTED);
    }
    if (version < 2 || version > 3) {
        *err = "GGUF version " + std::to_string(version) + " unsupported (v2 and v3 only)";
        return fail(LKHIP_E_UNSUPPORTED);
    }
    g->version = version;
    const uint64_t n_tensors = rd.get<uint64_t>();
    const uint64_t n_kv = rd.get<uint64_t>();
    if (!rd.ok) return fail(LKHIP_E_IO);
    std::map<std::string, Value> kv;
    for (uint64_t i = 0; i < n_kv && rd.ok; i++) {
        std::string key = rd.str();
        const uint32_t ty = rd.get<uint32_t>();
        if (!rd.ok) break;
        Value v = rd.value(ty, key);
        kv[key] = std::move(v);
    }
    if (!rd.ok) return fail(LKHIP_E_IO);

    struct Raw {
        std::string name;
        std::vector<uint64_t> ne;
        uint32_t type;
        uint64_t off;
    };
    std::vector<Raw> raw;
    std::map<std::string, std::pair<size_t, std::string>> unsupported;  // type name -> (count, example)
    for (uint64_t i = 0; i < n_tensors && rd.ok; i++) {
        Raw r;
        r.name = rd.str();
        const uint32_t nd = rd.get<uint32_t>();
        if (!rd.ok) break;
        if (nd == 0 || nd > 4) {
            *err = "tensor " + r.name + ": " + std::to_string(nd) + " dimensions";
            return fail(LKHIP_E_IO);
        }
        for (uint32_t d = 0; d < nd; d++) r.ne.push_back(rd.get<uint64_t>());
        r.type = rd.get<uint32_t>();
        r.off = rd.get<uint64_t>();
        if (!rd.ok) break;
        const TypeSize ts = type_size(r.type);
        const bool read_by_forward = !hf_name(r.name).empty();
        if (read_by_forward && !runs(r.type)) {
            // collect every refused type before failing (one run, one verdict)
            const std::string tn = ts.name ? ts.name : ("type " + std::to_string(r.type));
            auto& e = unsupported[tn];
            if (e.first++ == 0) e.second = r.name;
            continue;
        }
        if (!ts.blk) {
            if (read_by_forward) {
                *err = "tensor " + r.name + ": unknown GGUF type " + std::to_string(r.type);
                return fail(LKHIP_E_UNSUPPORTED);
            }
            continue;  // not read, size unknown: skip
        }
        if (r.ne[0] % ts.blk) {
            *err = "tensor " + r.name + ": row length " + std::to_string(r.ne[0]) + " is not a whole number of " +
                   ts.name + " blocks";
            return fail(LKHIP_E_IO);
        }
        raw.push_back(std::move(r));
    }
    if (!rd.ok) return fail(LKHIP_E_IO);
    g->n_file_tensors = (size_t)n_tensors;
    if (!unsupported.empty()) {
        size_t total = 0;
        std::string detail;
        for (auto& [tn, ce] : unsupported) {
            total += ce.first;
            if (!detail.empty()) detail += ", ";
            detail += tn + " (" + std::to_string(ce.first) + (ce.first == 1 ? " tensor" : " tensors") +
                      ", e.g. " + ce.second + ")";
        }
        *err = "this checkpoint uses " + std::to_string(unsupported.size()) +
               " weight type(s) the hip backend does not run, across " + std::to_string(total) + " of " +
               std::to_string(n_tensors) + " tensors: " + detail +
               ". Re-export the model with F16, Q8_0, Q4_0, Q5_0, Q4_K, Q5_K or Q6_K matrices.";
        return fail(LKHIP_E_UNSUPPORTED);
    }

    // data section: next alignment boundary after the header
    uint64_t align = 32;
    if (auto it = kv.find("general.alignment"); it != kv.end()) {
        const Value& v = it->second;
        const uint64_t a = v.kind == Value::U ? v.u : (v.kind == Value::I && v.i > 0 ? (uint64_t)v.i : 0);
        if (a == 0 || (a & (a - 1))) {
            *err = "general.alignment is invalid";
            return fail(LKHIP_E_IO);
        }
        align = a;
    }
    const size_t data_start = (rd.p + align - 1) / align * align;

    // config (src/gguf/arch.rs:164-227)
    auto find = [&](const std::string& k) -> const Value* {
        auto it = kv.find(k);
        return it == kv.end() ? nullptr : &it->second;
    };
    const Value* av = find("general.architecture");
    if (!av || av->kind != Value::S) {
        *err = "GGUF key general.architecture is missing";
        return fail(LKHIP_E_IO);
    }
    g->arch = av->s;
    if (g->arch != "llama" && g->arch != "qwen2") {
        *err = "GGUF architecture \"" + g->arch + "\" is not supported by the hip backend (llama, qwen2 are)";
        return fail(LKHIP_E_UNSUPPORTED);
    }
    std::string missing;
    auto get_u = [&](const std::string& suffix, uint64_t dflt, bool required) -> uint64_t {
        const Value* v = find(g->arch + "." + suffix);
        if (v && v->kind == Value::U) return v->u;
        if (v && v->kind == Value::I && v->i >= 0) return (uint64_t)v->i;
        if (required && missing.empty()) missing = g->arch + "." + suffix;
        return dflt;
    };
    auto get_f = [&](const std::string& suffix, double dflt, bool required) -> double {
        const Value* v = find(g->arch + "." + suffix);
        if (v && v->kind == Value::F) return v->f;
        if (required && missing.empty()) missing = g->arch + "." + suffix;
        return dflt;
    };
    lkhip_config& c = g->cfg;
    c.hidden_size = (uint32_t)get_u("embedding_length", 0, true);
    c.intermediate_size = (uint32_t)get_u("feed_forward_length", 0, true);
    c.num_hidden_layers = (uint32_t)get_u("block_count", 0, true);
    c.num_attention_heads = (uint32_t)get_u("attention.head_count", 0, true);
    c.num_key_value_heads = (uint32_t)get_u("attention.head_count_kv", 0, true);
    c.rms_norm_eps = (float)get_f("attention.layer_norm_rms_epsilon", 0, true);
    c.rope_theta = (float)get_f("rope.freq_base", 10000.0, false);
    c.max_position_embeddings = (uint32_t)get_u("context_length", 4096, false);
    c.head_dim = (uint32_t)get_u("attention.key_length", 0, false);
    if (!missing.empty()) {
        *err = "GGUF key " + missing + " is missing";
        return fail(LKHIP_E_IO);
    }
    // vocab: the token list, else the explicit key, else the embedding rows
    uint64_t vocab = 0;
    if (const Value* t = find("tokenizer.ggml.tokens"); t && t->kind == Value::ARR) vocab = t->arr_len;
    if (!vocab) vocab = get_u("vocab_size", 0, false);

    for (Raw& r : raw) {
        const std::string hf = hf_name(r.name);
        if (hf.empty()) continue;
        const TypeSize ts = type_size(r.type);
        uint64_t n_el = 1;
        for (uint64_t d : r.ne) n_el *= d;
        const uint64_t nbytes = n_el / ts.blk * ts.bytes;
        if (r.off > g->map_len || data_start > g->map_len - r.off || nbytes > g->map_len - data_start - r.off) {
            *err = "tensor " + r.name + ": " + std::to_string(nbytes) + " bytes at data offset " +
                   std::to_string(r.off) + " run past the file";
            return fail(LKHIP_E_IO);
        }
        if (r.ne.size() > 2) {
            *err = "tensor " + r.name + ": " + std::to_string(r.ne.size()) + "-D tensors are not read by the decode step";
            return fail(LKHIP_E_UNSUPPORTED);
        }
        LkGgufTensor t;
        t.name = hf;
        t.gguf_name = r.name;
        t.type = r.type;
        t.n_dims = (uint32_t)r.ne.size();
        if (t.n_dims == 2) {  // GGUF ne is fastest-first: [cols, rows]
            t.dims[0] = r.ne[1];
            t.dims[1] = r.ne[0];
        } else {
            t.dims[0] = r.ne[0];
        }
        t.data = (const uint8_t*)g->map + data_start + r.off;
        t.nbytes = nbytes;
        if (hf == "model.embed_tokens.weight" && !vocab) vocab = t.dims[0];
        g->tensors.push_back(std::move(t));
    }
    c.vocab_size = (uint32_t)vocab;
    g->llama_permuted = g->arch == "llama";  // the converter permutes llama q/k rows (arch.rs:271-286)
    return LKHIP_OK;
}

void lk_gguf_close(LkGguf* g) {
    if (g->map) munmap(g->map, g->map_len);
    g->map = nullptr;
    g->map_len = 0;
    g->tensors.clear();
}
