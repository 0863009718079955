// gguf.h -- the GGUF v2/v3 container reader behind lkhip_engine_create_gguf
// (GgufFile::open, src/gguf/container.rs:162-261; model_config and hf_name,
// src/gguf/arch.rs:164-270).  Host code only.
#pragma once
#include <stdint.h>
#include <stddef.h>

#include <string>
#include <vector>

#include "../../include/lokal_hip.h"

// One tensor of the file, named the HF way, its bytes inside the mapping.
struct LkGgufTensor {
    std::string name;      // HF name (model.layers.N.self_attn.q_proj.weight, ...)
    std::string gguf_name; // as written in the file (blk.N.attn_q.weight, ...)
    uint32_t type = 0;     // GGUF type id
    uint32_t n_dims = 0;
    uint64_t dims[2] = {0, 0};  // row-major: [rows, cols] (n_dims 1: [n])
    const uint8_t* data = nullptr;
    uint64_t nbytes = 0;
};

struct LkGguf {
    uint32_t version = 0;
    std::string arch;
    lkhip_config cfg{};
    bool llama_permuted = false;  // q/k rows carry the llama converter's permutation
    std::vector<LkGgufTensor> tensors;  // only those the forward pass reads
    size_t n_file_tensors = 0;
    // the file mapping; released by lk_gguf_close
    void* map = nullptr;
    size_t map_len = 0;
};

// Parses `path`.  0 on success; otherwise an LKHIP_E_* code with the reason
// in *err (one line, the reference's refusal style).
int lk_gguf_open(const char* path, LkGguf* out, std::string* err);
void lk_gguf_close(LkGguf* g);
