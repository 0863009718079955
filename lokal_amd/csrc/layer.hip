// layer.hip -- the small fused layer kernels of the decode step: RMSNorm,
// RoPE-pair rotation (+ the f16 KV-cache write), SwiGLU, argmax, and the
// per-step bookkeeping kernel that feeds the next token on the device.
#include "lkhip_common.h"

// ---------------------------------------------------------------- RMSNorm
// math::rmsnorm (src/math.rs:45-49): s = 1/sqrt(dot(x,x)/n + eps); y = (x*s)*w.
// One block per row; fp32 sum of squares by wave reductions.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      uint32_t n, float eps, float* __restrict__ y) {
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    __shared__ float part[4];
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
    ss = lk_wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += 256) yr[i] = __fmul_rn(__fmul_rn(xr[i], scale), w[i]);
}

hipError_t lk_rmsnorm_launch(const float* x, const float* w, uint32_t rows, uint32_t n, float eps, float* y,
                             hipStream_t st) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, st, x, w, n, eps, y);
    return hipGetLastError();
}

// ------------------------------------------------------------------- RoPE
// model::rope (src/model.rs:268-279): pair (i, i+hd/2) of each head turns by
// pos * theta^(-2i/hd) (lk_rot_pair).

// The inverse frequencies of a by-value LkFreq, copied into LDS with
// compile-time indices.  Indexed by a lane-varying i as a kernel argument,
// the table made the compiler copy the whole struct into every thread's
// scratch at kernel entry (~40 MB of scratch writes per launch at 512 rows).
// Call before any early return: it ends with a block barrier.
#define LK_FREQ_TO_LDS(fr, fs)                                \
    __shared__ float fs[64];                                  \
    if (threadIdx.x == 0) {                                   \
        _Pragma("unroll") for (int k_ = 0; k_ < 64; k_++) fs[k_] = (fr).f[k_]; \
    }                                                         \
    __syncthreads()

__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ x, uint32_t rows, uint32_t n, uint32_t hd,
                                                   const uint32_t* __restrict__ pos, const LkFreq fr) {
    LK_FREQ_TO_LDS(fr, fs);
    const uint32_t half = hd / 2;
    const uint32_t pairs_per_row = n / 2;
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (size_t)rows * pairs_per_row) return;
    const uint32_t r = (uint32_t)(t / pairs_per_row), pr = (uint32_t)(t % pairs_per_row);
    const uint32_t head = pr / half, i = pr % half;
    float* hx = x + (size_t)r * n + (size_t)head * hd;
    float a = hx[i], b = hx[i + half];
    lk_rot_pair(a, b, __fmul_rn((float)pos[r], fs[i]));
    hx[i] = a;
    hx[i + half] = b;
}

hipError_t lk_rope_launch(float* x, uint32_t rows, uint32_t n, uint32_t head_dim, const uint32_t* pos,
                          const LkFreq& freq, hipStream_t st) {
    const size_t total = (size_t)rows * (n / 2);
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, rows, n, head_dim,
                       pos, freq);
    return hipGetLastError();
}

// Decode step: rotate q in place and k, then write k and v of this position
// into the f16 cache laid out [slot][kv_head][max_seq][64] (the KV append of
// src/model.rs:228-231, stored f16 as the GPU path does).  qkv rows are
// [q (n_heads*64) | k (n_kv*64) | v (n_kv*64)].
__device__ __forceinline__ void kv_store(uint16_t* p, float v) { *p = __half_as_ushort(__float2half_rn(v)); }
__device__ __forceinline__ void kv_store(float* p, float v) { *p = v; }

template <typename KV>
__global__ __launch_bounds__(256) void rope_kv_kernel(float* __restrict__ qkv, uint32_t n_heads, uint32_t n_kv,
                                                      const LkFreq fr, const LkStepState* __restrict__ st,
                                                      const uint32_t* __restrict__ pos_rows,
                                                      KV* __restrict__ kc, KV* __restrict__ vc,
                                                      uint32_t max_seq, uint64_t slot_stride,
                                                      const uint32_t* __restrict__ slots) {
    LK_FREQ_TO_LDS(fr, fs);
    const uint32_t r = blockIdx.y;
    const uint32_t pos = pos_rows ? pos_rows[r] : st->pos;
    const uint32_t slot = slots ? slots[r] : r;
    const uint32_t qd = n_heads * 64, kvd = n_kv * 64;
    float* row = qkv + (size_t)r * (qd + 2 * kvd);
    const uint32_t t = blockIdx.x * 256 + threadIdx.x;
    const uint32_t nq_pairs = n_heads * 32, nk_pairs = n_kv * 32;
    const float fpos = (float)pos;
    if (t < nq_pairs) {
        const uint32_t head = t / 32, i = t % 32;
        float* h = row + head * 64;
        float a = h[i], b = h[i + 32];
        lk_rot_pair(a, b, __fmul_rn(fpos, fs[i]));
        h[i] = a;
        h[i + 32] = b;
    } else if (t < nq_pairs + nk_pairs) {
        const uint32_t u = t - nq_pairs, head = u / 32, i = u % 32;
        float* h = row + qd + head * 64;
        float a = h[i], b = h[i + 32];
        lk_rot_pair(a, b, __fmul_rn(fpos, fs[i]));
        h[i] = a;
        h[i + 32] = b;
        KV* dst = kc + (size_t)slot * slot_stride + ((size_t)head * max_seq + pos) * 64;
        kv_store(dst + i, a);
        kv_store(dst + i + 32, b);
    } else if (t < nq_pairs + nk_pairs + kvd) {
        const uint32_t u = t - nq_pairs - nk_pairs, head = u / 64, d = u % 64;
        const float v = row[qd + kvd + u];
        kv_store(vc + (size_t)slot * slot_stride + ((size_t)head * max_seq + pos) * 64 + d, v);
    }
}

hipError_t lk_rope_kv_launch(float* qkv, uint32_t n_heads, uint32_t n_kv, const LkFreq& freq,
                             const LkStepState* st_dev, const uint32_t* pos_rows, uint32_t n_rows, void* kcache,
                             void* vcache, int kv_f32, uint32_t max_seq, uint64_t slot_stride, const uint32_t* slots,
                             hipStream_t st) {
    const uint32_t work = n_heads * 32 + n_kv * 32 + n_kv * 64;
    dim3 grid((work + 255) / 256, n_rows);
    if (kv_f32)
        hipLaunchKernelGGL(rope_kv_kernel<float>, grid, dim3(256), 0, st, qkv, n_heads, n_kv, freq, st_dev, pos_rows,
                           (float*)kcache, (float*)vcache, max_seq, slot_stride, slots);
    else
        hipLaunchKernelGGL(rope_kv_kernel<uint16_t>, grid, dim3(256), 0, st, qkv, n_heads, n_kv, freq, st_dev,
                           pos_rows, (uint16_t*)kcache, (uint16_t*)vcache, max_seq, slot_stride, slots);
    return hipGetLastError();
}

// ----------------------------------------------------------------- SwiGLU
// src/model.rs:247-249 with math::silu (src/math.rs:68-70): silu(g) * u,
// silu(x) = x / (1 + exp(-x)).
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     uint32_t n, float* __restrict__ out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float x = g[i];
    out[i] = __fmul_rn(x / (1.0f + expf(-x)), u[i]);
}

hipError_t lk_swiglu_launch(const float* g, const float* u, uint32_t n, float* out, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, st, g, u, n, out);
    return hipGetLastError();
}

// ----------------------------------------------------------------- argmax
__device__ __forceinline__ uint64_t max_key_block(uint64_t k) {
    __shared__ uint64_t part[16];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = __shfl_xor(k, m, 64);
        k = o > k ? o : k;
    }
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nw = (blockDim.x + 63) / 64;
        for (int w = 1; w < nw; w++) k = part[w] > k ? part[w] : k;
        part[0] = k;
    }
    __syncthreads();
    return part[0];
}

// sampler::argmax (src/sampler.rs:67-75) per row, first max wins.
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float* __restrict__ x, uint32_t n,
                                                           uint32_t* __restrict__ out) {
    const float* xr = x + (size_t)blockIdx.x * n;
    uint64_t k = 0;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const uint64_t kk = lk_argmax_key(xr[i], i);
        k = kk > k ? kk : k;
    }
    k = max_key_block(k);
    if (threadIdx.x == 0) out[blockIdx.x] = lk_argmax_idx(k);
}

hipError_t lk_argmax_rows_launch(const float* x, uint32_t rows, uint32_t n, uint32_t* out, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(1024), 0, st, x, n, out);
    return hipGetLastError();
}

// End of a decode step: fold the lm_head's per-block argmax keys, then either
// feed the next prompt id (prefill) or the argmax (greedy decode, as
// generate.rs:101-118 does at -t 0), and advance the position.
__global__ __launch_bounds__(1024) void step_finish_kernel(const uint64_t* __restrict__ keys, uint32_t n_keys,
                                                           LkStepState* __restrict__ st,
                                                           const uint32_t* __restrict__ feed,
                                                           uint32_t* __restrict__ ids_out) {
    uint64_t k = 0;
    for (uint32_t i = threadIdx.x; i < n_keys; i += blockDim.x) k = keys[i] > k ? keys[i] : k;
    k = max_key_block(k);
    if (threadIdx.x == 0) {
        const uint32_t best = lk_argmax_idx(k);
        LkStepState s = *st;
        if (s.n_feed > 0) {
            s.token = feed[s.fed];
            s.fed += 1;
            s.n_feed -= 1;
        } else {
            if (ids_out) ids_out[s.n_out] = best;
            s.n_out += 1;
            s.token = best;
        }
        s.pos += 1;
        *st = s;
    }
}

hipError_t lk_step_finish_launch(const uint64_t* keys, uint32_t n_keys, LkStepState* st_dev, const uint32_t* feed_ids,
                                 uint32_t* ids_out, hipStream_t st) {
    hipLaunchKernelGGL(step_finish_kernel, dim3(1), dim3(1024), 0, st, keys, n_keys, st_dev, feed_ids, ids_out);
    return hipGetLastError();
}

// ------------------------------------------------ rows-path fused consumers
// The residual add of a split-K GEMM's partials (src/model.rs:235-237,
// :253-255; summed in split order, as gemm_reduce_kernel would) fused with the
// RMSNorm that reads the new residual (src/math.rs:45-49).  One block per row.
__global__ __launch_bounds__(1024) void rows_accnorm_kernel(float* __restrict__ x, const float* __restrict__ part,
                                                            uint32_t ks, uint32_t rows, uint32_t n,
                                                            const float* __restrict__ w, float eps,
                                                            float* __restrict__ y) {
    // 1024 threads: one element each at the model widths, so a thread's ks
    // partial loads are all in flight together
    const uint32_t r = blockIdx.x;
    float* xr = x + (size_t)r * n;
    __shared__ float red[16];
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += 1024) {
        float v = xr[i];
        if (ks) {
            v += lk_sum_splits(part + (size_t)r * n + i, (size_t)rows * n, ks);
            xr[i] = v;
        }
        ss = fmaf(v, v, ss);
    }
    ss = lk_wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) tot += red[i];
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += 1024) y[(size_t)r * n + i] = __fmul_rn(__fmul_rn(xr[i], scale), w[i]);
}

hipError_t lk_rows_accnorm_launch(float* x, const float* part, uint32_t ks, uint32_t rows, uint32_t n,
                                  const float* w, float eps, float* y, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(rows_accnorm_kernel, dim3(rows), dim3(1024), 0, st, x, part, ks, rows, n, w, eps, y);
    return hipGetLastError();
}

// The QKV split-K sum (+ q/k/v bias, src/model.rs:27-35) fused with RoPE and
// the KV append of rope_kv_kernel.
template <typename KV>
__global__ __launch_bounds__(256) void rows_rope_kv_kernel(float* __restrict__ qkv, const float* __restrict__ part,
                                                           uint32_t ks, const float* __restrict__ bq,
                                                           const float* __restrict__ bk,
                                                           const float* __restrict__ bv, uint32_t n_heads,
                                                           uint32_t n_kv, const LkFreq fr,
                                                           const uint32_t* __restrict__ pos_rows, uint32_t rows,
                                                           KV* __restrict__ kc, KV* __restrict__ vc,
                                                           uint32_t max_seq, uint64_t slot_stride,
                                                           const uint32_t* __restrict__ slots) {
    LK_FREQ_TO_LDS(fr, fs);
    const uint32_t r = blockIdx.y;
    const uint32_t pos = pos_rows[r];
    const uint32_t slot = slots[r];
    const uint32_t qd = n_heads * 64, kvd = n_kv * 64, qkvd = qd + 2 * kvd;
    float* row = qkv + (size_t)r * qkvd;
    // element idx of the row, with bias b[bi] (the caller names q, k or v's
    // bias: a select between the three pointers had become a lookup table in
    // scratch, and by-reference captures had put the arguments there too)
    auto val = [=](uint32_t idx, const float* b, uint32_t bi) -> float {
        if (!ks) return row[idx];
        const float a = lk_sum_splits(part + (size_t)r * qkvd + idx, (size_t)rows * qkvd, ks);
        return b ? a + b[bi] : a;
    };
    const uint32_t t = blockIdx.x * 256 + threadIdx.x;
    const uint32_t nq_pairs = n_heads * 32, nk_pairs = n_kv * 32;
    const float fpos = (float)pos;
    if (t < nq_pairs) {
        const uint32_t head = t / 32, i = t % 32;
        const uint32_t o = head * 64 + i;
        float a = val(o, bq, o), b = val(o + 32, bq, o + 32);
        lk_rot_pair(a, b, __fmul_rn(fpos, fs[i]));
        row[o] = a;
        row[o + 32] = b;
    } else if (t < nq_pairs + nk_pairs) {
        const uint32_t u = t - nq_pairs, head = u / 32, i = u % 32;
        const uint32_t o = qd + head * 64 + i;
        float a = val(o, bk, o - qd), b = val(o + 32, bk, o - qd + 32);
        lk_rot_pair(a, b, __fmul_rn(fpos, fs[i]));
        KV* dst = kc + (size_t)slot * slot_stride + ((size_t)head * max_seq + pos) * 64;
        kv_store(dst + i, a);
        kv_store(dst + i + 32, b);
    } else if (t < nq_pairs + nk_pairs + kvd) {
        const uint32_t u = t - nq_pairs - nk_pairs, head = u / 64, d = u % 64;
        kv_store(vc + (size_t)slot * slot_stride + ((size_t)head * max_seq + pos) * 64 + d, val(qd + kvd + u, bv, u));
    }
}

hipError_t lk_rows_rope_kv_launch(float* qkv, const float* part, uint32_t ks, const float* bq, const float* bk,
                                  const float* bv, uint32_t n_heads, uint32_t n_kv, const LkFreq& freq,
                                  const uint32_t* pos_rows, uint32_t n_rows, void* kcache, void* vcache, int kv_f32,
                                  uint32_t max_seq, uint64_t slot_stride, const uint32_t* slots, hipStream_t st) {
    if (n_rows == 0) return hipSuccess;
    const uint32_t work = n_heads * 32 + n_kv * 32 + n_kv * 64;
    dim3 grid((work + 255) / 256, n_rows);
    if (kv_f32)
        hipLaunchKernelGGL(rows_rope_kv_kernel<float>, grid, dim3(256), 0, st, qkv, part, ks, bq, bk, bv, n_heads,
                           n_kv, freq, pos_rows, n_rows, (float*)kcache, (float*)vcache, max_seq, slot_stride, slots);
    else
        hipLaunchKernelGGL(rows_rope_kv_kernel<uint16_t>, grid, dim3(256), 0, st, qkv, part, ks, bq, bk, bv, n_heads,
                           n_kv, freq, pos_rows, n_rows, (uint16_t*)kcache, (uint16_t*)vcache, max_seq, slot_stride,
                           slots);
    return hipGetLastError();
}

// Greedy step of a batch of sequences (generate.rs:101-118 at -t 0, one row
// per sequence) in two passes: every block takes the first-max key
// (src/sampler.rs:67-75) of one LK_ARGMAX_SLICE-wide slice of one row, then
// one wave per row folds the slice keys, records the winner as the row's next
// output id (out_ids is [step][n_rows]) and feeds it back as the row's next
// token at the next position.  meta holds u32 arrays
// [ids | pos | slots | ctx | steps], each `cap` long.
__global__ __launch_bounds__(256) void argmax_slices_kernel(const float* __restrict__ x, uint32_t n,
                                                            uint64_t* __restrict__ keys) {
    const uint32_t r = blockIdx.y, sl = blockIdx.x, ns = gridDim.x;
    const float* xr = x + (size_t)r * n;
    const uint32_t i0 = sl * LK_ARGMAX_SLICE, i1 = i0 + LK_ARGMAX_SLICE < n ? i0 + LK_ARGMAX_SLICE : n;
    uint64_t k = 0;
    for (uint32_t i = i0 + threadIdx.x; i < i1; i += 256) {
        const uint64_t kk = lk_argmax_key(xr[i], i);
        k = kk > k ? kk : k;
    }
    k = max_key_block(k);
    if (threadIdx.x == 0) keys[(size_t)r * ns + sl] = k;
}

__global__ __launch_bounds__(64) void rows_fold_kernel(const uint64_t* __restrict__ keys, uint32_t ns,
                                                       uint32_t* __restrict__ meta, uint32_t cap, uint32_t n_rows,
                                                       uint32_t* __restrict__ out_ids) {
    const uint32_t r = blockIdx.x;
    uint64_t k = 0;
    for (uint32_t i = threadIdx.x; i < ns; i += 64) k = keys[(size_t)r * ns + i] > k ? keys[(size_t)r * ns + i] : k;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = __shfl_xor(k, m, 64);
        k = o > k ? o : k;
    }
    if (threadIdx.x == 0) {
        const uint32_t id = lk_argmax_idx(k);
        uint32_t* ids = meta;
        uint32_t* pos = meta + cap;
        uint32_t* ctx = meta + 3 * cap;
        uint32_t* steps = meta + 4 * cap;
        out_ids[(size_t)steps[r] * n_rows + r] = id;
        steps[r] += 1;
        ids[r] = id;
        pos[r] += 1;
        ctx[r] = pos[r] + 1;
    }
}

hipError_t lk_rows_greedy2_launch(const float* logits, uint32_t n_rows, uint32_t n, uint64_t* keys, uint32_t* meta,
                                  uint32_t cap, uint32_t* out_ids, hipStream_t st) {
    if (n_rows == 0) return hipSuccess;
    const uint32_t ns = (n + LK_ARGMAX_SLICE - 1) / LK_ARGMAX_SLICE;
    hipLaunchKernelGGL(argmax_slices_kernel, dim3(ns, n_rows), dim3(256), 0, st, logits, n, keys);
    hipLaunchKernelGGL(rows_fold_kernel, dim3(n_rows), dim3(64), 0, st, keys, ns, meta, cap, n_rows, out_ids);
    return hipGetLastError();
}
