// attention.h -- internal interface of the gfx950 split-K decode attention.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jllm_hip {

struct AttnArgs {
    uint16_t* out;            // fp16 [n_heads x head_dim]
    const uint16_t* q;        // fp16 [n_heads x head_dim]
    const void* k;            // int8 or fp16 [seq][n_kv * cache_head_dim]
    const void* v;
    const float* ks;          // fp32 [pos][n_kv] (int8 only; may be null -> 1)
    const float* vs;
    float* part;              // partials: m [H*S] | l [H*S] | acc [H*S*hd]
    int n_heads, n_kv, head_dim, cache_head_dim, seq, window, n_splits;
    float scale;
};

int attn_splits(int seq_len, int n_kv);
size_t attn_partials_floats(int n_heads, int n_splits, int head_dim);
hipError_t attn_launch(const AttnArgs& a, bool kv_int8, hipStream_t st);

}  // namespace jllm_hip
