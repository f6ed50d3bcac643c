// layer_ops.h -- internal interface of the decoder-layer kernels around the
// quantized matmuls: RMSNorm, SwiGLU, residual add, RoPE (+ fused q/k norm
// and KV-cache store), embedding-row dequant and greedy argmax.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jllm_hip {

constexpr int ROPE_MAX_HALF = 64;          // head_dim <= 128

// Per-call rotary frequencies, computed on the host and passed by value:
// freq[i] = 1 / theta^(2i / head_dim) for the head_dim/2 pairs.
struct RopeFreq {
    float f[ROPE_MAX_HALF];
};
void rope_frequencies(RopeFreq& fr, int head_dim, float theta);

hipError_t rmsnorm_launch(uint16_t* out, const uint16_t* x, const uint16_t* res, const void* w, int rows, int dim,
                          float eps, bool w_fp32, hipStream_t st);
hipError_t swiglu_launch(uint16_t* out, const uint16_t* gate, const uint16_t* up, int64_t n, hipStream_t st);
hipError_t vec_add_launch(uint16_t* out, const uint16_t* a, const uint16_t* b, int64_t n, hipStream_t st);

// q [N][q_stride], k [N][k_stride] rotated in place; token t at position
// start_pos + t, or *pos_dev + t when pos_dev is not null (read on the
// device, so a captured graph stays valid for every position).  k may be
// null (n_kv = 0).
hipError_t rope_launch(uint16_t* q, uint16_t* k, int n_heads, int n_kv, int head_dim, int start_pos, int N,
                       int q_stride, int k_stride, const RopeFreq& fr, bool neox, hipStream_t st,
                       const int* pos_dev = nullptr);

// Post-projection step of attention for N tokens: optional q/k RMSNorm
// (weights q_norm/k_norm, fp32 or fp16), RoPE of q and k (both in place),
// then k and v stored into the cache rows of positions start_pos + t: int8
// with a per-(position, kv head) absmax scale, or fp16 copies.  The cache
// pointers address the row of position start_pos.
struct QKPostArgs {
    uint16_t* q;              // [N][n_heads * hd]
    uint16_t* k;              // [N][n_kv * hd]
    const uint16_t* v;        // [N][n_kv * hd]
    const void* q_norm;       // [hd] or null (no q RMSNorm)
    const void* k_norm;       // [hd] or null (no k RMSNorm)
    void* k_dst;              // row t at t * kv_stride elements, head h at h * cache_head_dim
    void* v_dst;
    float* k_scales;          // [t][n_kv] (int8 only; may be null)
    float* v_scales;
    int64_t kv_stride;
    int n_heads, n_kv, head_dim, cache_head_dim, start_pos, N;
    float eps;
    int norm_fp32, neox, kv_int8;
    RopeFreq fr;
    // input row strides (elements) of q and of k / v; 0 = packed rows
    int64_t q_in_stride = 0, kv_in_stride = 0;
    // when not null the first position is *pos_dev (read on the device) and
    // k_dst / v_dst / k_scales / v_scales address position 0 of the layer
    const int* pos_dev = nullptr;
};
hipError_t qk_post_launch(const QKPostArgs& a, hipStream_t st);

// rows for tokens[t] (device array) or, when tokens is null, token0; with
// vocab > 0 an id outside [0, vocab) yields a zero row
hipError_t embed_launch(uint16_t* dst, const void* W, int type, const int32_t* tokens, int token0, int N, int hidden,
                        int vocab, hipStream_t st);
hipError_t argmax_launch(int32_t* out, const float* x, int n, hipStream_t st);

}  // namespace jllm_hip
