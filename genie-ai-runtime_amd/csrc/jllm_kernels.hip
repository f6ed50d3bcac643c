// jllm_kernels.hip -- the namespace jllm C++ entry points (the reference's
// include/jllm_kernels.h signatures) as thin forwards to the C ABI.
#include "jllm_kernels.h"
#include "jllm_hip.h"
#include "kq_common.h"
#include "fill_size.h"
#include <cstdio>

namespace {

using jllm_fill::fill_bytes;

__global__ void zero_fill_kernel(uint8_t* p, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

// zero `bytes` bytes at p on the stream, with a kernel (no memset node, so a
// captured graph replays it correctly); sizes come from fill_bytes, which is
// 0 for a negative or overflowing shape
void zero_fill(void* p, size_t bytes, hipStream_t st) {
    if (!p || bytes == 0) return;
    const size_t blocks = (bytes + 255) / 256 < 4096 ? (bytes + 255) / 256 : 4096;
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (uint8_t*)p, bytes);
}

void report(int st, const char* fn, void* out, size_t bytes, hipStream_t stream) {
    if (st == JLLM_OK) return;
    fprintf(stderr, "[jllm] %s failed: %s; %s\n", fn, jllm_hip_status_string(st),
            out && bytes ? "output zero-filled" : "data left unchanged");
    zero_fill(out, bytes, stream);
}

inline const uint16_t* H(const half* p) { return reinterpret_cast<const uint16_t*>(p); }
inline uint16_t* H(half* p) { return reinterpret_cast<uint16_t*>(p); }

}  // namespace

namespace jllm {

void gemv_q4(half* y, const void* W_q4, const half*, const half* x, int M, int K, int, hipStream_t stream) {
    gemv_quant(y, W_q4, 12, x, M, K, stream);
}

void gemv_quant(half* y, const void* W, int type, const half* x, int M, int K, hipStream_t stream) {
    report(jllm_hip_gemv_quant(H(y), W, type, H(x), M, K, stream), "gemv_quant", y, fill_bytes({M}, 2), stream);
}

void gemv_quant_add(half* y, const void* W, int type, const half* x, const half* residual, int M, int K,
                    hipStream_t stream) {
    report(jllm_hip_gemv_quant_add(H(y), W, type, H(x), H(residual), M, K, stream), "gemv_quant_add", y,
           fill_bytes({M}, 2), stream);
}

void gemv_quant_pair(half* y0, const void* W0, int t0, int M0, half* y1, const void* W1, int t1, int M1,
                     const half* x, int K, hipStream_t stream) {
    const int st = jllm_hip_gemv_quant_pair(H(y0), W0, t0, M0, H(y1), W1, t1, M1, H(x), K, stream);
    report(st, "gemv_quant_pair", y0, fill_bytes({M0}, 2), stream);
    if (st) zero_fill(y1, fill_bytes({M1}, 2), stream);
}

void gemv_quant_triple(half* y0, const void* W0, int t0, int M0, half* y1, const void* W1, int t1, int M1,
                       half* y2, const void* W2, int t2, int M2, const half* x, int K, hipStream_t stream) {
    const int st = jllm_hip_gemv_quant_triple(H(y0), W0, t0, M0, H(y1), W1, t1, M1, H(y2), W2, t2, M2, H(x), K,
                                              stream);
    report(st, "gemv_quant_triple", y0, fill_bytes({M0}, 2), stream);
    if (st) { zero_fill(y1, fill_bytes({M1}, 2), stream); zero_fill(y2, fill_bytes({M2}, 2), stream); }
}

void gemv_quant_f32(float* y, const void* W, int type, const half* x, int M, int K, hipStream_t stream) {
    report(jllm_hip_gemv_quant_f32(y, W, type, H(x), M, K, stream), "gemv_quant_f32", y, fill_bytes({M}, 4), stream);
}

void gemm_quant_batched(half* y, const void* W, int type, const half* x, int M, int N, int K, hipStream_t stream) {
    report(jllm_hip_gemm_quant_batched(H(y), W, type, H(x), M, N, K, stream), "gemm_quant_batched", y,
           fill_bytes({M, N}, 2), stream);
}

void quantize_q8_1(const half* x, void* y, int K, hipStream_t stream) {
    report(jllm_hip_quantize_q8_1(H(x), y, K, stream), "quantize_q8_1", y, fill_bytes({K / 32}, 36), stream);
}

void gemm_q4k_mmq_llama(half* y, const void* W, const half* x, int M, int N, int K, hipStream_t stream) {
    gemm_quant_batched(y, W, 12, x, M, N, K, stream);
}

void gemm_q6k_mmq_llama(half* y, const void* W, const half* x, int M, int N, int K, hipStream_t stream) {
    gemm_quant_batched(y, W, 14, x, M, N, K, stream);
}

void flash_attention_decode(half* output, const half* q, const void* k_cache, const void* v_cache, int n_heads,
                            int n_kv_heads, int head_dim, int cache_head_dim, int seq_len, float scale,
                            bool kv_int8, const float* k_scales, const float* v_scales, int window,
                            hipStream_t stream) {
    report(jllm_hip_flash_attention_decode(H(output), H(q), k_cache, v_cache, n_heads, n_kv_heads, head_dim,
                                           cache_head_dim, seq_len, scale, kv_int8 ? 1 : 0, k_scales, v_scales,
                                           window, stream),
           "flash_attention_decode", output, fill_bytes({n_heads, head_dim}, 2), stream);
}

void flash_attention_decode_dyn(half* output, const half* q, const void* k_cache, const void* v_cache, int n_heads,
                                int n_kv_heads, int head_dim, int cache_head_dim, const int* d_pos, float scale,
                                bool kv_int8, const float* kv_scales, int window, int n_splits, hipStream_t stream) {
    const size_t bytes = fill_bytes({n_heads, head_dim}, 2);
    if (kv_int8) {
        fprintf(stderr, "[jllm] flash_attention_decode_dyn: an INT8 cache needs separate K and V scales (use the "
                        "overload taking k_scales and v_scales); output zero-filled\n");
        zero_fill(output, bytes, stream);
        return;
    }
    (void)kv_scales;
    report(jllm_hip_flash_attention_decode_dyn(H(output), H(q), k_cache, v_cache, n_heads, n_kv_heads, head_dim,
                                               cache_head_dim, d_pos, scale, 0, nullptr, nullptr, window, n_splits,
                                               stream),
           "flash_attention_decode_dyn", output, bytes, stream);
}

void flash_attention_decode_dyn(half* output, const half* q, const void* k_cache, const void* v_cache, int n_heads,
                                int n_kv_heads, int head_dim, int cache_head_dim, const int* d_pos, float scale,
                                bool kv_int8, const float* k_scales, const float* v_scales, int window, int n_splits,
                                hipStream_t stream) {
    report(jllm_hip_flash_attention_decode_dyn(H(output), H(q), k_cache, v_cache, n_heads, n_kv_heads, head_dim,
                                               cache_head_dim, d_pos, scale, kv_int8 ? 1 : 0, k_scales, v_scales,
                                               window, n_splits, stream),
           "flash_attention_decode_dyn", output, fill_bytes({n_heads, head_dim}, 2), stream);
}

// in-place on fp32 logits: left unchanged on failure
void softmax_inplace(float* x, int n, hipStream_t stream) {
    report(jllm_hip_softmax_inplace(x, n, stream), "softmax_inplace", nullptr, 0, stream);
}

int decode_attn_splits(int seq_len) { return jllm_hip_decode_attn_splits(seq_len); }

float* get_splitk_partials(int n_heads, int n_splits, int head_dim) {
    return jllm_hip_get_splitk_partials(n_heads, n_splits, head_dim);
}

void fp16_to_int8(int8_t* dst, float* scale_out, const half* src, int rows, int cols, hipStream_t stream) {
    const int st = jllm_hip_fp16_to_int8(dst, scale_out, H(src), rows, cols, stream);
    report(st, "fp16_to_int8", dst, fill_bytes({rows, cols}, 1), stream);
    if (st) zero_fill(scale_out, fill_bytes({rows}, 4), stream);
}

bool dequant_embedding_row(half* dst, const void* W, int ggml_type, int token_id, int hidden_dim, hipStream_t stream) {
    const int st = jllm_hip_dequant_embedding_row(H(dst), W, ggml_type, token_id, hidden_dim, stream);
    report(st, "dequant_embedding_row", dst, fill_bytes({hidden_dim}, 2), stream);
    return st == JLLM_OK;
}

void fused_rmsnorm_residual(half* output, const half* x, const half* residual, const void* weight, int rows,
                            int hidden_dim, float eps, bool weight_fp32, hipStream_t stream) {
    report(jllm_hip_fused_rmsnorm_residual(H(output), H(x), H(residual), weight, rows, hidden_dim, eps,
                                           weight_fp32 ? 1 : 0, stream),
           "fused_rmsnorm_residual", output, fill_bytes({rows, hidden_dim}, 2),
           stream);
}

void fused_swiglu(half* output, const half* gate, const half* up, int rows, int intermediate_dim, hipStream_t stream) {
    report(jllm_hip_fused_swiglu(H(output), H(gate), H(up), rows, intermediate_dim, stream), "fused_swiglu", output,
           fill_bytes({rows, intermediate_dim}, 2), stream);
}

void rope_precompute_table(int max_seq, int head_dim, float theta_base) {
    (void)jllm_hip_rope_precompute_table(max_seq, head_dim, theta_base);
}
void rope_clear_tables() { jllm_hip_rope_clear_tables(); }

// in-place operations: on failure the data is left as it was (no zero fill)
void rope_inplace(half* q, half* k, int n_heads, int n_kv_heads, int head_dim, int position, float theta_base,
                  bool neox, hipStream_t stream) {
    report(jllm_hip_rope_inplace(H(q), H(k), n_heads, n_kv_heads, head_dim, position, theta_base, neox ? 1 : 0,
                                 stream),
           "rope_inplace", nullptr, 0, stream);
}

void rope_inplace_batched(half* q, half* k, int n_heads, int n_kv_heads, int head_dim, int start_pos, int N,
                          int q_stride, int k_stride, float theta_base, bool neox, hipStream_t stream) {
    report(jllm_hip_rope_inplace_batched(H(q), H(k), n_heads, n_kv_heads, head_dim, start_pos, N, q_stride, k_stride,
                                         theta_base, neox ? 1 : 0, stream),
           "rope_inplace_batched", nullptr, 0, stream);
}

void rope_inplace_store_kv_fp16(half* q, half* k, const half* v, half* k_cache_dst, half* v_cache_dst, int n_heads,
                                int n_kv_heads, int head_dim, int position, float theta_base, bool neox,
                                hipStream_t stream) {
    report(jllm_hip_qk_norm_rope_store_kv(H(q), H(k), H(v), nullptr, nullptr, 0, 0.0f, k_cache_dst, v_cache_dst,
                                          nullptr, nullptr, (int64_t)n_kv_heads * head_dim, n_heads, n_kv_heads,
                                          head_dim, head_dim, position, 1, theta_base, neox ? 1 : 0, 0, stream),
           "rope_inplace_store_kv_fp16", nullptr, 0, stream);
}

void rope_inplace_store_kv_fp16_batched(half* q, half* k, const half* v, half* k_cache_base, half* v_cache_base,
                                        int kv_slot, int n_heads, int n_kv_heads, int head_dim, int start_pos, int N,
                                        int q_stride, int kv_stride, float theta_base, bool neox, hipStream_t stream) {
    report(jllm_hip_rope_inplace_store_kv_fp16_batched(H(q), H(k), H(v), H(k_cache_base), H(v_cache_base), kv_slot,
                                                       n_heads, n_kv_heads, head_dim, start_pos, N, q_stride,
                                                       kv_stride, theta_base, neox ? 1 : 0, stream),
           "rope_inplace_store_kv_fp16_batched", nullptr, 0, stream);
}

void rope_inplace_store_kv_fp16_dyn(half* q, half* k, const half* v, half* k_cache_layer_base,
                                    half* v_cache_layer_base, int n_heads, int n_kv_heads, int head_dim,
                                    int cache_head_dim, const int* d_pos, float theta_base, bool neox,
                                    hipStream_t stream) {
    report(jllm_hip_rope_inplace_store_kv_fp16_dyn(H(q), H(k), H(v), H(k_cache_layer_base), H(v_cache_layer_base),
                                                   n_heads, n_kv_heads, head_dim, cache_head_dim, d_pos, theta_base,
                                                   neox ? 1 : 0, stream),
           "rope_inplace_store_kv_fp16_dyn", nullptr, 0, stream);
}

void rope_inplace_dyn(half* q, half* k, int n_heads, int n_kv_heads, int head_dim, const int* d_pos,
                      float theta_base, bool neox, hipStream_t stream) {
    report(jllm_hip_rope_inplace_dyn(H(q), H(k), n_heads, n_kv_heads, head_dim, d_pos, theta_base, neox ? 1 : 0,
                                     stream),
           "rope_inplace_dyn", nullptr, 0, stream);
}

void fused_geglu(half* output, const half* gate, const half* up, int rows, int intermediate_dim, hipStream_t stream) {
    report(jllm_hip_fused_geglu(H(output), H(gate), H(up), rows, intermediate_dim, stream), "fused_geglu", output,
           fill_bytes({rows, intermediate_dim}, 2), stream);
}

void vec_scale(half* x, int n, float s, hipStream_t stream) {
    report(jllm_hip_vec_scale(H(x), n, s, stream), "vec_scale", nullptr, 0, stream);
}

void logit_softcap(float* x, int n, float cap, hipStream_t stream) {
    report(jllm_hip_logit_softcap(x, n, cap, stream), "logit_softcap", nullptr, 0, stream);
}

void gemv_dense(half* out, const void* W, int wtype, const half* x, int M, int K, hipStream_t stream) {
    report(jllm_hip_gemv_dense(H(out), W, wtype, H(x), M, K, stream), "gemv_dense", out,
           fill_bytes({M}, 2), stream);
}

void gemm_dense_batched(half* out, const void* W, int wtype, const half* x, int M, int N, int K, hipStream_t stream) {
    report(jllm_hip_gemm_dense_batched(H(out), W, wtype, H(x), M, N, K, stream), "gemm_dense_batched", out,
           fill_bytes({M, N}, 2), stream);
}

void flash_attention_prefill_batched(half* output, const half* q, const void* k_cache, const void* v_cache,
                                     int n_heads, int n_kv_heads, int head_dim, int cache_head_dim, int N,
                                     int start_pos, float scale, bool kv_int8, const float* k_scales,
                                     const float* v_scales, int window, hipStream_t stream) {
    report(jllm_hip_flash_attention_prefill_batched(H(output), H(q), k_cache, v_cache, n_heads, n_kv_heads, head_dim,
                                                    cache_head_dim, N, start_pos, scale, kv_int8 ? 1 : 0, k_scales,
                                                    v_scales, window, stream),
           "flash_attention_prefill_batched", output,
           fill_bytes({N, n_heads, head_dim}, 2), stream);
}

}  // namespace jllm
