// capi_layer.hip -- C ABI of the decoder-layer kernels around the quantized
// matmuls (RMSNorm, SwiGLU, residual add, RoPE, fused q/k post-processing
// with KV store, embedding dequant, greedy argmax).
#include "capi_common.h"
#include "layer_ops.h"

using namespace jllm_hip;

namespace {
inline bool aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }
}  // namespace

extern "C" {

int jllm_hip_fused_rmsnorm_residual(uint16_t* out, const uint16_t* x, const uint16_t* residual, const void* weight,
                                    int rows, int hidden_dim, float eps, int weight_fp32, void* stream) {
    if (rows < 0 || hidden_dim <= 0 || hidden_dim % 2 != 0) return JLLM_ERR_INVALID;
    if (rows == 0) return JLLM_OK;
    if (!out || !x || !weight || !aligned4(out) || !aligned4(x) || (residual && !aligned4(residual)) ||
        ((uintptr_t)weight & (weight_fp32 ? 3u : 1u)))
        return JLLM_ERR_INVALID;
    return launch_status(rmsnorm_launch(out, x, residual, weight, rows, hidden_dim, eps, weight_fp32 != 0,
                                        (hipStream_t)stream), "rmsnorm");
}

int jllm_hip_fused_swiglu(uint16_t* out, const uint16_t* gate, const uint16_t* up, int rows, int intermediate_dim,
                          void* stream) {
    if (rows < 0 || intermediate_dim < 0) return JLLM_ERR_INVALID;
    const int64_t n = (int64_t)rows * intermediate_dim;
    if (n == 0) return JLLM_OK;
    if (!out || !gate || !up) return JLLM_ERR_INVALID;
    return launch_status(swiglu_launch(out, gate, up, n, (hipStream_t)stream), "swiglu");
}

int jllm_hip_vec_add(uint16_t* out, const uint16_t* a, const uint16_t* b, int64_t n, void* stream) {
    if (n < 0) return JLLM_ERR_INVALID;
    if (n == 0) return JLLM_OK;
    if (!out || !a || !b) return JLLM_ERR_INVALID;
    return launch_status(vec_add_launch(out, a, b, n, (hipStream_t)stream), "vec_add");
}

int jllm_hip_rope_precompute_table(int max_seq, int head_dim, float theta_base) {
    (void)theta_base;
    if (max_seq < 0 || head_dim <= 0 || head_dim % 2 != 0 || head_dim > 2 * ROPE_MAX_HALF) return JLLM_ERR_INVALID;
    return JLLM_OK;
}

void jllm_hip_rope_clear_tables(void) {}

int jllm_hip_rope_inplace_batched(uint16_t* q, uint16_t* k, int n_heads, int n_kv_heads, int head_dim, int start_pos,
                                  int N, int q_stride, int k_stride, float theta_base, int neox, void* stream) {
    if (n_heads < 0 || n_kv_heads < 0 || N < 0 || start_pos < 0) return JLLM_ERR_INVALID;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 2 * ROPE_MAX_HALF) {
        fprintf(stderr, "[rope] head_dim=%d: need an even head_dim <= %d\n", head_dim, 2 * ROPE_MAX_HALF);
        return JLLM_ERR_INVALID;
    }
    if (!k) n_kv_heads = 0;
    if (N == 0 || n_heads + n_kv_heads == 0) return JLLM_OK;
    if ((n_heads && !q) || q_stride < n_heads * head_dim || (n_kv_heads && k_stride < n_kv_heads * head_dim))
        return JLLM_ERR_INVALID;
    RopeFreq fr;
    rope_frequencies(fr, head_dim, theta_base);
    return launch_status(rope_launch(q, k, n_heads, n_kv_heads, head_dim, start_pos, N, q_stride, k_stride, fr,
                                     neox != 0, (hipStream_t)stream), "rope");
}

int jllm_hip_rope_inplace(uint16_t* q, uint16_t* k, int n_heads, int n_kv_heads, int head_dim, int position,
                          float theta_base, int neox, void* stream) {
    return jllm_hip_rope_inplace_batched(q, k, n_heads, n_kv_heads, head_dim, position, 1, n_heads * head_dim,
                                         n_kv_heads * head_dim, theta_base, neox, stream);
}

int jllm_hip_qk_norm_rope_store_kv(uint16_t* q, uint16_t* k, const uint16_t* v, const void* q_norm,
                                   const void* k_norm, int norm_fp32, float eps, void* k_dst, void* v_dst,
                                   float* k_scales, float* v_scales, int64_t kv_stride, int n_heads, int n_kv_heads,
                                   int head_dim, int cache_head_dim, int start_pos, int N, float theta_base, int neox,
                                   int kv_int8, void* stream) {
    if (n_heads <= 0 || n_kv_heads <= 0 || N < 0 || start_pos < 0 || cache_head_dim < head_dim ||
        kv_stride < (int64_t)n_kv_heads * cache_head_dim)
        return JLLM_ERR_INVALID;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 2 * ROPE_MAX_HALF) {
        fprintf(stderr, "[qk_post] head_dim=%d: need an even head_dim <= %d\n", head_dim, 2 * ROPE_MAX_HALF);
        return JLLM_ERR_INVALID;
    }
    if (N == 0) return JLLM_OK;
    // the engine norms q and k only when the layer has both weights (decode.cu:1443)
    if (!q || !k || !v || !k_dst || !v_dst || (q_norm == nullptr) != (k_norm == nullptr)) return JLLM_ERR_INVALID;
    QKPostArgs a;
    a.q = q; a.k = k; a.v = v; a.q_norm = q_norm; a.k_norm = k_norm;
    a.k_dst = k_dst; a.v_dst = v_dst; a.k_scales = k_scales; a.v_scales = v_scales; a.kv_stride = kv_stride;
    a.n_heads = n_heads; a.n_kv = n_kv_heads; a.head_dim = head_dim; a.cache_head_dim = cache_head_dim;
    a.start_pos = start_pos; a.N = N; a.eps = eps;
    a.norm_fp32 = norm_fp32 != 0; a.neox = neox != 0; a.kv_int8 = kv_int8 != 0;
    rope_frequencies(a.fr, head_dim, theta_base);
    return launch_status(qk_post_launch(a, (hipStream_t)stream), "qk_post");
}

int jllm_hip_rope_inplace_dyn(uint16_t* q, uint16_t* k, int n_heads, int n_kv_heads, int head_dim,
                              const int32_t* d_pos, float theta_base, int neox, void* stream) {
    if (n_heads < 0 || n_kv_heads < 0 || !d_pos) return JLLM_ERR_INVALID;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 2 * ROPE_MAX_HALF) {
        fprintf(stderr, "[rope] head_dim=%d: need an even head_dim <= %d\n", head_dim, 2 * ROPE_MAX_HALF);
        return JLLM_ERR_INVALID;
    }
    if (!k) n_kv_heads = 0;
    if (n_heads + n_kv_heads == 0) return JLLM_OK;
    if (n_heads && !q) return JLLM_ERR_INVALID;
    RopeFreq fr;
    rope_frequencies(fr, head_dim, theta_base);
    return launch_status(rope_launch(q, k, n_heads, n_kv_heads, head_dim, 0, 1, n_heads * head_dim,
                                     n_kv_heads * head_dim, fr, neox != 0, (hipStream_t)stream, d_pos), "rope");
}

namespace {
// RoPE of q and k plus an fp16 copy of k and v into the cache (no norms):
// the reference's rope_inplace_store_kv_fp16 family on the fused front
int rope_store_fp16(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_dst, uint16_t* v_dst,
                    int64_t cache_row_stride, int n_heads, int n_kv_heads, int head_dim, int cache_head_dim,
                    int start_pos, const int32_t* d_pos, int N, int64_t q_in_stride, int64_t kv_in_stride,
                    float theta_base, int neox, void* stream) {
    if (n_heads <= 0 || n_kv_heads <= 0 || N < 0 || start_pos < 0 || cache_head_dim < head_dim ||
        cache_row_stride < (int64_t)n_kv_heads * cache_head_dim || q_in_stride < (int64_t)n_heads * head_dim ||
        kv_in_stride < (int64_t)n_kv_heads * head_dim)
        return JLLM_ERR_INVALID;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 2 * ROPE_MAX_HALF) {
        fprintf(stderr, "[rope] head_dim=%d: need an even head_dim <= %d\n", head_dim, 2 * ROPE_MAX_HALF);
        return JLLM_ERR_INVALID;
    }
    if (N == 0) return JLLM_OK;
    if (!q || !k || !v || !k_dst || !v_dst) return JLLM_ERR_INVALID;
    QKPostArgs a;
    a.q = q; a.k = k; a.v = v; a.q_norm = nullptr; a.k_norm = nullptr;
    a.k_dst = k_dst; a.v_dst = v_dst; a.k_scales = nullptr; a.v_scales = nullptr; a.kv_stride = cache_row_stride;
    a.n_heads = n_heads; a.n_kv = n_kv_heads; a.head_dim = head_dim; a.cache_head_dim = cache_head_dim;
    a.start_pos = start_pos; a.N = N; a.eps = 0.0f;
    a.norm_fp32 = 0; a.neox = neox != 0; a.kv_int8 = 0;
    a.q_in_stride = q_in_stride; a.kv_in_stride = kv_in_stride; a.pos_dev = d_pos;
    rope_frequencies(a.fr, head_dim, theta_base);
    return launch_status(qk_post_launch(a, (hipStream_t)stream), "rope_store_kv");
}
}  // namespace

int jllm_hip_rope_inplace_store_kv_fp16_dyn(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_cache_layer_base,
                                            uint16_t* v_cache_layer_base, int n_heads, int n_kv_heads, int head_dim,
                                            int cache_head_dim, const int32_t* d_pos, float theta_base, int neox,
                                            void* stream) {
    if (!d_pos) return JLLM_ERR_INVALID;
    return rope_store_fp16(q, k, v, k_cache_layer_base, v_cache_layer_base, (int64_t)n_kv_heads * cache_head_dim,
                           n_heads, n_kv_heads, head_dim, cache_head_dim, 0, d_pos, 1, (int64_t)n_heads * head_dim,
                           (int64_t)n_kv_heads * head_dim, theta_base, neox, stream);
}

int jllm_hip_rope_inplace_store_kv_fp16_batched(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_cache_base,
                                                uint16_t* v_cache_base, int kv_slot, int n_heads, int n_kv_heads,
                                                int head_dim, int start_pos, int N, int q_stride, int kv_stride,
                                                float theta_base, int neox, void* stream) {
    return rope_store_fp16(q, k, v, k_cache_base, v_cache_base, kv_slot, n_heads, n_kv_heads, head_dim, head_dim,
                           start_pos, nullptr, N, q_stride, kv_stride, theta_base, neox, stream);
}

int jllm_hip_dequant_embedding_rows(uint16_t* dst, const void* W, int ggml_type, const int32_t* tokens, int N,
                                    int hidden_dim, int vocab, void* stream) {
    if (ggml_type < 12 || ggml_type > 14) return JLLM_ERR_UNSUPPORTED;
    if (N < 0 || vocab <= 0 || hidden_dim <= 0 || hidden_dim % 256 != 0) return JLLM_ERR_INVALID;
    if (N == 0) return JLLM_OK;
    if (!dst || !tokens || ((uintptr_t)dst & 15u)) return JLLM_ERR_INVALID;
    const void* Wd = resolve_weight(W);
    if (!Wd) return JLLM_ERR_POINTER;
    return launch_status(embed_launch(dst, Wd, ggml_type, tokens, 0, N, hidden_dim, vocab, (hipStream_t)stream), "embedding");
}

int jllm_hip_dequant_embedding_row(uint16_t* dst, const void* W, int ggml_type, int token_id, int hidden_dim,
                                   void* stream) {
    if (ggml_type != 12 && ggml_type != 14) return JLLM_ERR_UNSUPPORTED;
    if (token_id < 0 || hidden_dim <= 0 || hidden_dim % 256 != 0) return JLLM_ERR_INVALID;
    if (!dst || ((uintptr_t)dst & 15u)) return JLLM_ERR_INVALID;
    const void* Wd = resolve_weight(W);
    if (!Wd) return JLLM_ERR_POINTER;
    return launch_status(embed_launch(dst, Wd, ggml_type, nullptr, token_id, 1, hidden_dim, 0, (hipStream_t)stream),
                         "embedding");
}

int jllm_hip_argmax_f32(int32_t* out, const float* logits, int n, void* stream) {
    if (!out || !logits || n <= 0 || ((uintptr_t)logits & 3u)) return JLLM_ERR_INVALID;
    return launch_status(argmax_launch(out, logits, n, (hipStream_t)stream), "argmax");
}

}  // extern "C"
