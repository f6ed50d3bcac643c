// The engine side of the drop-in boundary, for the GPU tests: each ec_*
// function makes ONE call of a namespace jllm C++ entry point
// (include/jllm_kernels.h) with the argument types the engine uses (half*,
// hipStream_t, bool), so a test exercises the C++ layer itself -- including
// its error path, which reports on stderr and zero-fills the output.  Built
// into tests/cxx/libengine_calls.so (linked against libjllm_hip.so only,
// plus model_registry_stub.cpp standing in for the engine's model.cpp) by
// __graft_entry__.build(); test infrastructure, not part of the library.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>
#include "jllm_kernels.h"

#define HP(p) reinterpret_cast<half*>(p)
#define CHP(p) reinterpret_cast<const half*>(p)
#define ST(s) reinterpret_cast<hipStream_t>(s)

extern "C" {

void ec_gemv_quant(void* y, const void* W, int t, const void* x, int M, int K, void* s) {
    jllm::gemv_quant(HP(y), W, t, CHP(x), M, K, ST(s));
}
void ec_gemv_quant_add(void* y, const void* W, int t, const void* x, const void* r, int M, int K, void* s) {
    jllm::gemv_quant_add(HP(y), W, t, CHP(x), CHP(r), M, K, ST(s));
}
void ec_gemv_quant_pair(void* y0, const void* W0, int t0, int M0, void* y1, const void* W1, int t1, int M1,
                        const void* x, int K, void* s) {
    jllm::gemv_quant_pair(HP(y0), W0, t0, M0, HP(y1), W1, t1, M1, CHP(x), K, ST(s));
}
void ec_gemv_quant_triple(void* y0, const void* W0, int t0, int M0, void* y1, const void* W1, int t1, int M1,
                          void* y2, const void* W2, int t2, int M2, const void* x, int K, void* s) {
    jllm::gemv_quant_triple(HP(y0), W0, t0, M0, HP(y1), W1, t1, M1, HP(y2), W2, t2, M2, CHP(x), K, ST(s));
}
void ec_gemv_quant_f32(float* y, const void* W, int t, const void* x, int M, int K, void* s) {
    jllm::gemv_quant_f32(y, W, t, CHP(x), M, K, ST(s));
}
void ec_gemm_quant_batched(void* y, const void* W, int t, const void* x, int M, int N, int K, void* s) {
    jllm::gemm_quant_batched(HP(y), W, t, CHP(x), M, N, K, ST(s));
}
void ec_flash_attention_decode(void* out, const void* q, const void* k, const void* v, int H, int KV, int hd,
                               int chd, int seq, float scale, int i8, const float* ks, const float* vs, int window,
                               void* s) {
    jllm::flash_attention_decode(HP(out), CHP(q), k, v, H, KV, hd, chd, seq, scale, i8 != 0, ks, vs, window, ST(s));
}
// the reference signature (one kv_scales pointer)
void ec_flash_attention_decode_dyn1(void* out, const void* q, const void* k, const void* v, int H, int KV, int hd,
                                    int chd, const int* d_pos, float scale, int i8, const float* kvs, int window,
                                    int n_splits, void* s) {
    jllm::flash_attention_decode_dyn(HP(out), CHP(q), k, v, H, KV, hd, chd, d_pos, scale, i8 != 0, kvs, window,
                                     n_splits, ST(s));
}
void ec_flash_attention_decode_dyn2(void* out, const void* q, const void* k, const void* v, int H, int KV, int hd,
                                    int chd, const int* d_pos, float scale, int i8, const float* ks, const float* vs,
                                    int window, int n_splits, void* s) {
    jllm::flash_attention_decode_dyn(HP(out), CHP(q), k, v, H, KV, hd, chd, d_pos, scale, i8 != 0, ks, vs, window,
                                     n_splits, ST(s));
}
void ec_flash_attention_prefill_batched(void* out, const void* q, const void* k, const void* v, int H, int KV, int hd,
                                        int chd, int N, int start, float scale, int i8, const float* ks,
                                        const float* vs, int window, void* s) {
    jllm::flash_attention_prefill_batched(HP(out), CHP(q), k, v, H, KV, hd, chd, N, start, scale, i8 != 0, ks, vs,
                                          window, ST(s));
}
void ec_quantize_q8_1(const void* x, void* y, int K, void* s) { jllm::quantize_q8_1(CHP(x), y, K, ST(s)); }
int ec_decode_attn_splits(int seq) { return jllm::decode_attn_splits(seq); }
float* ec_get_splitk_partials(int H, int S, int hd) { return jllm::get_splitk_partials(H, S, hd); }
void ec_fp16_to_int8(int8_t* dst, float* sc, const void* src, int rows, int cols, void* s) {
    jllm::fp16_to_int8(dst, sc, CHP(src), rows, cols, ST(s));
}
void ec_fused_rmsnorm_residual(void* out, const void* x, const void* r, const void* w, int rows, int dim, float eps,
                               int wf32, void* s) {
    jllm::fused_rmsnorm_residual(HP(out), CHP(x), CHP(r), w, rows, dim, eps, wf32 != 0, ST(s));
}
void ec_fused_swiglu(void* out, const void* g, const void* u, int rows, int dim, void* s) {
    jllm::fused_swiglu(HP(out), CHP(g), CHP(u), rows, dim, ST(s));
}
void ec_fused_geglu(void* out, const void* g, const void* u, int rows, int dim, void* s) {
    jllm::fused_geglu(HP(out), CHP(g), CHP(u), rows, dim, ST(s));
}
void ec_vec_scale(void* x, int n, float f, void* s) { jllm::vec_scale(HP(x), n, f, ST(s)); }
void ec_logit_softcap(float* x, int n, float cap, void* s) { jllm::logit_softcap(x, n, cap, ST(s)); }
void ec_softmax_inplace(float* x, int n, void* s) { jllm::softmax_inplace(x, n, ST(s)); }
void ec_gemv_dense(void* out, const void* W, int wt, const void* x, int M, int K, void* s) {
    jllm::gemv_dense(HP(out), W, wt, CHP(x), M, K, ST(s));
}
void ec_gemm_dense_batched(void* out, const void* W, int wt, const void* x, int M, int N, int K, void* s) {
    jllm::gemm_dense_batched(HP(out), W, wt, CHP(x), M, N, K, ST(s));
}
void ec_rope_inplace(void* q, void* k, int H, int KV, int hd, int pos, float theta, int neox, void* s) {
    jllm::rope_inplace(HP(q), HP(k), H, KV, hd, pos, theta, neox != 0, ST(s));
}
void ec_rope_inplace_dyn(void* q, void* k, int H, int KV, int hd, const int* d_pos, float theta, int neox, void* s) {
    jllm::rope_inplace_dyn(HP(q), HP(k), H, KV, hd, d_pos, theta, neox != 0, ST(s));
}
void ec_rope_inplace_store_kv_fp16(void* q, void* k, const void* v, void* kd, void* vd, int H, int KV, int hd, int pos,
                                   float theta, int neox, void* s) {
    jllm::rope_inplace_store_kv_fp16(HP(q), HP(k), CHP(v), HP(kd), HP(vd), H, KV, hd, pos, theta, neox != 0, ST(s));
}
void ec_rope_inplace_store_kv_fp16_dyn(void* q, void* k, const void* v, void* kb, void* vb, int H, int KV, int hd,
                                       int chd, const int* d_pos, float theta, int neox, void* s) {
    jllm::rope_inplace_store_kv_fp16_dyn(HP(q), HP(k), CHP(v), HP(kb), HP(vb), H, KV, hd, chd, d_pos, theta,
                                         neox != 0, ST(s));
}
void ec_rope_inplace_store_kv_fp16_batched(void* q, void* k, const void* v, void* kb, void* vb, int kv_slot, int H,
                                           int KV, int hd, int start, int N, int q_stride, int kv_stride, float theta,
                                           int neox, void* s) {
    jllm::rope_inplace_store_kv_fp16_batched(HP(q), HP(k), CHP(v), HP(kb), HP(vb), kv_slot, H, KV, hd, start, N,
                                             q_stride, kv_stride, theta, neox != 0, ST(s));
}
int ec_dequant_embedding_row(void* dst, const void* W, int t, int tok, int hidden, void* s) {
    return jllm::dequant_embedding_row(HP(dst), W, t, tok, hidden, ST(s)) ? 1 : 0;
}
void ec_register_mapped_weight_region(const void* host, const void* dev, int64_t bytes) {
    jllm::register_mapped_weight_region(host, dev, bytes);
}
void ec_clear_mapped_weight_region(const void* host) { jllm::clear_mapped_weight_region(host); }

}  // extern "C"
