// capi_common.h -- host-side helpers shared by the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <mutex>
#include "../../include/jllm_hip.h"

namespace jllm_hip {

// Resolve a weight pointer the GPU can read: a registered mapped region's
// device alias, else the pointer itself when HIP reports device or managed
// memory (resolve_weight_device_ptr, gemv_q4.cu:105-128).  nullptr if
// neither.
const void* resolve_weight(const void* W);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline int launch_status(hipError_t e, const char* tag) {
    if (e == hipSuccess) return JLLM_OK;
    fprintf(stderr, "[%s] launch failed: %s\n", tag, hipGetErrorString(e));
    return JLLM_ERR_LAUNCH;
}

// Per-device, lazily grown device scratch that is never freed (the
// reference's static scratch semantics, e.g. gemv_q4.cu:1309-1321).  A
// request larger than the current buffer allocates a new one (rounded up
// to a power of two, at least 1 MiB, zeroed once) and RETIRES the old one
// without freeing it: a HIP graph captured earlier keeps pointing at memory
// that stays valid (and is no longer handed out).  Growth is a hipMalloc,
// so it must not happen during stream capture: size the scratch with one
// eager call (e.g. get_splitk_partials) before capturing.
struct DeviceScratch {
    static constexpr int MAXDEV = 64;
    void* ptr[MAXDEV] = {};
    size_t cap[MAXDEV] = {};
    int retired[MAXDEV] = {};
    std::mutex mu;
    void* get(size_t bytes) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return nullptr;
        std::lock_guard<std::mutex> lk(mu);
        if (bytes > cap[dev]) {
            if (bytes > ((size_t)1 << 40)) {
                fprintf(stderr, "[scratch] request of %zu bytes refused (over 1 TiB: an invalid size)\n", bytes);
                return nullptr;
            }
            size_t want = (size_t)1 << 20;
            while (want < bytes) want <<= 1;
            void* p = nullptr;
            if (hipMalloc(&p, want) != hipSuccess) {
                (void)hipGetLastError();
                fprintf(stderr, "[scratch] hipMalloc of %zu bytes failed (inside a stream capture? size the "
                                "scratch with an eager call first)\n", want);
                return nullptr;
            }
            // zeroed once, synchronously, at allocation (never inside a
            // stream, so graph capture never records it)
            if (hipMemset(p, 0, want) != hipSuccess) { (void)hipFree(p); (void)hipGetLastError(); return nullptr; }
            if (ptr[dev]) retired[dev]++;      // the old buffer stays allocated for graphs that captured it
            ptr[dev] = p;
            cap[dev] = want;
        }
        return ptr[dev];
    }
};

// Several batched GEMMs of one activation x [N x K] (the decoder's Q/K/V and
// gate/up): the activation is quantised once per quantiser kind present
// (DS4 for Q4_K, D4 for Q6_K; Q5_K needs none), then each product runs as
// jllm_hip_gemm_quant_batched would (fp16 out).  Types and shapes are
// checked as there.
// quantized: the activation's codes are already in the quantiser scratch
// (norm_rows reported so for this x, N, K and these outputs).
struct GemmOut { uint16_t* y; const void* W; int type; int M; };
int gemm_batched_shared_x(const char* tag, const GemmOut* outs, int n, const uint16_t* x, int N, int K, void* stream,
                          bool quantized = false);
// The decoder's prefill Q/K/V of one activation x (normed, quantised
// already when `quantized`) with the attention front fa (q/k RMSNorm, RoPE,
// KV-cache store) in the GEMM's epilogue, when the shapes allow it (all
// three Q4_K, head_dim 128, a grid that needs no split-K): *done = true and
// every output as gemm_batched_shared_x followed by
// jllm_hip_qk_norm_rope_store_kv would leave it; else *done = false and
// nothing ran.
// The prefill attention (jllm_hip_flash_attention_prefill_batched) whose
// epilogue also quantises the output rows for the next GEMM when quant is
// given and the kernel form allows it (*quantized = true: codes[npad
// rows] as the MMQ activation quantiser writes them, int8 codes + DS4
// words when i8, else fp16 codes + D4 words).
struct AttnQuant { void* codes; uint32_t* scl; int npad; bool i8; };
int prefill_attention(uint16_t* out, const uint16_t* q, const void* k, const void* v, int n_heads, int n_kv_heads,
                      int head_dim, int cache_head_dim, int N, int start_pos, float scale, int kv_int8,
                      const float* k_scales, const float* v_scales, int window, const AttnQuant* quant, void* stream,
                      bool* quantized);
// the quantiser scratch of an N x K activation for weight type `type` (12
// or 14; the pointers gemm_batched_res / gemm_batched_shared_x read)
int q8_codes(const char* tag, int type, int N, int K, AttnQuant* q);
// The decoder's prefill gate/up of one activation x (quantised already when
// `quantized`) with the SwiGLU and its quantisation for the down GEMM of
// type down_type in the GEMM's epilogue, when the shapes allow it (both
// Q4_K, equal M, M % 64 == 0, no split-K): *done = true and *act holds the
// down GEMM's activation codes (pass it as gemm_batched_res's pre); else
// *done = false and nothing ran.
int gate_up_swiglu_prefill(const char* tag, const GemmOut* gu, const uint16_t* x, int N, int K, bool quantized,
                           int down_type, AttnQuant* act, bool* done, void* stream);
struct QKPostArgs;
int qkv_front_prefill(const char* tag, const GemmOut* qkv, const uint16_t* x, int N, int K, bool quantized,
                      const QKPostArgs& fa, void* stream, bool* done);
// Rows of the residual stream whose residual add is left to the next step
// (gemm_batched_res with `defer`): mode 0: y [N x M] is complete; 1: y holds
// the product, y = half(y + res) still to do; 2: the product is still S
// fp32 split-K partials ws [S][N][M], y = half(half(sum) + res) to do.
struct ResidualRows { uint16_t* y; const uint16_t* res; const float* ws; int S; int mode; };
// y [N x M] = half(half(a . W^T) + res) with a = x, or, when up is given,
// a = half(silu(x) * up) (the SwiGLU of gate x and up, formed inside the
// activation quantiser; act_tmp [N x K] holds it where a path needs it in
// memory): the engine's projection + residual add (decode.cu:1830-1884).
int gemm_batched_res(const char* tag, uint16_t* y, const void* W, int type, const uint16_t* x, const uint16_t* up,
                     uint16_t* act_tmp, const uint16_t* res, int M, int N, int K, void* stream,
                     ResidualRows* defer = nullptr, const AttnQuant* pre = nullptr);
// completes deferred rows (y [N x M] as gemm_batched_res without defer writes it)
int residual_finish(const char* tag, const ResidualRows& r, int N, int M, void* stream);
// The deferred rows completed, then normed [N x H] = RMSNorm(y) with weights
// w (jllm_hip_fused_rmsnorm_residual's bits), and, for N > 1, the activation
// codes of the kinds that outs needs, in one pass where the shapes allow
// (*quantized = true: call gemm_batched_shared_x with quantized = true; the
// fp16 rows are then written only when an output reads them, i.e. Q5_K).
int norm_rows(const char* tag, const ResidualRows& r, int N, int H, uint16_t* normed, const void* w, bool w_fp32,
              float eps, const GemmOut* outs, int n, bool* quantized, void* stream);

// The decoder's supported shapes (jllm_hip_decoder_create, jllm_hip_gguf_config):
// false, with the reason on stderr, for a configuration a later step would reject.
bool decoder_config_ok(const jllm_hip_decoder_config& c);

}  // namespace jllm_hip
