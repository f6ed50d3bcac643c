// capi_aux.hip -- C ABI of the kernels outside the Llama/Qwen decode path
// (Gemma GeGLU / scale / soft-cap / dense projections, logits softmax).
#include "capi_common.h"
#include "aux_ops.h"

using namespace jllm_hip;

extern "C" {

int jllm_hip_fused_geglu(uint16_t* out, const uint16_t* gate, const uint16_t* up, int rows, int intermediate_dim,
                         void* stream) {
    if (rows < 0 || intermediate_dim < 0) return JLLM_ERR_INVALID;
    const int64_t n = (int64_t)rows * intermediate_dim;
    if (n == 0) return JLLM_OK;
    if (!out || !gate || !up) return JLLM_ERR_INVALID;
    return launch_status(geglu_launch(out, gate, up, n, (hipStream_t)stream), "geglu");
}

int jllm_hip_vec_scale(uint16_t* x, int64_t n, float s, void* stream) {
    if (n < 0) return JLLM_ERR_INVALID;
    if (n == 0) return JLLM_OK;
    if (!x) return JLLM_ERR_INVALID;
    return launch_status(vec_scale_launch(x, n, s, (hipStream_t)stream), "vec_scale");
}

int jllm_hip_logit_softcap(float* x, int64_t n, float cap, void* stream) {
    if (n < 0 || !(cap > 0.0f)) return JLLM_ERR_INVALID;
    if (n == 0) return JLLM_OK;
    if (!x) return JLLM_ERR_INVALID;
    return launch_status(softcap_launch(x, n, cap, (hipStream_t)stream), "logit_softcap");
}

int jllm_hip_softmax_inplace(float* x, int n, void* stream) {
    if (n <= 0 || !x) return JLLM_ERR_INVALID;
    return launch_status(softmax_launch(x, n, (hipStream_t)stream), "softmax");
}

int jllm_hip_gemm_dense_batched(uint16_t* out, const void* W, int wtype, const uint16_t* x, int M, int N, int K,
                                void* stream) {
    if (wtype != 0 && wtype != 1 && wtype != 30) return JLLM_ERR_UNSUPPORTED;
    if (M < 0 || N < 0 || K <= 0 || N > 65535) return JLLM_ERR_INVALID;
    if (M == 0 || N == 0) return JLLM_OK;
    if (!out || !x || ((uintptr_t)x & 1u)) return JLLM_ERR_INVALID;
    const void* Wd = resolve_weight(W);
    if (!Wd) return JLLM_ERR_POINTER;
    if ((uintptr_t)Wd & (wtype == 0 ? 3u : 1u)) return JLLM_ERR_INVALID;
    return launch_status(dense_launch(out, Wd, wtype, x, M, N, K, (hipStream_t)stream), "dense");
}

int jllm_hip_gemv_dense(uint16_t* out, const void* W, int wtype, const uint16_t* x, int M, int K, void* stream) {
    return jllm_hip_gemm_dense_batched(out, W, wtype, x, M, 1, K, stream);
}

}  // extern "C"
