/*
 * jllm_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul hot path.
 *
 * Plain C: pointers, sizes and an int status.  fp16 buffers are passed as
 * uint16_t* holding IEEE binary16 bit patterns; `stream` is a hipStream_t
 * (NULL = the default stream).  Every entry point is asynchronous on the
 * given stream and returns JLLM_OK once its kernels are enqueued.
 *
 * Each declaration names the genie-ai-runtime interface it replaces
 * (include/jllm_kernels.h unless stated otherwise).  Unlike the reference,
 * nothing here falls back to a host computation: an unsupported type or a
 * pointer the GPU cannot read is reported as an error (and logged to stderr)
 * instead of being computed on the CPU.
 *
 * Requirements shared by the GEMV/GEMM entry points: ggml_type is 12 (Q4_K)
 * or 14 (Q6_K); K is a positive multiple of 256; W and x are 16-byte
 * aligned device (or registered mapped) pointers; K <= 28672.
 */
#ifndef JLLM_HIP_H
#define JLLM_HIP_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    JLLM_OK = 0,
    JLLM_ERR_INVALID = -1,      /* bad size, null or misaligned pointer */
    JLLM_ERR_UNSUPPORTED = -2,  /* ggml type other than Q4_K / Q6_K     */
    JLLM_ERR_LAUNCH = -3,       /* the HIP runtime rejected a launch    */
    JLLM_ERR_NOMEM = -4,        /* scratch allocation failed            */
    JLLM_ERR_POINTER = -5       /* weight pointer not visible to the GPU */
};

const char* jllm_hip_status_string(int status);

/* Mapped-weight registry.  Replaces register_mapped_weight_region,
 * clear_mapped_weight_region, resolve_mapped_weight_device_ptr
 * (jllm_kernels.h:40-43, defined in src/engine/model.cpp:39-66). */
int         jllm_hip_register_mapped_weight_region(const void* host_base, const void* device_base, int64_t bytes);
void        jllm_hip_clear_mapped_weight_region(const void* host_base);
const void* jllm_hip_resolve_mapped_weight_device_ptr(const void* host_ptr);

/* y[M] (fp16) = W[M x K] . x[K].  Q4_K and Q6_K use the int8 MMVQ path
 * (activation quantised to q8_1).  Replaces gemv_quant, jllm_kernels.h:64
 * (dispatch gemv_q4.cu:1245-1306). */
int jllm_hip_gemv_quant(uint16_t* y, const void* W, int ggml_type, const uint16_t* x,
                        int M, int K, void* stream);

/* y = half(half(W . x) + residual); float-dequant arithmetic.
 * Replaces gemv_quant_add, jllm_kernels.h:78 (gemv_q4.cu:1562-1616). */
int jllm_hip_gemv_quant_add(uint16_t* y, const void* W, int ggml_type, const uint16_t* x,
                            const uint16_t* residual, int M, int K, void* stream);

/* Two / three outputs sharing one activation.  MMVQ when both are Q4_K
 * (pair) or all are Q4_K/Q6_K (triple).  Replaces gemv_quant_pair :92 and
 * gemv_quant_triple :106 (gemv_q4.cu:1375-1560). */
int jllm_hip_gemv_quant_pair(uint16_t* y0, const void* W0, int ggml_type0, int M0,
                             uint16_t* y1, const void* W1, int ggml_type1, int M1,
                             const uint16_t* x, int K, void* stream);
int jllm_hip_gemv_quant_triple(uint16_t* y0, const void* W0, int ggml_type0, int M0,
                               uint16_t* y1, const void* W1, int ggml_type1, int M1,
                               uint16_t* y2, const void* W2, int ggml_type2, int M2,
                               const uint16_t* x, int K, void* stream);

/* fp32 output.  Q4_K: MMVQ; Q6_K: float dequant.  Replaces gemv_quant_f32,
 * jllm_kernels.h:148 (gemv_q4.cu:1323-1369). */
int jllm_hip_gemv_quant_f32(float* y, const void* W, int ggml_type, const uint16_t* x,
                            int M, int K, void* stream);

/* fp32 output, float-dequant arithmetic for both types: the GPU form of the
 * host scalar path gemv_quant_cpu (gemv_q4.cu:2519-2631).  No reference
 * counterpart on the GPU; for callers that want the dequant arithmetic. */
int jllm_hip_gemv_quant_dequant_f32(float* y, const void* W, int ggml_type, const uint16_t* x,
                                    int M, int K, void* stream);

/* q8_1 quantiser in the reference block layout {u16 d, u16 s, i8 qs[32]}
 * (36 B per 32 values).  Replaces quantize_q8_1, gemv_q4.cu:468. */
int jllm_hip_quantize_q8_1(const uint16_t* x, void* y, int K, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* JLLM_HIP_H */
