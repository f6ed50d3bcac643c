// aux_ops.h -- internal interface of the kernels outside the Llama/Qwen
// decode path (Gemma GeGLU / scale / soft-cap / dense projections, logits
// softmax).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jllm_hip {

hipError_t geglu_launch(uint16_t* out, const uint16_t* gate, const uint16_t* up, int64_t n, hipStream_t st);
hipError_t vec_scale_launch(uint16_t* x, int64_t n, float s, hipStream_t st);
hipError_t softcap_launch(float* x, int64_t n, float cap, hipStream_t st);
hipError_t softmax_launch(float* x, int n, hipStream_t st);
// out [N][M] fp16 = x [N][K] . W^T, W dense [M][K]: wtype 0 F32, 1 F16, 30 BF16
hipError_t dense_launch(uint16_t* out, const void* W, int wtype, const uint16_t* x, int M, int N, int K,
                        hipStream_t st);

}  // namespace jllm_hip
