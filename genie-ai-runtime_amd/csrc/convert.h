// convert.h -- internal interface of the KV quantiser.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jllm_hip {
hipError_t fp16_to_int8_launch(int8_t* dst, float* scale_out, const uint16_t* src, int rows, int cols, hipStream_t st);
}
