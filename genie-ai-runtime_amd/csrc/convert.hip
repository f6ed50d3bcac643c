// convert.hip -- fp16 -> int8 per-row KV quantiser (fp16_to_int8_kernel,
// convert.cu:26-69): scale = absmax/127, q = rn(v * (127/absmax)) clamped to
// +-127, inv = 0 for an all-zero row.  One workgroup per row; the absmax is a
// wave-shuffle + LDS reduction (max is exact, so the result is order-free).
#include "kq_common.h"
#include "convert.h"

namespace jllm_hip {

__global__ __launch_bounds__(256) void fp16_to_int8_kernel(int8_t* __restrict__ dst, float* __restrict__ scale_out,
                                                           const uint16_t* __restrict__ src, int cols) {
    __shared__ float red[4];
    const int row = blockIdx.x, t = threadIdx.x;
    const int64_t off = (int64_t)row * cols;
    float mx = 0.0f;
    for (int c = t; c < cols; c += blockDim.x) mx = fmaxf(mx, fabsf(f16_bits_to_f32(src[off + c])));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float scale = mx / 127.0f;
    const float inv = scale > 0.0f ? 127.0f / mx : 0.0f;
    if (t == 0 && scale_out) scale_out[row] = scale;
    for (int c = t; c < cols; c += blockDim.x) {
        int q = (int)__builtin_rintf(f16_bits_to_f32(src[off + c]) * inv);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        dst[off + c] = (int8_t)q;
    }
}

hipError_t fp16_to_int8_launch(int8_t* dst, float* scale_out, const uint16_t* src, int rows, int cols, hipStream_t st) {
    hipLaunchKernelGGL(fp16_to_int8_kernel, dim3(rows), dim3(256), 0, st, dst, scale_out, src, cols);
    return hipGetLastError();
}

}  // namespace jllm_hip
