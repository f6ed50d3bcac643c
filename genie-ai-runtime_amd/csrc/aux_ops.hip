// aux_ops.hip -- the remaining kernels the engine calls through
// include/jllm_kernels.h outside the Llama/Qwen decode path: the Gemma
// family's GeGLU, in-place scale, final-logit soft-cap and dense (F32 / F16 /
// BF16) projections, and the standalone logits softmax.  None of them is on
// the quantized-matmul hot path; they exist so the engine links against this
// library with the reference's kernel translation units removed.
//
// Arithmetic, operation by operation in fp32 with fp16 rounding at the same
// points as the reference:
//   GeGLU     geglu_kernel           convert.cu:121-151
//   vec_scale vec_scale_kernel       convert.cu:155-170
//   soft-cap  logit_softcap_kernel   convert.cu:173-181
//   softmax   softmax_kernel         softmax.cu:15-81
//   dense     gemv_dense_kernel / gemm_dense_batched_kernel gemv_q4.cu:2815-2885
#include <float.h>
#include <math.h>
#include "kq_common.h"
#include "aux_ops.h"

namespace jllm_hip {

typedef uint32_t u32x4x __attribute__((ext_vector_type(4)));
typedef float f32x4x __attribute__((ext_vector_type(4)));

// gelu_tanh(g) * u, gelu_tanh(g) = 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3)))
__device__ __forceinline__ float geglu_val(float g, float u) {
#pragma clang fp contract(off)
    const float k = 0.7978845608028654f;
    return 0.5f * g * (1.0f + tanhf(k * (g + 0.044715f * g * g * g))) * u;
}

__global__ __launch_bounds__(256) void geglu_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ gate,
                                                    const uint16_t* __restrict__ up, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = f32_to_f16_bits(geglu_val(f16_bits_to_f32(gate[i]), f16_bits_to_f32(up[i])));
}

// x *= s.  The reference multiplies element pairs in fp16 by half(s) (one
// rounding of the exact product) and a trailing odd element in fp32 by s.
__global__ __launch_bounds__(256) void vec_scale_kernel(uint16_t* __restrict__ x, int64_t n, float s) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const bool paired = i < (n & ~(int64_t)1);
    const float f = paired ? round_to_f16(s) : s;
    x[i] = f32_to_f16_bits(f16_bits_to_f32(x[i]) * f);
}

__global__ __launch_bounds__(256) void softcap_kernel(float* __restrict__ x, int64_t n, float cap) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = cap * tanhf(x[i] / cap);
}

// One workgroup of 1024 threads: max, then e = exp(x - max) stored in place
// with the sum, then x *= 1/sum (the reference's three passes).
constexpr int SM_THREADS = 1024;
__device__ __forceinline__ float wsum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wmax(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__global__ __launch_bounds__(SM_THREADS) void softmax_kernel(float* __restrict__ x, int n) {
    __shared__ float red[SM_THREADS / 64];
    const int t = threadIdx.x, w = t >> 6;
    float m = -FLT_MAX;
    for (int i = t; i < n; i += SM_THREADS) m = fmaxf(m, x[i]);
    m = wmax(m);
    if ((t & 63) == 0) red[w] = m;
    __syncthreads();
    m = red[0];
    for (int i = 1; i < SM_THREADS / 64; i++) m = fmaxf(m, red[i]);
    __syncthreads();
    float s = 0.0f;
    for (int i = t; i < n; i += SM_THREADS) {
        const float e = expf(x[i] - m);
        x[i] = e;
        s += e;
    }
    s = wsum(s);
    if ((t & 63) == 0) red[w] = s;
    __syncthreads();
    s = 0.0f;
    for (int i = 0; i < SM_THREADS / 64; i++) s += red[i];
    const float inv = 1.0f / s;
    for (int i = t; i < n; i += SM_THREADS) x[i] *= inv;
}

// Dense projection out[t][m] = half(sum_k W[m][k] x[t][k]), W row-major
// [M][K] of F32 (wtype 0), F16 (1) or BF16 (30).  One wave per (row, token):
// each lane takes 8 consecutive weights per step (16- or 32-byte loads when
// the row is 16-byte aligned, element loads otherwise), fp32 accumulation,
// one wave reduction.
template <int WT>
__device__ __forceinline__ float dense_w(const void* W, int64_t i) {
    if (WT == 0) return ((const float*)W)[i];
    const uint32_t h = ((const uint16_t*)W)[i];
    if (WT == 1) return f16_bits_to_f32(h);
    return __builtin_bit_cast(float, h << 16);
}
template <int WT>
__device__ __forceinline__ void dense_w8(const void* W, int64_t i, float (&w)[8]) {
    if (WT == 0) {
        const f32x4x a = *(const f32x4x*)((const float*)W + i), b = *(const f32x4x*)((const float*)W + i + 4);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
        const u32x4x a = *(const u32x4x*)((const uint16_t*)W + i);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (WT == 1) {
                const half2_t h = as_h2(a[e]);
                w[2 * e] = (float)h[0];
                w[2 * e + 1] = (float)h[1];
            } else {
                w[2 * e] = __builtin_bit_cast(float, a[e] << 16);
                w[2 * e + 1] = __builtin_bit_cast(float, a[e] & 0xFFFF0000u);
            }
        }
    }
}

template <int WT, bool VEC>
__global__ __launch_bounds__(256) void dense_kernel(uint16_t* __restrict__ out, const void* __restrict__ W,
                                                    const uint16_t* __restrict__ x, int M, int K) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), tok = blockIdx.y, l = threadIdx.x & 63;
    if (row >= M) return;                                      // whole wave exits together
    const int64_t wb = (int64_t)row * K;
    const uint16_t* xt = x + (int64_t)tok * K;
    float acc = 0.0f;
    int k0 = 0;
    if (VEC) {
        const int kv = K & ~511;                               // 64 lanes x 8
        for (int k = 8 * l; k < kv; k += 512) {
            float w[8];
            dense_w8<WT>(W, wb + k, w);
            const u32x4x xv = *(const u32x4x*)(xt + k);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const half2_t h = as_h2(xv[e]);
                acc += w[2 * e] * (float)h[0];
                acc += w[2 * e + 1] * (float)h[1];
            }
        }
        k0 = kv;
    }
    for (int k = k0 + l; k < K; k += 64) acc += dense_w<WT>(W, wb + k) * f16_bits_to_f32(xt[k]);
    acc = wsum(acc);
    if (l == 0) out[(int64_t)tok * M + row] = f32_to_f16_bits(acc);
}

hipError_t geglu_launch(uint16_t* out, const uint16_t* gate, const uint16_t* up, int64_t n, hipStream_t st) {
    hipLaunchKernelGGL(geglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, gate, up, n);
    return hipGetLastError();
}

hipError_t vec_scale_launch(uint16_t* x, int64_t n, float s, hipStream_t st) {
    hipLaunchKernelGGL(vec_scale_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n, s);
    return hipGetLastError();
}

hipError_t softcap_launch(float* x, int64_t n, float cap, hipStream_t st) {
    hipLaunchKernelGGL(softcap_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n, cap);
    return hipGetLastError();
}

hipError_t softmax_launch(float* x, int n, hipStream_t st) {
    hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(SM_THREADS), 0, st, x, n);
    return hipGetLastError();
}

hipError_t dense_launch(uint16_t* out, const void* W, int wtype, const uint16_t* x, int M, int N, int K,
                        hipStream_t st) {
    const int eb = wtype == 0 ? 4 : 2;
    const bool vec = ((uintptr_t)W % 16) == 0 && ((int64_t)K * eb) % 16 == 0 && ((uintptr_t)x % 16) == 0 && K % 8 == 0;
    const dim3 g((unsigned)((M + 3) / 4), (unsigned)N);
#define DENSE_CASE(WT)                                                                              \
    if (vec) hipLaunchKernelGGL((dense_kernel<WT, true>), g, dim3(256), 0, st, out, W, x, M, K);   \
    else     hipLaunchKernelGGL((dense_kernel<WT, false>), g, dim3(256), 0, st, out, W, x, M, K);
    switch (wtype) {
    case 0: DENSE_CASE(0) break;
    case 1: DENSE_CASE(1) break;
    case 30: DENSE_CASE(30) break;
    default: return hipErrorInvalidValue;
    }
#undef DENSE_CASE
    return hipGetLastError();
}

}  // namespace jllm_hip
