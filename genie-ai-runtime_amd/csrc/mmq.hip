// mmq.hip -- prefill GEMM (MMQ) for Q4_K / Q6_K weights on gfx950.
//
// y[t][r] = sum_k x[t][k] * W[r][k] for N tokens, M weight rows, with the
// activation quantised to q8_1 in 32-value blocks (the reference's DS4 / D4
// quantisers, bit-exact) and every 32-weight (Q4_K) / 16-weight (Q6_K)
// group dotted EXACTLY, then scaled in fp32 -- the arithmetic of the
// reference's default prefill path (mmq_q4k_llama.cu:92-453,
// mmq_q6k_llama.cu:71-483):
//   Q4_K: sum += half(d*sc_j) * d8_j * C_j ;  sum += half(-dmin*m_j) * sumx_j
//   Q6_K: per 128-half, tmp += float(C_g0*sc_g0 + C_g1*sc_g1) * d8 (per 32),
//         sum += tmp * d.
//
// Matrix-core mapping.  The reference scales every 32-wide int32 dot in
// fp32, and on gfx950 one fp32 VALU op costs as much as ~64 int8 MACs on the
// matrix cores, so both kernels are bound by that epilogue, not by the
// matrix cores.
//   Q4_K: each 32-wide dot is one v_mfma_i32_32x32x32_i8 per 32 x 32 tile
//         (exact int32, K = 32 = one sub-block); the scale products
//         half(d*sc_j)*d8_j (exact: two fp16 values) come from a
//         v_mfma_f32_32x32x8_f16 outer product, so each element costs one
//         cvt and one fma per sub-block; the min term
//         sum_j half(-dmin*m_j)*sumx_j is one K = 8 f16 MFMA per half
//         super-block.  Activation codes are int8.
//   Q6_K: (q-32)*sc (|.| <= 1024) and the activation codes (-127..127) are
//         exact in fp16, their products exact in fp32, every partial sum
//         below 2^24, so v_mfma_f32_32x32x16_f16 gives C_g0*sc_g0 +
//         C_g1*sc_g1 exactly; the per-token d8 is a lane constant.
//         Activation codes are written by the quantiser as fp16 values, and
//         the weights are converted in the kernel (byte -> fp16 with
//         v_perm_b32 and one packed-fp16 fma).
//
// Tiles: Q4_K 128 rows x 64 tokens (4 waves of 32 x 64), Q6_K 128 x 128
// (4 waves of 32 x 128).  The K loop runs over half super-blocks; each
// lane's weight bytes go straight into registers one stage ahead, the
// activation codes shared by the workgroup go from global memory straight
// to LDS (buffer_load ... lds).  Tiles are handed out so that each XCD
// (blockIdx % 8) works on a contiguous range of row tiles.
#include "kq_common.h"
#include "mmq.h"
#include "qk_front.h"
#include "quant_chunk.h"
#include <algorithm>
#include <stdlib.h>

namespace jllm_hip {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4m __attribute__((ext_vector_type(4)));
typedef float f32x4m __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2m __attribute__((ext_vector_type(2)));
typedef _Float16 h8m __attribute__((ext_vector_type(8)));
typedef _Float16 h4m __attribute__((ext_vector_type(4)));
typedef float f32x16m __attribute__((ext_vector_type(16)));

constexpr int MMQ_THREADS = 256;
constexpr int TM = 128;                 // rows per workgroup tile (4 waves x 32)
constexpr int TN = MMQ_TILE_N;          // tokens per workgroup tile (64)

// ---------------------------------------------------------------------------
// activation quantiser (quantize_mmq_q8_1_ds4 / _d4, mmq_q4k_llama.cu:383-404,
// mmq_q6k_llama.cu:424-438): per 32 values d = amax/127, q = rn(v*(1/d)) with
// no clamp; DS4 stores half(d), half(sum v) with the sum taken in the order
// of a 5-step xor butterfly; D4 stores float d.  One thread per value, 32
// lanes per block, so the shuffle butterfly reproduces that order exactly.
__global__ __launch_bounds__(256) void quantize_mmq_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q8,
                                                           int N, int K, int Npad, int ds4) {
    const int blk = blockIdx.x * 2 + (threadIdx.x >> 7);      // (kb, col) pair index
    const int nblk = (K / 128) * Npad;
    if (blk >= nblk) return;                                   // whole 128-thread halves exit together
    const int kb = blk / Npad, col = blk % Npad;
    const int t = threadIdx.x & 127, sub = t >> 5, lane = t & 31;
    const float v = col < N ? f16_bits_to_f32(x[(int64_t)col * K + kb * 128 + t]) : 0.0f;
    float amax = fabsf(v), sum = v;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        sum += __shfl_xor(sum, o, 64);
    }
    const float d = amax / 127.0f;
    const float dinv = d > 0.0f ? 1.0f / d : 0.0f;
    uint8_t* out = q8 + (int64_t)blk * 144;
    out[16 + sub * 32 + lane] = (uint8_t)(int8_t)(int)__builtin_rintf(v * dinv);
    if (lane == 0) {
        if (ds4) {
            *(uint32_t*)(out + 4 * sub) = (uint32_t)f32_to_f16_bits(d) | ((uint32_t)f32_to_f16_bits(sum) << 16);
        } else {
            *(float*)(out + 4 * sub) = d;
        }
    }
}

hipError_t quantize_mmq_launch(const uint16_t* x, void* q8, int N, int K, int Npad, bool ds4, hipStream_t st) {
    const int nblk = (K / 128) * Npad;
    hipLaunchKernelGGL(quantize_mmq_kernel, dim3((nblk + 1) / 2), dim3(256), 0, st, x, (uint8_t*)q8, N, K, Npad, ds4 ? 1 : 0);
    return hipGetLastError();
}

// The same quantisation (same codes, d and sum, same butterfly order) in the
// layout the MMQ kernels read: codes as fp16 values, [K/256][Npad][256], and
// one 32-bit scale word per 32 values, [K/32][Npad] (DS4: half d | half sum
// << 16; D4: float d).
// Four lanes per 32-value block, 8 values (one 16-byte load) per lane.  The
// block sum is added in the order of a 32-lane butterfly (xor 16, 8, 4, 2,
// 1 over the value index), the order of the reference-layout quantiser
// above: index bit 4 pairs lanes sub ^ 2, bit 3 lanes sub ^ 1, bits 2..0
// stay within the lane -- so d and the sum are the same floats.
// SW: the values are half(silu(gate) * up) of two fp16 inputs (x = gate,
// x2 = up), formed here exactly as the SwiGLU kernel rounds them.
// I8: the codes as int8 bytes [K/256][Npad][256] (the Q4_K kernel's layout)
// instead of fp16 values.
template <bool SW, bool I8>
__global__ __launch_bounds__(256) void quantize_mmq_f16_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ x2,
                                                               void* __restrict__ codes,
                                                               uint32_t* __restrict__ scl, int N, int K, int Npad,
                                                               int ds4) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;     // (col, kb32, sub), sub fastest
    const int kb = K / 32;
    const int64_t nthr = (int64_t)Npad * kb * 4;
    if (gid >= nthr) return;                                          // whole 4-lane groups exit together
    const int sub = (int)(gid & 3);
    const int64_t cb = gid >> 2;
    const int kb32 = (int)(cb % kb), col = (int)(cb / kb);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (col < N) {
        const int64_t off = (int64_t)col * K + kb32 * 32 + 8 * sub;
        const u32x4m u = *(const u32x4m*)(x + off);
        w[0] = u.x; w[1] = u.y; w[2] = u.z; w[3] = u.w;
        if (SW) {
            const u32x4m u2 = *(const u32x4m*)(x2 + off);
            const uint32_t w2[4] = {u2.x, u2.y, u2.z, u2.w};
#pragma unroll
            for (int e = 0; e < 4; e++)
                w[e] = (uint32_t)f32_to_f16_bits(silu_mul(f16_bits_to_f32(w[e] & 0xFFFFu), f16_bits_to_f32(w2[e] & 0xFFFFu))) |
                       ((uint32_t)f32_to_f16_bits(silu_mul(f16_bits_to_f32(w[e] >> 16), f16_bits_to_f32(w2[e] >> 16))) << 16);
        }
    }
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; e++) { v[2 * e] = f16_bits_to_f32(w[e] & 0xFFFFu); v[2 * e + 1] = f16_bits_to_f32(w[e] >> 16); }
    quant_chunk<I8>(v, sub, kb32, col, Npad, codes, scl, ds4 != 0);
}

// RMSNorm and the MMQ activation quantisation of a block of residual-stream
// rows in one pass, the residual add that produces the rows optionally in
// front (the decoder's prefill).  One GS-thread workgroup per token row
// (rows N .. Npad-1: padding, zero codes).  Per row:
//   MODE 0: v = y (read only);
//   MODE 1: y = half(y + res) (the residual add of vec_add);
//   MODE 2: y = half(half(sum_s ws[s]) + res) (splitk_reduce_kernel<2>, the
//           partials added in order s = 0, 1, ...);
// then normed = half(v * rrms * w) with the sum of squares taken in the
// order of rmsnorm_kernel<GS, 8> (thread t: chunks t, t + GS, ...; pairs;
// wave_sum; for GS = 256 the four wave sums as (0 + 1) + (2 + 3)), and the
// normed values quantised by quant_chunk for the kinds whose codes pointer
// is set -- so every output has the bits of the separate kernels.
template <bool WF32, int GS, int MODE>
__global__ __launch_bounds__(GS) void norm_quant_kernel(NormQuantArgs a) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    constexpr int MAXC = 2;                              // chunks per thread: dim <= 2 * GS * 8
    const int t = threadIdx.x, n = blockIdx.x, H = a.H;
    const bool live = n < a.N;
    const int64_t off = (int64_t)(live ? n : 0) * H;
    float v[MAXC][8];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        const int i = (t + GS * c) * 8;
#pragma unroll
        for (int e = 0; e < 8; e++) v[c][e] = 0.0f;
        if (!live || i >= H) continue;
        const u32x4m u = *(const u32x4m*)(a.y + off + i);
        uint32_t w[4] = {u.x, u.y, u.z, u.w};
        if (MODE == 1) {
            const u32x4m r = *(const u32x4m*)(a.res + off + i);
            const uint32_t rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int e = 0; e < 4; e++)
                w[e] = (uint32_t)f32_to_f16_bits(f16_bits_to_f32(w[e] & 0xFFFFu) + f16_bits_to_f32(rr[e] & 0xFFFFu)) |
                       ((uint32_t)f32_to_f16_bits(f16_bits_to_f32(w[e] >> 16) + f16_bits_to_f32(rr[e] >> 16)) << 16);
        } else if (MODE == 2) {
            const int64_t nm = (int64_t)a.N * H;
            f32x4m p0 = *(const f32x4m*)(a.ws + off + i), p1 = *(const f32x4m*)(a.ws + off + i + 4);
            for (int s = 1; s < a.S; s++) {
                const f32x4m q0 = *(const f32x4m*)(a.ws + (int64_t)s * nm + off + i);
                const f32x4m q1 = *(const f32x4m*)(a.ws + (int64_t)s * nm + off + i + 4);
                p0.x += q0.x; p0.y += q0.y; p0.z += q0.z; p0.w += q0.w;
                p1.x += q1.x; p1.y += q1.y; p1.z += q1.z; p1.w += q1.w;
            }
            const float ps[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
            const u32x4m r = *(const u32x4m*)(a.res + off + i);
            const uint32_t rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int e = 0; e < 4; e++)
                w[e] = (uint32_t)f32_to_f16_bits(round_to_f16(ps[2 * e]) + f16_bits_to_f32(rr[e] & 0xFFFFu)) |
                       ((uint32_t)f32_to_f16_bits(round_to_f16(ps[2 * e + 1]) + f16_bits_to_f32(rr[e] >> 16)) << 16);
        }
        if (MODE != 0) *(u32x4m*)(a.y + off + i) = u32x4m{w[0], w[1], w[2], w[3]};
#pragma unroll
        for (int e = 0; e < 4; e++) { v[c][2 * e] = f16_bits_to_f32(w[e] & 0xFFFFu); v[c][2 * e + 1] = f16_bits_to_f32(w[e] >> 16); }
#pragma unroll
        for (int e = 0; e < 8; e += 2) ss += v[c][e] * v[c][e] + v[c][e + 1] * v[c][e + 1];
    }
    ss = wave_sum(ss);
    if (GS == 256) {
        if ((t & 63) == 0) red[t >> 6] = ss;
        __syncthreads();
        ss = (red[0] + red[1]) + (red[2] + red[3]);
    }
    const float rrms = 1.0f / sqrtf(ss / (float)H + a.eps);
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        const int ci = t + GS * c, i = ci * 8;
        if (i >= H) continue;                            // whole 4-lane groups (H % 32 == 0)
        float q[8];
        if (live) {
            float wv[8];
            if (WF32) {
                const f32x4m w0 = *(const f32x4m*)((const float*)a.w + i), w1 = *(const f32x4m*)((const float*)a.w + i + 4);
                wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w; wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
            } else {
                const u32x4m hw = *(const u32x4m*)((const uint16_t*)a.w + i);
                const uint32_t h[4] = {hw.x, hw.y, hw.z, hw.w};
#pragma unroll
                for (int e = 0; e < 4; e++) { wv[2 * e] = f16_bits_to_f32(h[e] & 0xFFFFu); wv[2 * e + 1] = f16_bits_to_f32(h[e] >> 16); }
            }
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                o[e] = (uint32_t)f32_to_f16_bits(v[c][2 * e] * rrms * wv[2 * e]) |
                       ((uint32_t)f32_to_f16_bits(v[c][2 * e + 1] * rrms * wv[2 * e + 1]) << 16);
            if (a.normed) *(u32x4m*)(a.normed + off + i) = u32x4m{o[0], o[1], o[2], o[3]};
#pragma unroll
            for (int e = 0; e < 4; e++) { q[2 * e] = f16_bits_to_f32(o[e] & 0xFFFFu); q[2 * e + 1] = f16_bits_to_f32(o[e] >> 16); }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) q[e] = 0.0f;
        }
        if (a.c8) quant_chunk<true>(q, ci & 3, ci >> 2, n, a.Npad, a.c8, a.s8, true);
        if (a.c16) quant_chunk<false>(q, ci & 3, ci >> 2, n, a.Npad, a.c16, a.s16, false);
    }
}

template <bool WF32, int GS>
static void norm_quant_go(const NormQuantArgs& a, hipStream_t st) {
    const dim3 g((unsigned)a.Npad), b(GS);
    if (a.mode == 0) hipLaunchKernelGGL((norm_quant_kernel<WF32, GS, 0>), g, b, 0, st, a);
    else if (a.mode == 1) hipLaunchKernelGGL((norm_quant_kernel<WF32, GS, 1>), g, b, 0, st, a);
    else hipLaunchKernelGGL((norm_quant_kernel<WF32, GS, 2>), g, b, 0, st, a);
}

bool norm_quant_supported(const NormQuantArgs& a, bool w_fp32) {
    const uintptr_t al = (uintptr_t)a.y | (uintptr_t)a.normed | (uintptr_t)(a.res ? a.res : a.y) |
                         (uintptr_t)(a.ws ? a.ws : (const float*)a.y);
    return a.H > 0 && a.H % 32 == 0 && a.H <= 4096 && a.N >= 0 && a.Npad >= a.N && al % 16 == 0 &&
           (uintptr_t)a.w % (w_fp32 ? 32 : 16) == 0 && a.mode >= 0 && a.mode <= 2 &&
           (a.mode != 2 || a.S >= 1);
}

hipError_t norm_quant_launch(const NormQuantArgs& a, bool w_fp32, hipStream_t st) {
    if (!norm_quant_supported(a, w_fp32)) return hipErrorInvalidValue;
    if (a.Npad == 0) return hipSuccess;
    // the thread count per row of rmsnorm_kernel for this width
    if (w_fp32) { if (a.H > 1024) norm_quant_go<true, 256>(a, st); else norm_quant_go<true, 64>(a, st); }
    else        { if (a.H > 1024) norm_quant_go<false, 256>(a, st); else norm_quant_go<false, 64>(a, st); }
    return hipGetLastError();
}

hipError_t quantize_mmq_f16_launch(const uint16_t* x, void* codes, uint32_t* scl, int N, int K, int Npad,
                                   bool ds4, hipStream_t st, const uint16_t* up, bool i8) {
    const int64_t nthr = (int64_t)Npad * (K / 32) * 4;
    const dim3 g((unsigned)((nthr + 255) / 256));
    const int d4 = ds4 ? 1 : 0;
    if (i8) {
        if (up) hipLaunchKernelGGL((quantize_mmq_f16_kernel<true, true>), g, dim3(256), 0, st, x, up, codes, scl, N, K, Npad, d4);
        else    hipLaunchKernelGGL((quantize_mmq_f16_kernel<false, true>), g, dim3(256), 0, st, x, x, codes, scl, N, K, Npad, d4);
    } else {
        if (up) hipLaunchKernelGGL((quantize_mmq_f16_kernel<true, false>), g, dim3(256), 0, st, x, up, codes, scl, N, K, Npad, d4);
        else    hipLaunchKernelGGL((quantize_mmq_f16_kernel<false, false>), g, dim3(256), 0, st, x, x, codes, scl, N, K, Npad, d4);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// tile scheduling

__device__ __forceinline__ int xcd_tile(int bid, int tiles) {
    const int full = tiles - tiles % 8;
    if (bid >= full) return bid;
    return (bid % 8) * (full / 8) + bid / 8;
}


// ---------------------------------------------------------------------------
// weight code -> fp16 conversions.  v_perm_b32 interleaves each code byte
// with 0x64, giving the fp16 value 1024 + byte; one packed fp16 subtract
// removes the bias exactly.

__device__ __forceinline__ h8m bytes_to_h8(u32x2m w, float bias) {
    const uint32_t hi = 0x64646464u;
    u32x4m p;
    p.x = __builtin_amdgcn_perm(hi, w.x, 0x04010400u);
    p.y = __builtin_amdgcn_perm(hi, w.x, 0x04030402u);
    p.z = __builtin_amdgcn_perm(hi, w.y, 0x04010400u);
    p.w = __builtin_amdgcn_perm(hi, w.y, 0x04030402u);
    const _Float16 b = (_Float16)bias;
    return __builtin_bit_cast(h8m, p) - h8m{b, b, b, b, b, b, b, b};
}

// 8 Q6_K codes q (bytes 0..63) -> 8 fp16 values (q - 32) * sc, in one fused
// multiply-add of the biased halves 1024 + q: (1024 + q) sc - 1056 sc is
// formed exactly before its single rounding, and |(q - 32) sc| <= 1024 is
// exact in fp16
__device__ __forceinline__ h8m q6_to_h8_scaled(u32x2m w, _Float16 sc) {
    const uint32_t hi = 0x64646464u;
    u32x4m p;
    p.x = __builtin_amdgcn_perm(hi, w.x, 0x04010400u);
    p.y = __builtin_amdgcn_perm(hi, w.x, 0x04030402u);
    p.z = __builtin_amdgcn_perm(hi, w.y, 0x04010400u);
    p.w = __builtin_amdgcn_perm(hi, w.y, 0x04030402u);
    const _Float16 off = (_Float16)-1056.0f * sc;       // exact: 1056 * |sc| <= 33792 = 1056 * 2^5
    return __builtin_elementwise_fma(__builtin_bit_cast(h8m, p), h8m{sc, sc, sc, sc, sc, sc, sc, sc},
                                     h8m{off, off, off, off, off, off, off, off});
}


__device__ __forceinline__ f32x16m mfma16(h8m a, h8m b, f32x16m c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Q4_K on the int8 matrix cores.
//
// Per 32-wide sub-block j the dots C_j = sum q4 * q8 (q4 in 0..15, q8 in
// -127..127) are one v_mfma_i32_32x32x32_i8 per 32 x 32 (rows x tokens)
// tile -- exact int32, K = 32 is exactly one sub-block.  The epilogue the
// format forces, sum += half(d*sc_j) * d8_j * C_j, takes the scale product
// S = half(d*sc_j) * d8_j (two fp16 values, exact in fp32) from a
// v_mfma_f32_32x32x8_f16 outer product, so each output element costs the
// VALU one cvt and one fma per sub-block; the min term sum_j half(-dmin*m_j)
// * sumx_j of a half super-block is one more K = 8 f16 MFMA accumulating
// straight into the fp32 result.  (A register-only microbenchmark of this
// step, genie-ai-runtime_amd/microbench/mmq_ceiling.hip, bounds it at ~20 %
// of the int8 peak: the fp32 epilogue, not the matrix cores, is the limit.)
//
// Workgroup tile 128 rows x 64 tokens, 4 waves of 32 rows x 64 tokens (two
// 32 x 32 tiles sharing the weight operand).  The K loop runs over half
// super-blocks ("stages" of 128 weights).  A wave's weight bytes are its
// own: each lane loads its 2 x 16 code bytes of the next stage (and, once
// per super-block, its row's 16-byte header) straight into registers one
// stage ahead.  The activation codes and scale words, shared by the four
// waves, go from global memory straight to LDS (buffer_load ... lds) in a
// ring of four stages, a super-block ahead; the 16-byte pieces of a token are
// XOR-swizzled so the B-operand reads of a wave hit distinct banks.
constexpr int ST_B = TN * 128;              // activation codes of a stage: 64 tokens x 128 B
constexpr int ST_S = 4 * TN * 4;            // scale words: 4 sub-blocks x 64 tokens
constexpr int ST_BYTES = ST_B + ST_S;
constexpr int NRING = 4;

typedef __attribute__((address_space(3))) void lds_void;

// piece P (16 B) of token t's 128 code bytes sits at position P ^ swz_b(t),
// so that any 8 (and any 16) consecutive lanes of an operand read hit
// distinct 16-byte bank groups
__host__ __device__ __forceinline__ int swz_b(int tok) { return (tok ^ (tok >> 3)) & 7; }

// Codes of the next GEMM's activation written by a GEMM epilogue: int8
// codes + DS4 words (i8) or fp16 codes + D4 words, Npad token rows
struct MmqActOut {
    void* codes;
    uint32_t* scl;
    int i8;
};

// OUT: 0: fp16 y [N][M], 1: fp32 y [N][M], 2: int32 dots [N][M][K/32], 3:
// fp16 y of the Q/K/V multi-launch followed by the attention front (fa), 4:
// gate (W[0]) and up (W[1]) of equal M, tile rt = rows [64 rt, 64 rt + 64)
// of both (waves 0-1 gate, 2-3 up), the SwiGLU half(silu(gate) * up) of
// the fp16 products quantised into ao (the down GEMM's activation)
template <int OUT, int TT>
__device__ __forceinline__ void mmq_q4k_body(const MmqSegs& sg, const uint8_t* __restrict__ codes,
                                             const uint32_t* __restrict__ scl, int N, int K, int Npad, int sps,
                                             const QKPostArgs* fa, const MmqActOut* ao = nullptr) {
    // TT 32-token halves per tile (2: the 128 x 64 tile; 1: 128 x 32, twice
    // the workgroups for grids that would leave SIMDs idle)
    constexpr int TNv = 32 * TT, STB = TNv * 128, STBYTES = STB + 4 * TNv * 4;
    __shared__ __attribute__((aligned(16))) uint8_t smem[NRING * STBYTES];

    const int nb = K / QK_K, nst = 2 * nb;
    // split-K: this workgroup's stages [k0, k1) (whole super-blocks)
    const int k0 = 2 * (int)blockIdx.y * sps, k1 = min(nst, k0 + 2 * sps);
    const int n_rt = sg.rt0[3], n_tt = Npad / TNv;
    const int tile = xcd_tile(blockIdx.x, n_rt * n_tt);
    const int rt = tile / n_tt;
    const int wq = OUT == 4 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) : 0;
    const int sgi = OUT == 4 ? (wq >> 1) : (rt >= sg.rt0[1] ? (rt >= sg.rt0[2] ? 2 : 1) : 0);
    void* __restrict__ y = sg.y[sgi];
    const uint8_t* __restrict__ W = sg.W[sgi];
    const int M = sg.M[sgi];
    // OUT 4: wave w's rows are 64 rt + 32 (w & 1) + lane (of gate or up)
    const int row0 = OUT == 4 ? 64 * rt - 64 * (wq >> 1) : (rt - sg.rt0[sgi]) * TM, col0 = (tile % n_tt) * TNv;
    // w in a scalar register: the LDS addresses and row offsets derived from
    // it stay scalar (9728 x 2560 at N = 512 63.5 -> 58.4 us)
    const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63, li = l & 31, g = l >> 5;
    const int arow = 32 * w + li;                      // this lane's A-operand row

    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0,
                                                                         (int)((int64_t)M * nb * Q4K_BYTES), 0x00020000);
    const __amdgpu_buffer_rsrc_t rC = __builtin_amdgcn_make_buffer_rsrc((void*)codes, (short)0,
                                                                         (int)((int64_t)K * Npad), 0x00020000);
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc((void*)scl, (short)0,
                                                                         (int)((int64_t)(K / 32) * Npad * 4), 0x00020000);
    // this lane's row (rows past M re-read the last row): code bytes 16g..
    // of each 32-byte pair, and the 16-byte block header
    const int voRow = min(row0 + arow, M - 1) * nb * Q4K_BYTES;
    // DMA slots: slot q (16 B) of the codes region is written by lane q % 64 of
    // wave q / 64 (TT instructions per wave); the scale words go as 4-byte
    // slots, 64 per wave (TT = 1: waves 2, 3 repeat the words of waves 0, 1
    // -- the same values to the same LDS words -- so that every wave issues
    // the same loads)
    int voB[TT];
#pragma unroll
    for (int i = 0; i < TT; i++) {
        const int q = (TT * w + i) * 64 + l;
        const int tok = q >> 3, pos = q & 7;
        voB[i] = (col0 + tok) * 256 + 16 * (pos ^ swz_b(tok));
    }
    const int qw = (w * 64 + l) % (4 * TNv);
    const int voS = (qw / TNv * Npad + col0 + qw % TNv) * 4;   // word (jl, tok) of the stage

    auto issue_b = [&](int k) {                        // TT + 1 DMA instructions per wave
        uint8_t* st = smem + (k % NRING) * STBYTES;
        const int b = k >> 1, s = k & 1;
#pragma unroll
        for (int i = 0; i < TT; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rC, (lds_void*)(st + (TT * w + i) * 1024), 16, voB[i],
                                                     b * Npad * 256 + 128 * s, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rS, (lds_void*)(st + STB + (TT == 2 ? w : (w & 1)) * 256), 4, voS,
                                                 (b * 8 + 4 * s) * Npad * 4, 0, 0);
    };
    // this lane's weight code bytes of stage k: pair 0 and pair 1 (16 B each)
    auto load_a = [&](int k, u32x4m (&a)[2]) {
        const int b = k >> 1, s = k & 1;
#pragma unroll
        for (int pp = 0; pp < 2; pp++)
            a[pp] = __builtin_amdgcn_raw_buffer_load_b128(rW, voRow + 16 + 16 * g, b * Q4K_BYTES + 64 * s + 32 * pp, 0);
    };

    f32x16m acc[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) acc[tt] = f32x16m{};
    int b_c[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) b_c[tt] = g ^ swz_b(32 * tt + li);   // B-read position = 2 * jl ^ b_c

    // Scale operands of the current super-block: lane (row, g) holds
    // half(d*sc_j) and half(-dmin*m_j) of its row for the sub-blocks j = 4g ..
    // 4g+3 in the K slots of a K = 8 f16 MFMA operand.  The scale product of
    // sub-block j is the MFMA of that operand with d8_j of each token in slot
    // j (zeros elsewhere); the min term of a stage is one MFMA with the
    // stage's four sum x_j in their slots.
    h4m As = h4m{}, Am = h4m{};
    auto scales = [&](const u32x4m hdr) {
        // the 6-bit (sc, m) of sub-blocks 4g .. 4g+3, one per byte (get_scale_min_k4 layout)
        uint32_t SC, MM;
        if (g == 0) {
            SC = hdr.y & 0x3F3F3F3Fu;
            MM = hdr.z & 0x3F3F3F3Fu;
        } else {
            SC = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
            MM = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
        }
        // half(d*sc) and half(-dmin*m) as the reference rounds them, in packed
        // fp16: the bytes become the halves 1024 + v (a byte permute against
        // 0x64 bytes), minus 1024 is v exactly, and one fp16 multiply rounds
        // the exact product d*v once -- the same half as the fp32 product
        // (exact: 11 x 6 bits) converted to fp16
        const uint32_t hi = 0x64646464u;
        const h4m k1024 = h4m{(_Float16)1024.0f, (_Float16)1024.0f, (_Float16)1024.0f, (_Float16)1024.0f};
        const h4m scv = __builtin_bit_cast(h4m, u32x2m{__builtin_amdgcn_perm(hi, SC, 0x04010400u),
                                                        __builtin_amdgcn_perm(hi, SC, 0x04030402u)}) - k1024;
        const h4m mv = __builtin_bit_cast(h4m, u32x2m{__builtin_amdgcn_perm(hi, MM, 0x04010400u),
                                                       __builtin_amdgcn_perm(hi, MM, 0x04030402u)}) - k1024;
        const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu));
        const _Float16 mh = -__builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
        As = scv * h4m{dh, dh, dh, dh};
        Am = mv * h4m{mh, mh, mh, mh};
    };

    auto compute = [&](int k, const u32x4m (&a)[2]) {
        const uint8_t* st = smem + (k % NRING) * STBYTES;
        const int b = k >> 1, s = k & 1;
        const uint32_t* sS = (const uint32_t*)(st + STB);
        const bool mine = g == s;                      // this lane group's K slots belong to the stage
        uint32_t sw[TT][4];
        i32x4 Bv[TT];
        auto read_b = [&](int jl) {
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
                Bv[tt] = *(const i32x4*)(st + (32 * tt + li) * 128 + 16 * ((2 * jl) ^ b_c[tt]));
        };
        read_b(0);
#pragma unroll
        for (int jl = 0; jl < 4; jl++) {
            const int j = 4 * s + jl;
            const u32x4m araw = a[jl >> 1];            // low nibbles: sub-block 2p, high: 2p+1
            const i32x4 Ai = __builtin_bit_cast(i32x4, (jl & 1) ? ((araw >> 4u) & 0x0F0F0F0Fu) : (araw & 0x0F0F0F0Fu));
            i32x16 C[TT];
            f32x16m S[TT];
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                if (OUT != 2) {
                    sw[tt][jl] = sS[jl * TNv + 32 * tt + li];               // half d8 | half sum x << 16
                    // d8 in K slot jl of this lane group's four (the stage's), zeros elsewhere
                    const uint32_t dv = (jl & 1) ? (sw[tt][jl] << 16) : (sw[tt][jl] & 0xFFFFu);
                    u32x2m bs = u32x2m{0u, 0u};
                    if (jl < 2) bs.x = mine ? dv : 0u;
                    else        bs.y = mine ? dv : 0u;
                    S[tt] = __builtin_amdgcn_mfma_f32_32x32x8f16(As, __builtin_bit_cast(h4m, bs), f32x16m{}, 0, 0, 0);
                }
                C[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ai, Bv[tt], i32x16{}, 0, 0, 0);
            }
            // the epilogue at raised wave priority: the waves of a workgroup
            // leave the barrier together, and a wave whose MFMA results are
            // in finishes its VALU work before the others' issue slots take
            // it (same arithmetic; TTFT 8.86 -> 8.74 ms)
            __builtin_amdgcn_s_setprio(1);
            if (jl < 3) read_b(jl + 1);
            if (OUT == 2) {
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int r = row0 + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3);
                        const int col = col0 + 32 * tt + li;
                        if (r < M && col < N) ((int*)y)[((int64_t)col * M + r) * (K / 32) + b * 8 + j] = C[tt][v];
                    }
            } else {
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[tt][v] = __builtin_fmaf(S[tt][v], (float)C[tt][v], acc[tt][v]);
            }
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (OUT != 2) {
            // min term of the stage's four sub-blocks: sum_j half(-dmin*m_j) * sum x_j
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                u32x2m bm;
                bm.x = mine ? ((sw[tt][0] >> 16) | (sw[tt][1] & 0xFFFF0000u)) : 0u;
                bm.y = mine ? ((sw[tt][2] >> 16) | (sw[tt][3] & 0xFFFF0000u)) : 0u;
                acc[tt] = __builtin_amdgcn_mfma_f32_32x32x8f16(Am, __builtin_bit_cast(h4m, bm), acc[tt], 0, 0, 0);
            }
        }
    };

    // Stage pipeline (k0 is even, k1 - k0 is even; a stage is half a
    // super-block, slot k % 4 of the ring).  The loads of a wave complete in
    // issue order and a plain s_barrier (no memory fence: a fence would wait
    // for every load in flight) after the DMA has landed makes every wave's
    // copy visible; it also orders every wave's reads of the slots that the
    // next DMA overwrites.  Past the last stage the loads repeat the last
    // stage (in bounds; the same bytes into its own slot), so every
    // iteration has the same load count and the waits are unconditional.
    u32x4m a0[2], a1[2];
    u32x4m hdr = __builtin_amdgcn_raw_buffer_load_b128(rW, voRow, (k0 >> 1) * Q4K_BYTES, 0);
    load_a(k0, a0);
    issue_b(k0);
    issue_b(k0 + 1);
    __builtin_amdgcn_s_waitcnt(0x0F70);                // everything of stage k0 (and k0+1's DMA)
    __builtin_amdgcn_s_barrier();
    // One workgroup barrier per super-block: both halves of the next
    // super-block are DMA'd into the other two ring slots while this one is
    // computed (the A-operand registers are waited for by the compiler).
    // The barrier's wait vmcnt(3) leaves only the newest header and A loads
    // (issued after that DMA) in flight.  (One barrier per half super-block
    // with a ring of three slots: 1-2 % slower, same bits.)
#pragma unroll 1
    for (int k = k0; k < k1; k += 2) {
        const int kl = k1 - 1;
        if (OUT != 2) scales(hdr);
        load_a(k + 1, a1);
        __builtin_amdgcn_sched_barrier(0);
        issue_b(min(k + 2, kl));
        issue_b(min(k + 3, kl));
        __builtin_amdgcn_sched_barrier(0);
        compute(k, a0);
        hdr = __builtin_amdgcn_raw_buffer_load_b128(rW, voRow, (min(k + 2, kl) >> 1) * Q4K_BYTES, 0);
        load_a(min(k + 2, kl), a0);
        __builtin_amdgcn_sched_barrier(0);
        compute(k + 1, a1);
        __builtin_amdgcn_s_waitcnt(0x0F73);            // vmcnt(3): the DMA of k+2, k+3 has landed
        __builtin_amdgcn_s_barrier();
    }
    if (OUT == 2) return;
    if (OUT == 4) {
        // fp16 products to LDS [token][64 gate rows | 64 up rows] (rows
        // padded to 130 halves), then per (token, 8 consecutive rows) the
        // SwiGLU as the quantiser's SW form rounds it and quant_chunk (the 4
        // lanes of an aligned quad: one 32-row block)
        constexpr int FT_LD = 130;
        static_assert(TNv * FT_LD * 2 <= NRING * STBYTES, "SwiGLU tile exceeds the LDS ring");
        uint16_t* T = (uint16_t*)smem;
        __builtin_amdgcn_s_waitcnt(0);                 // the ring's last DMA has landed
        __syncthreads();
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int v = 0; v < 16; v++)
                T[(32 * tt + li) * FT_LD + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3)] = f32_to_f16_bits(acc[tt][v]);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TT; j++) {
            const int e = t + MMQ_THREADS * j, tl = e >> 3, c8 = e & 7, tok = col0 + tl;
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float gv = f16_bits_to_f32(T[tl * FT_LD + 8 * c8 + i]);
                const float uv = f16_bits_to_f32(T[tl * FT_LD + 64 + 8 * c8 + i]);
                v[i] = tok < N ? f16_bits_to_f32(f32_to_f16_bits(silu_mul(gv, uv))) : 0.0f;
            }
            const int kb32 = (64 * rt + 8 * c8) >> 5, sub = c8 & 3;
            if (ao->i8) quant_chunk<true>(v, sub, kb32, tok, Npad, ao->codes, ao->scl, true);
            else        quant_chunk<false>(v, sub, kb32, tok, Npad, ao->codes, ao->scl, false);
        }
        return;
    }
    if (OUT == 3) {
        // The tile is one head (128 rows) of q, k or v (segment 0 / 1 / 2)
        // for 64 tokens.  Its fp16 values (y as the plain launch stores it)
        // go to LDS, [token][row] with rows padded to FT_LD halves, then
        // each wave runs the attention front (qk_post_kernel's front_finish)
        // for 16 tokens: lane l holds the rotary pair (i0, i1); v is also
        // stored as y.
        constexpr int FT_LD = 130;
        static_assert(TNv * FT_LD * 2 <= NRING * STBYTES, "front tile exceeds the LDS ring");
        uint16_t* T = (uint16_t*)smem;
        __builtin_amdgcn_s_waitcnt(0);                 // the ring's last DMA has landed
        __syncthreads();
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int v = 0; v < 16; v++)
                T[(32 * tt + li) * FT_LD + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3)] = f32_to_f16_bits(acc[tt][v]);
        __syncthreads();
        const QKPostArgs& a = *fa;
        const int kind = sgi, head = rt - sg.rt0[sgi];
        const int64_t qs = (int64_t)a.n_heads * 128, ks = (int64_t)a.n_kv * 128;
        int i0, i1;
        front_idx(128, a.neox != 0, l, i0, i1);
        const void* norm = kind < 2 ? (kind == 0 ? a.q_norm : a.k_norm) : nullptr;
        float w0 = 0.0f, w1 = 0.0f;
        front_weights(norm, a.norm_fp32 != 0, true, i0, i1, w0, w1);
        const float fq = a.fr.f[l];
        for (int j = 0; j < TNv / 4; j++) {
            const int tl = (TNv / 4) * w + j, tok = col0 + tl;
            if (tok >= N) break;                       // uniform across the wave
            const float v0 = f16_bits_to_f32(T[tl * FT_LD + i0]), v1 = f16_bits_to_f32(T[tl * FT_LD + i1]);
            if (kind == 2) {
                uint16_t* yv = (uint16_t*)y + (int64_t)tok * M + row0;
                yv[i0] = T[tl * FT_LD + i0];
                yv[i1] = T[tl * FT_LD + i1];
            }
            front_finish(a, kind, head, tok, 0, a.start_pos + tok, l, true, i0, i1, v0, v1, w0, w1, fq, qs, ks);
        }
        return;
    }
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        const int tok = col0 + 32 * tt + li;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = row0 + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3);
            if (r < M && tok < N) {
                if (OUT == 1) ((float*)y)[(int64_t)blockIdx.y * N * M + (int64_t)tok * M + r] = acc[tt][v];
                else          ((uint16_t*)y)[(int64_t)tok * M + r] = f32_to_f16_bits(acc[tt][v]);
            }
        }
    }
}

template <int OUT, int TT>
__global__ __launch_bounds__(MMQ_THREADS, 3)
void mmq_q4k_kernel(MmqSegs sg, const uint8_t* __restrict__ codes, const uint32_t* __restrict__ scl, int N, int K,
                    int Npad, int sps) {
    mmq_q4k_body<OUT, TT>(sg, codes, scl, N, K, Npad, sps, nullptr);
}

template <int TT>
__global__ __launch_bounds__(MMQ_THREADS, 3)
void mmq_q4k_front_kernel(MmqSegs sg, const uint8_t* __restrict__ codes, const uint32_t* __restrict__ scl, int N,
                          int K, int Npad, QKPostArgs fa) {
    mmq_q4k_body<3, TT>(sg, codes, scl, N, K, Npad, K / QK_K, &fa);
}

template <int TT>
__global__ __launch_bounds__(MMQ_THREADS, 3)
void mmq_q4k_swiglu_kernel(MmqSegs sg, const uint8_t* __restrict__ codes, const uint32_t* __restrict__ scl, int N,
                           int K, int Npad, MmqActOut ao) {
    mmq_q4k_body<4, TT>(sg, codes, scl, N, K, Npad, K / QK_K, nullptr, &ao);
}

// 32-token halves per Q4_K workgroup tile for a launch of `waves` waves
// with 64-token tiles.  The 32-token tile keeps 97-101 VGPRs and 18 KB of
// LDS, so a CU holds 5 of its workgroups instead of 3; it decodes each
// weight operand for half the tokens.  Measured (us, 64-token / 32-token
// tiles, quantiser and split-K reduce included): Q/K/V multi-launch 6144 x
// 2560 at N = 512 (384 tiles) 54.8 / 48.0, with the attention front 51.6 /
// 43.7; 9728 x 2560 at N = 512 (608) 72.5 / 69.5, at N = 64 30.7 / 29.9;
// O 2560 x 4096 at N = 512 (160 tiles x 3 ranges) 47.9 / 46.7; gate/up +
// SwiGLU at N = 512 (1216 tiles) 89.1 / 100.3 -- the smaller tile wins
// below ~1024 workgroups.  The outputs are the same bits either way.
int q4k_tt(int64_t waves) {
#ifdef JLLM_MMQ_TT_DEBUG
    if (const char* e = getenv("JLLM_MMQ_TT")) return atoi(e) == 1 ? 1 : 2;
#endif
    return waves < 4 * 1024 ? 1 : 2;
}

// ---------------------------------------------------------------------------
// Q6_K on the f16 matrix cores, 128 x 128 workgroup tiles.
//
// (q - 32) * sc (|.| <= 1024) and the q8 codes (fp16 values -127..127) are
// exact in fp16 and every 32-wide sum stays below 2^24, so two
// v_mfma_f32_32x32x16_f16 give each 32-wide block's C_g0*sc_g0 + C_g1*sc_g1
// exactly; the reference's per-half accumulation tmp += C * d8 (per 32),
// sum += tmp * d (mmq_q6k_llama.cu:264-364) is then one fma per element per
// block plus one per half.  The weight decode (6-bit code, minus 32, times
// the group scale) costs the VALU about two operations per weight, so a
// workgroup of 4 waves covers 128 rows x 128 tokens: each wave 32 rows x
// 128 tokens (four 32x32 MFMA tiles), every decoded weight operand serving
// 128 tokens.  K order inside a 32-wide block: lane group g holds elements
// 16g..16g+15 (one 16-group, so one scale per lane and block, and 16
// contiguous ql / qh bytes per lane); the activation operand is read from
// LDS in the same order.  Per half super-block ("stage"): each lane loads
// its row's three 16-byte pieces (low / high ql, qh) into registers one
// stage ahead (aligned 20-byte windows realigned with funnel shifts: Q6_K
// blocks are 2-byte aligned), and the scales + d once per super-block; the
// 128 tokens' fp16 codes (32 KB) and d8 words go from global memory straight
// to LDS (buffer_load ... lds), one stage ahead in a ring of two, 16-byte
// pieces of a token XOR-swizzled so the operand reads are conflict-free.

constexpr int Q6_TN = 128;                   // tokens per workgroup tile
constexpr int Q6_ST_B = Q6_TN * 256;         // fp16 codes of a stage: 128 tokens x 128 values
constexpr int Q6_ST_S = 4 * Q6_TN * 4;       // d8 words: 4 blocks x 128 tokens
constexpr int Q6_ST_BYTES = Q6_ST_B + Q6_ST_S;

// piece P (16 B, 8 codes) of token t's 128 codes of a stage sits at position
// P ^ (t & 15): 16 consecutive tokens reading one piece hit 16 bank groups
__device__ __forceinline__ int swz6(int tok) { return tok & 15; }

// 16 bytes at byte offset `off` of a buffer, read as an aligned 20-byte
// window (the window may run past the end of the buffer: those bytes read
// as zero) and realigned
__device__ __forceinline__ u32x4m load16_2a(__amdgpu_buffer_rsrc_t r, int off) {
    const int al = off & ~3;
    const uint32_t sh = (uint32_t)(off & 3) * 8u;
    const u32x4m w = __builtin_amdgcn_raw_buffer_load_b128(r, al, 0, 0);
    const uint32_t w4 = __builtin_amdgcn_raw_buffer_load_b32(r, al + 16, 0, 0);
    return u32x4m{__builtin_amdgcn_alignbit(w.y, w.x, sh), __builtin_amdgcn_alignbit(w.z, w.y, sh),
                  __builtin_amdgcn_alignbit(w.w, w.z, sh), __builtin_amdgcn_alignbit(w4, w.w, sh)};
}

template <int OUT>   // 0: fp16 y, 1: fp32 y (split-K partials), 2: int32 group dots [N][M][K/16]
__global__ __launch_bounds__(MMQ_THREADS, 2)
void mmq_q6k_kernel(void* __restrict__ y, const uint8_t* __restrict__ W, const uint16_t* __restrict__ codes,
                    const uint32_t* __restrict__ scl, int M, int N, int K, int Npad, int sps) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * Q6_ST_BYTES];
    __shared__ __attribute__((aligned(16))) float sDA[TM];             // d of the wave's rows, current super-block

    const int nb = K / QK_K, nst = 2 * nb;
    const int k0 = 2 * (int)blockIdx.y * sps, k1 = min(nst, k0 + 2 * sps);
    const int n_rt = (M + TM - 1) / TM, n_tt = (Npad + Q6_TN - 1) / Q6_TN;
    const int tile = xcd_tile(blockIdx.x, n_rt * n_tt);
    const int row0 = (tile / n_tt) * TM, col0 = (tile % n_tt) * Q6_TN;
    // w is wave-uniform: read into a scalar register, so the DMA's scalar
    // offsets that use it need no per-lane (waterfall) loop
    // w in a scalar register: the LDS addresses and row offsets derived from
    // it stay scalar (9728 x 2560 at N = 512 63.5 -> 58.4 us)
    const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63, li = l & 31, g = l >> 5;
    const int arow = 32 * w + li;

    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0,
                                                                         (int)((int64_t)M * nb * Q6K_BYTES), 0x00020000);
    const __amdgpu_buffer_rsrc_t rC = __builtin_amdgcn_make_buffer_rsrc((void*)codes, (short)0,
                                                                         (int)((int64_t)K * Npad * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc((void*)scl, (short)0,
                                                                         (int)((int64_t)(K / 32) * Npad * 4), 0x00020000);
    const int voRow = min(row0 + arow, M - 1) * nb * Q6K_BYTES;     // this lane's row

    // DMA: instruction i (0..7) of wave w fills LDS bytes [(8w + i) KiB, +1 KiB)
    // of the codes region: tokens 4(8w + i) + l/16, position l % 16
    const int lh = l >> 4, pl = l & 15;
    int xq[4];
#pragma unroll
    for (int j = 0; j < 4; j++) xq[j] = 16 * (pl ^ (4 * j + lh));
    const int voB = (col0 + 32 * w + lh) * 512;                      // + 2048 i + xq[i & 3]
    auto issue_b = [&](int k) {
        uint8_t* st = smem + (k & 1) * Q6_ST_BYTES;
        const int b = k >> 1, h = k & 1;
#pragma unroll
        for (int i = 0; i < 8; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rC, (lds_void*)(st + (8 * w + i) * 1024), 16, voB + xq[i & 3],
                                                     b * Npad * 512 + 256 * h + 2048 * i, 0, 0);
        // d8 of block 4h + w for tokens 64i + l
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rS, (lds_void*)(st + Q6_ST_B + (2 * w + i) * 256), 4,
                                                     (col0 + 64 * i + l) * 4, (b * 8 + 4 * h + w) * Npad * 4, 0, 0);
    };
    // this lane's weight pieces of stage k: ql bytes [16g, +16) and [32 + 16g, +16)
    // of the half, qh bytes [16g, +16)
    auto load_a = [&](int k, u32x4m (&a)[3]) {
        const int b = k >> 1, h = k & 1;
        const int base = voRow + b * Q6K_BYTES;
        a[0] = load16_2a(rW, base + 64 * h + 16 * g);
        a[1] = load16_2a(rW, base + 64 * h + 32 + 16 * g);
        a[2] = load16_2a(rW, base + 128 + 32 * h + 16 * g);
    };
    // scales[16] and d of super-block b: bytes 192..209 (a 20-byte window)
    auto load_hdr = [&](int b, u32x4m& sc, uint32_t& d) {
        const int off = voRow + b * Q6K_BYTES + 192;
        const int al = off & ~3;
        const uint32_t sh = (uint32_t)(off & 3) * 8u;
        const u32x4m ww = __builtin_amdgcn_raw_buffer_load_b128(rW, al, 0, 0);
        const uint32_t w4 = __builtin_amdgcn_raw_buffer_load_b32(rW, al + 16, 0, 0);
        sc = u32x4m{__builtin_amdgcn_alignbit(ww.y, ww.x, sh), __builtin_amdgcn_alignbit(ww.z, ww.y, sh),
                    __builtin_amdgcn_alignbit(ww.w, ww.z, sh), __builtin_amdgcn_alignbit(w4, ww.w, sh)};
        d = sh ? (w4 >> 16) : (w4 & 0xFFFFu);
    };

    f32x16m acc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = f32x16m{};

    auto compute = [&](int k, const u32x4m (&a)[3], const u32x4m& hsc) {
        const uint8_t* st = smem + (k & 1) * Q6_ST_BYTES;
        const int b = k >> 1, h = k & 1;
        const float* sD8 = (const float*)(st + Q6_ST_B);
        // the weight operands of the four 32-wide blocks: codes of elements
        // 32q + 16g .. +15 of the half, (ql >> nsh) & 15 | ((qh >> 2q) & 3) << 4,
        // as (q - 32) * sc (OUT 2: q - 32)
        h8m A[4][2];
        // the weight decode at raised wave priority (2560 x 9728 at N = 512
        // 88-90 -> 86 us, same arithmetic)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const u32x4m ql = (q & 1) ? a[1] : a[0];
            const uint32_t nsh = q >= 2 ? 4u : 0u, hsh = 2u * q;
            const u32x4m cw = ((ql >> nsh) & 0x0F0F0F0Fu) | (((a[2] >> hsh) & 0x03030303u) << 4u);
            if (OUT != 2) {
                const int gi = 8 * h + 2 * q + g;                // 16-group of this lane's elements
                const _Float16 sc = (_Float16)(float)(int)(int8_t)(uint8_t)(hsc[gi >> 2] >> (8 * (gi & 3)));
                A[q][0] = q6_to_h8_scaled(u32x2m{cw.x, cw.y}, sc);
                A[q][1] = q6_to_h8_scaled(u32x2m{cw.z, cw.w}, sc);
            } else {
                A[q][0] = bytes_to_h8(u32x2m{cw.x, cw.y}, 1056.0f);
                A[q][1] = bytes_to_h8(u32x2m{cw.z, cw.w}, 1056.0f);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        f32x4m dA[4];
        if (OUT != 2) {
#pragma unroll
            for (int m4 = 0; m4 < 4; m4++) dA[m4] = *(const f32x4m*)(&sDA[32 * w + 8 * m4 + 4 * g]);
        }
        // token tile by token tile: tmp = sum over the blocks q (in order) of
        // C * d8, then acc += tmp * d
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            const int tok = 32 * tt + li;
            const uint8_t* bt = st + tok * 256;
            f32x16m tmp = f32x16m{};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int P = 4 * q + 2 * g;
                const h8m B0 = *(const h8m*)(bt + 16 * (P ^ swz6(tok)));
                const h8m B1 = *(const h8m*)(bt + 16 * ((P + 1) ^ swz6(tok)));
                if (OUT == 2) {
                    // the two 16-groups separately: the other lane group's weights zeroed
#pragma unroll
                    for (int gg = 0; gg < 2; gg++) {
                        const h8m z = h8m{};
                        f32x16m C = mfma16(g == gg ? A[q][0] : z, B0, f32x16m{});
                        C = mfma16(g == gg ? A[q][1] : z, B1, C);
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const int r = row0 + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3);
                            const int tk = col0 + tok;
                            if (r < M && tk < N)
                                ((int*)y)[((int64_t)tk * M + r) * (K / 16) + b * 16 + 8 * h + 2 * q + gg] = (int)C[v];
                        }
                    }
                } else {
                    f32x16m C = mfma16(A[q][0], B0, f32x16m{});
                    C = mfma16(A[q][1], B1, C);                 // = C_g0*sc_g0 + C_g1*sc_g1, exact
                    const float d8 = sD8[q * Q6_TN + tok];
#pragma unroll
                    for (int v = 0; v < 16; v++) tmp[v] = __builtin_fmaf(C[v], d8, tmp[v]);
                }
            }
            if (OUT != 2) {
#pragma unroll
                for (int v = 0; v < 16; v++) acc[tt][v] = __builtin_fmaf(tmp[v], dA[v >> 2][v & 3], acc[tt][v]);
            }
        }
    };

    // Stage pipeline: stage k+1's weight pieces (and, before an even stage,
    // the next super-block's scales) into the other register set and its
    // codes + d8 into the other LDS buffer while stage k is computed; then
    // wait for everything (vmcnt(0)) and one barrier, which also orders all
    // reads of buffer k & 1 before the DMA of stage k+2 overwrites it.
    u32x4m a0[3], a1[3], hs0, hs1;
    uint32_t hd0, hd1;
    load_hdr(k0 >> 1, hs0, hd0);
    load_a(k0, a0);
    issue_b(k0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __builtin_amdgcn_s_barrier();
#pragma unroll 1
    for (int k = k0; k < k1; k += 2) {
        const int kl = k1 - 1;
        // even stage k: first half of super-block k/2 (scales hs0 / hd0)
        if (OUT != 2 && g == 0) sDA[arow] = f16_bits_to_f32(hd0);
        load_a(k + 1, a1);
        __builtin_amdgcn_sched_barrier(0);
        issue_b(k + 1);
        __builtin_amdgcn_wave_barrier();
        compute(k, a0, hs0);
        // next super-block's header (clamped: past the range it re-reads the last one)
        load_hdr(min(k + 2, kl) >> 1, hs1, hd1);
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __builtin_amdgcn_s_barrier();
        // odd stage k+1: second half, same scales
        // (past the last stage: stage k again, into the buffer nobody reads now)
        const int kn = k + 2 <= kl ? k + 2 : k;
        load_a(kn, a0);
        __builtin_amdgcn_sched_barrier(0);
        issue_b(kn);
        compute(k + 1, a1, hs0);
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __builtin_amdgcn_s_barrier();
        hs0 = hs1;
        hd0 = hd1;
    }
    if (OUT == 2) return;
#pragma unroll
    for (int tt = 0; tt < 4; tt++) {
        const int tok = col0 + 32 * tt + li;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = row0 + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3);
            if (r < M && tok < N) {
                if (OUT == 1) ((float*)y)[(int64_t)blockIdx.y * N * M + (int64_t)tok * M + r] = acc[tt][v];
                else          ((uint16_t*)y)[(int64_t)tok * M + r] = f32_to_f16_bits(acc[tt][v]);
            }
        }
    }
}

hipError_t mmq_launch(void* y, const uint8_t* W, int type, const void* codes, const uint32_t* scl, int M, int N,
                      int K, int Npad, int out_kind, int splits, hipStream_t st) {
    const int tn = type == TYPE_Q4_K ? TN : Q6_TN;
    const int tiles = ((M + TM - 1) / TM) * ((Npad + tn - 1) / tn);
    const int nb = K / QK_K;
    const int sps = (nb + splits - 1) / splits;
    if (splits < 1 || (splits > 1 && out_kind != 1) || (splits - 1) * sps >= nb) return hipErrorInvalidValue;
    const dim3 grid(tiles, splits);
    if (type == TYPE_Q4_K) {
        MmqSegs sg;
        for (int i = 0; i < 3; i++) { sg.W[i] = W; sg.y[i] = y; sg.M[i] = i == 0 ? M : 0; }
        sg.rt0[0] = 0;
        for (int i = 1; i < 4; i++) sg.rt0[i] = (M + TM - 1) / TM;
        const uint8_t* c8 = (const uint8_t*)codes;
        if (q4k_tt((int64_t)tiles * splits * 4) == 1) {
            const dim3 g1(2 * tiles, splits);
            if (out_kind == 0) hipLaunchKernelGGL((mmq_q4k_kernel<0, 1>), g1, dim3(MMQ_THREADS), 0, st, sg, c8, scl, N, K, Npad, sps);
            else if (out_kind == 1) hipLaunchKernelGGL((mmq_q4k_kernel<1, 1>), g1, dim3(MMQ_THREADS), 0, st, sg, c8, scl, N, K, Npad, sps);
            else hipLaunchKernelGGL((mmq_q4k_kernel<2, 1>), g1, dim3(MMQ_THREADS), 0, st, sg, c8, scl, N, K, Npad, sps);
        } else {
            if (out_kind == 0) hipLaunchKernelGGL((mmq_q4k_kernel<0, 2>), grid, dim3(MMQ_THREADS), 0, st, sg, c8, scl, N, K, Npad, sps);
            else if (out_kind == 1) hipLaunchKernelGGL((mmq_q4k_kernel<1, 2>), grid, dim3(MMQ_THREADS), 0, st, sg, c8, scl, N, K, Npad, sps);
            else hipLaunchKernelGGL((mmq_q4k_kernel<2, 2>), grid, dim3(MMQ_THREADS), 0, st, sg, c8, scl, N, K, Npad, sps);
        }
    } else {
        const uint16_t* c16 = (const uint16_t*)codes;
        if (out_kind == 0) hipLaunchKernelGGL(mmq_q6k_kernel<0>, grid, dim3(MMQ_THREADS), 0, st, y, W, c16, scl, M, N, K, Npad, sps);
        else if (out_kind == 1) hipLaunchKernelGGL(mmq_q6k_kernel<1>, grid, dim3(MMQ_THREADS), 0, st, y, W, c16, scl, M, N, K, Npad, sps);
        else hipLaunchKernelGGL(mmq_q6k_kernel<2>, grid, dim3(MMQ_THREADS), 0, st, y, W, c16, scl, M, N, K, Npad, sps);
    }
    return hipGetLastError();
}

// y[i] = sum over s = 0..S-1 (in order) of ws[s][i]; fp16 or fp32 out
// OUT 0: fp16, 1: fp32, 2: fp16 of fp16(sum) + res (the engine's residual add
// after the projection, one more fp16 rounding)
template <int OUT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(void* __restrict__ y, const float* __restrict__ ws,
                                                            int64_t n, int S, const uint16_t* __restrict__ res) {
#pragma clang fp contract(off)
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    if (i + 4 <= n && (n & 3) == 0) {
        f32x4m a = *(const f32x4m*)(ws + i);
        for (int s = 1; s < S; s++) {
            const f32x4m b = *(const f32x4m*)(ws + (int64_t)s * n + i);
            a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        }
        if (OUT == 1) {
            *(f32x4m*)((float*)y + i) = a;
        } else if (OUT == 2) {
            const u32x2m r = *(const u32x2m*)(res + i);
            const float s0 = round_to_f16(a.x) + f16_bits_to_f32(r.x & 0xFFFFu), s1 = round_to_f16(a.y) + f16_bits_to_f32(r.x >> 16);
            const float s2 = round_to_f16(a.z) + f16_bits_to_f32(r.y & 0xFFFFu), s3 = round_to_f16(a.w) + f16_bits_to_f32(r.y >> 16);
            *(u32x2m*)((uint16_t*)y + i) = u32x2m{(uint32_t)f32_to_f16_bits(s0) | ((uint32_t)f32_to_f16_bits(s1) << 16),
                                                  (uint32_t)f32_to_f16_bits(s2) | ((uint32_t)f32_to_f16_bits(s3) << 16)};
        } else {
            const u32x2m o = u32x2m{(uint32_t)f32_to_f16_bits(a.x) | ((uint32_t)f32_to_f16_bits(a.y) << 16),
                                    (uint32_t)f32_to_f16_bits(a.z) | ((uint32_t)f32_to_f16_bits(a.w) << 16)};
            *(u32x2m*)((uint16_t*)y + i) = o;
        }
        return;
    }
    for (int64_t e = i; e < i + 4 && e < n; e++) {
        float a = ws[e];
        for (int s = 1; s < S; s++) a += ws[(int64_t)s * n + e];
        if (OUT == 1) ((float*)y)[e] = a;
        else if (OUT == 2) ((uint16_t*)y)[e] = f32_to_f16_bits(round_to_f16(a) + f16_bits_to_f32(res[e]));
        else          ((uint16_t*)y)[e] = f32_to_f16_bits(a);
    }
}

hipError_t splitk_reduce_launch(void* y, const float* ws, int64_t n, int splits, int out_kind, hipStream_t st,
                                const uint16_t* res) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 1023) / 1024;
    if (out_kind == 1) hipLaunchKernelGGL(splitk_reduce_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, st, y, ws, n, splits, res);
    else if (res)      hipLaunchKernelGGL(splitk_reduce_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, st, y, ws, n, splits, res);
    else               hipLaunchKernelGGL(splitk_reduce_kernel<0>, dim3((unsigned)blocks), dim3(256), 0, st, y, ws, n, splits, res);
    return hipGetLastError();
}

hipError_t mmq_q4k_multi_launch(const uint8_t* const* W, void* const* y, const int* M, int nseg, const uint8_t* codes,
                                const uint32_t* scl, int N, int K, int Npad, hipStream_t st) {
    if (nseg < 1 || nseg > 3) return hipErrorInvalidValue;
    MmqSegs sg;
    sg.rt0[0] = 0;
    for (int i = 0; i < 3; i++) {
        const int j = i < nseg ? i : nseg - 1;
        sg.W[i] = W[j]; sg.y[i] = y[j]; sg.M[i] = i < nseg ? M[i] : 0;
        sg.rt0[i + 1] = sg.rt0[i] + (sg.M[i] + TM - 1) / TM;
    }
    const dim3 grid(sg.rt0[3] * (Npad / TN), 1);
    if (q4k_tt((int64_t)grid.x * 4) == 1)
        hipLaunchKernelGGL((mmq_q4k_kernel<0, 1>), dim3(2 * grid.x), dim3(MMQ_THREADS), 0, st, sg, codes, scl, N, K, Npad, K / QK_K);
    else
        hipLaunchKernelGGL((mmq_q4k_kernel<0, 2>), grid, dim3(MMQ_THREADS), 0, st, sg, codes, scl, N, K, Npad, K / QK_K);
    return hipGetLastError();
}

hipError_t mmq_q4k_qkv_front_launch(const uint8_t* const* W, uint16_t* const* y, const int* M, const uint8_t* codes,
                                    const uint32_t* scl, int N, int K, int Npad, const QKPostArgs& fa,
                                    hipStream_t st) {
    if (fa.head_dim != TM || M[0] != fa.n_heads * TM || M[1] != fa.n_kv * TM || M[2] != fa.n_kv * TM ||
        fa.q != y[0] || fa.k != y[1] || fa.v != y[2] || fa.q_in_stride || fa.kv_in_stride || fa.pos_dev)
        return hipErrorInvalidValue;
    MmqSegs sg;
    sg.rt0[0] = 0;
    for (int i = 0; i < 3; i++) {
        sg.W[i] = W[i]; sg.y[i] = y[i]; sg.M[i] = M[i];
        sg.rt0[i + 1] = sg.rt0[i] + M[i] / TM;
    }
    const dim3 grid(sg.rt0[3] * (Npad / TN), 1);
    if (q4k_tt((int64_t)grid.x * 4) == 1)
        hipLaunchKernelGGL(mmq_q4k_front_kernel<1>, dim3(2 * grid.x), dim3(MMQ_THREADS), 0, st, sg, codes, scl, N, K, Npad, fa);
    else
        hipLaunchKernelGGL(mmq_q4k_front_kernel<2>, grid, dim3(MMQ_THREADS), 0, st, sg, codes, scl, N, K, Npad, fa);
    return hipGetLastError();
}

hipError_t mmq_q4k_swiglu_launch(const uint8_t* gate, const uint8_t* up, int M, const uint8_t* codes,
                                 const uint32_t* scl, int N, int K, int Npad, void* act_codes, uint32_t* act_scl,
                                 bool act_i8, hipStream_t st) {
    if (M <= 0 || M % 64 || Npad % TN || Npad < N) return hipErrorInvalidValue;
    MmqSegs sg;
    sg.W[0] = gate; sg.W[1] = up; sg.W[2] = up;
    sg.y[0] = sg.y[1] = sg.y[2] = nullptr;
    sg.M[0] = M; sg.M[1] = M; sg.M[2] = 0;
    sg.rt0[0] = 0; sg.rt0[1] = M / 64; sg.rt0[2] = M / 64; sg.rt0[3] = M / 64;
    MmqActOut ao{act_codes, act_scl, act_i8 ? 1 : 0};
    const dim3 grid(sg.rt0[3] * (Npad / TN), 1);
    if (q4k_tt((int64_t)grid.x * 4) == 1)
        hipLaunchKernelGGL(mmq_q4k_swiglu_kernel<1>, dim3(2 * grid.x), dim3(MMQ_THREADS), 0, st, sg, codes, scl, N, K, Npad, ao);
    else
        hipLaunchKernelGGL(mmq_q4k_swiglu_kernel<2>, grid, dim3(MMQ_THREADS), 0, st, sg, codes, scl, N, K, Npad, ao);
    return hipGetLastError();
}

int mmq_splits(int M, int N, int K, int type) {
#ifdef JLLM_MMQ_TT_DEBUG
    if (const char* e = getenv(type == TYPE_Q6_K ? "JLLM_MMQ_S6" : "JLLM_MMQ_S4")) {
        const int S = atoi(e), nb0 = K / QK_K, sps0 = (nb0 + S - 1) / S;
        if (S > 0) return (nb0 + sps0 - 1) / sps0;
    }
#endif
    const bool q6 = type == TYPE_Q6_K;
    const int tn = q6 ? Q6_TN : TN;
    const int64_t tiles = (int64_t)((M + TM - 1) / TM) * ((N + tn - 1) / tn);
    const int nb = K / QK_K;
    if ((!q6 && tiles >= MMQ_MULTI_MIN_TILES) || nb < 4) return 1;
    // Ranges of whole super-blocks, chosen by a cost model fitted on MI355X.
    // The kernels are VALU-bound per CU: a launch takes about
    //   4 us + rounds x g(w) x (super-blocks per range),
    // w the workgroups a CU holds at once (ceil(workgroups / 256), at most
    // 3 for Q4_K, 2 for Q6_K, whose workgroups hold 69 KB of LDS), rounds the
    // waves of workgroups that takes; Q4_K g(1, 2, 3) = 2.85, 4.56, 6.27 us
    // (fitted on 9728 / 2560 / 1024 rows, K 2560 / 4096 / 9728, N 64-512),
    // Q6_K g(1, 2) = 6.0, 7.0 us (2560 / 9728 rows, K 4096 / 9728 / 2560,
    // N 64-1261); split-K adds ~5 us (Q4_K) / ~8 us (Q6_K) for the partials
    // and the reduce launch, and the fp32 partials' write and read at ~3 TB/s.
    // It picks the measured best count, or one within 2 %, in every fitted
    // case.
    const int wmax = q6 ? 2 : 3;
    auto g = [&](int64_t w) {
        if (q6) return w == 1 ? 6.0 : 7.0;
        return w == 1 ? 2.85 : (w == 2 ? 4.56 : 6.27);
    };
    int best = 1;
    double best_cost = 0.0;
    for (int S = 1; S <= std::min(q6 ? 19 : 16, nb); S++) {
        const int sps = (nb + S - 1) / S, eff = (nb + sps - 1) / sps;
        const int64_t c = (tiles * eff + 255) / 256;                 // workgroups per CU
        const int64_t rounds = (c + wmax - 1) / wmax, w = std::min<int64_t>(c, wmax);
        double cost = 4.0 + (double)rounds * g(w) * sps;
        if (eff > 1) cost += (q6 ? 8.0 : 5.0) + (double)eff * N * M * 8.0 / 3.0e6;
        if (S == 1 || cost < best_cost) { best = eff; best_cost = cost; }
    }
    return best;
}

}  // namespace jllm_hip
