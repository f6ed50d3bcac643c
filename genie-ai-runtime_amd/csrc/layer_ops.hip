// layer_ops.hip -- the decoder-layer kernels that sit between the quantized
// matmuls (gfx950): RMSNorm (+residual), SwiGLU, residual add, RoPE, the
// fused q/k-norm + RoPE + KV-cache store, embedding-row dequant and greedy
// argmax.  All are HBM/latency-bound element-wise or row-reduction kernels:
// 16-byte loads where the layout allows, wave64 shuffle reductions, no LDS
// beyond a few cross-wave partials.
//
// Arithmetic follows the reference kernels operation by operation in fp32
// (no FMA contraction where the reference's result is a rounded product
// chain), with fp16 rounding at the same points:
//   RMSNorm   fused_rmsnorm_residual_kernel  fused_norm.cu:33-101
//   SwiGLU    swiglu_kernel                  convert.cu:85-112
//   vec_add   vec_add_kernel                 decode.cu:60-78
//   RoPE      rope_kernel / rope_batched_kernel rope.cu:322-367, :476-497
//   KV int8   fp16_to_int8_kernel            convert.cu:26-69
//   embedding dequant_embedding_q4k/q6k_kernel gemv_q4.cu:793-864
//   argmax    sample_greedy (host)           sample.cpp:160-170
#include <float.h>
#include <limits.h>
#include <math.h>
#include "kq_common.h"
#include "layer_ops.h"
#include "qk_front.h"

namespace jllm_hip {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// RMSNorm: out = half((x + res) * rrms * w), rrms = 1/sqrt(sum((x+res)^2)/dim
// + eps).  GS threads per row (64: one wave per row for head-sized rows, 256:
// one workgroup per hidden-sized row).  Two passes over the row; the second
// re-reads x from cache.  out may alias x (each element is read before it is
// written, by the same thread).  VEC = 8 (16-byte accesses) or 2.
template <bool WF32, bool RES, int GS, int VEC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t* out, const uint16_t* x, const uint16_t* res,
                                                      const void* w, int rows, int dim, float eps) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    constexpr int RPB = 256 / GS;                        // rows per block
    const int t = threadIdx.x % GS, rb = threadIdx.x / GS;
    const int row = blockIdx.x * RPB + rb;
    const bool live = row < rows;
    const int64_t off = (int64_t)(live ? row : 0) * dim;
    auto load = [&](const uint16_t* p, int i, float (&v)[VEC]) {
        if (VEC == 8) {
            const u32x4v u = *(const u32x4v*)(p + off + i);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const half2_t h = as_h2(u[e]);
                v[2 * e] = (float)h[0];
                v[2 * e + 1] = (float)h[1];
            }
        } else {
            const half2_t h = as_h2(*(const uint32_t*)(p + off + i));
            v[0] = (float)h[0];
            v[1] = (float)h[1];
        }
    };
    auto row_vals = [&](int i, float (&v)[VEC]) {
        load(x, i, v);
        if (RES) {
            float r[VEC];
            load(res, i, r);
#pragma unroll
            for (int e = 0; e < VEC; e++) v[e] += r[e];
        }
    };
    float ss = 0.0f;
    if (live)
        for (int i = t * VEC; i < dim; i += GS * VEC) {
            float v[VEC];
            row_vals(i, v);
#pragma unroll
            for (int e = 0; e < VEC; e += 2) ss += v[e] * v[e] + v[e + 1] * v[e + 1];
        }
    ss = wave_sum(ss);
    if (GS == 256) {
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = (red[0] + red[1]) + (red[2] + red[3]);
    }
    if (!live) return;
    const float rrms = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = t * VEC; i < dim; i += GS * VEC) {
        float v[VEC], wv[VEC];
        row_vals(i, v);
        if (WF32) {
#pragma unroll
            for (int e = 0; e < VEC; e++) wv[e] = ((const float*)w)[i + e];
        } else {
#pragma unroll
            for (int e = 0; e < VEC; e++) wv[e] = f16_bits_to_f32(((const uint16_t*)w)[i + e]);
        }
        uint32_t o[VEC / 2];
#pragma unroll
        for (int e = 0; e < VEC; e += 2)
            o[e / 2] = (uint32_t)f32_to_f16_bits(v[e] * rrms * wv[e]) |
                       ((uint32_t)f32_to_f16_bits(v[e + 1] * rrms * wv[e + 1]) << 16);
        if (VEC == 8) *(u32x4v*)(out + off + i) = u32x4v{o[0], o[1], o[2], o[3]};
        else *(uint32_t*)(out + off + i) = o[0];
    }
}

template <bool WF32, bool RES>
static void rmsnorm_go(uint16_t* out, const uint16_t* x, const uint16_t* res, const void* w, int rows, int dim,
                       float eps, hipStream_t st) {
    const bool v8 = dim % 8 == 0 && ((uintptr_t)out | (uintptr_t)x | (uintptr_t)(res ? res : x)) % 16 == 0 &&
                    (uintptr_t)w % (WF32 ? 32 : 16) == 0;
    if (dim <= 1024) {
        const dim3 g((rows + 3) / 4);
        if (v8) hipLaunchKernelGGL((rmsnorm_kernel<WF32, RES, 64, 8>), g, dim3(256), 0, st, out, x, res, w, rows, dim, eps);
        else hipLaunchKernelGGL((rmsnorm_kernel<WF32, RES, 64, 2>), g, dim3(256), 0, st, out, x, res, w, rows, dim, eps);
    } else {
        const dim3 g(rows);
        if (v8) hipLaunchKernelGGL((rmsnorm_kernel<WF32, RES, 256, 8>), g, dim3(256), 0, st, out, x, res, w, rows, dim, eps);
        else hipLaunchKernelGGL((rmsnorm_kernel<WF32, RES, 256, 2>), g, dim3(256), 0, st, out, x, res, w, rows, dim, eps);
    }
}

hipError_t rmsnorm_launch(uint16_t* out, const uint16_t* x, const uint16_t* res, const void* w, int rows, int dim,
                          float eps, bool w_fp32, hipStream_t st) {
    if (w_fp32) {
        if (res) rmsnorm_go<true, true>(out, x, res, w, rows, dim, eps, st);
        else rmsnorm_go<true, false>(out, x, res, w, rows, dim, eps, st);
    } else {
        if (res) rmsnorm_go<false, true>(out, x, res, w, rows, dim, eps, st);
        else rmsnorm_go<false, false>(out, x, res, w, rows, dim, eps, st);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Element-wise: SwiGLU out = half(g / (1 + e^-g) * u) and the residual add
// out = half(a + b).  Eight elements per thread (16-byte accesses) over the
// aligned body, one element per thread for the tail.

template <int OP, bool V>
__global__ __launch_bounds__(256) void eltwise_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ a,
                                                      const uint16_t* __restrict__ b, int64_t n) {
#pragma clang fp contract(off)
    const int64_t i8 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (V && i8 + 8 <= n) {
        const u32x4v ua = *(const u32x4v*)(a + i8), ub = *(const u32x4v*)(b + i8);
        u32x4v o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const half2_t ha = as_h2(ua[e]), hb = as_h2(ub[e]);
            float r0, r1;
            if (OP == 0) { r0 = silu_mul((float)ha[0], (float)hb[0]); r1 = silu_mul((float)ha[1], (float)hb[1]); }
            else { r0 = (float)ha[0] + (float)hb[0]; r1 = (float)ha[1] + (float)hb[1]; }
            o[e] = (uint32_t)f32_to_f16_bits(r0) | ((uint32_t)f32_to_f16_bits(r1) << 16);
        }
        *(u32x4v*)(out + i8) = o;
    } else {
        for (int64_t i = i8; i < n && i < i8 + 8; i++) {
            const float fa = f16_bits_to_f32(a[i]), fb = f16_bits_to_f32(b[i]);
            out[i] = f32_to_f16_bits(OP == 0 ? silu_mul(fa, fb) : fa + fb);
        }
    }
}

template <int OP>
static hipError_t eltwise_go(uint16_t* out, const uint16_t* a, const uint16_t* b, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int64_t thr = (n + 7) / 8;
    const dim3 g((unsigned)((thr + 255) / 256));
    if ((((uintptr_t)out | (uintptr_t)a | (uintptr_t)b) & 15) == 0)
        hipLaunchKernelGGL((eltwise_kernel<OP, true>), g, dim3(256), 0, st, out, a, b, n);
    else
        hipLaunchKernelGGL((eltwise_kernel<OP, false>), g, dim3(256), 0, st, out, a, b, n);
    return hipGetLastError();
}
hipError_t swiglu_launch(uint16_t* out, const uint16_t* gate, const uint16_t* up, int64_t n, hipStream_t st) {
    return eltwise_go<0>(out, gate, up, n, st);
}
hipError_t vec_add_launch(uint16_t* out, const uint16_t* a, const uint16_t* b, int64_t n, hipStream_t st) {
    return eltwise_go<1>(out, a, b, n, st);
}

// ---------------------------------------------------------------------------
// RoPE.  freq[i] = 1 / theta^(2i/hd) is computed on the host in fp32 exactly
// as the reference writes it (1.0f / powf(theta, (2.0f*i)/hd)); the angle
// is the fp32 product position * freq[i] and cos/sin are evaluated on it,
// so the rounding of the angle matches the reference.  Pair i is
// (i, i + hd/2) for neox, (2i, 2i+1) otherwise.
void rope_frequencies(RopeFreq& fr, int head_dim, float theta) {
    for (int i = 0; i < ROPE_MAX_HALF; i++)
        fr.f[i] = i < head_dim / 2 ? 1.0f / powf(theta, (2.0f * (float)i) / (float)head_dim) : 0.0f;
}

__device__ __forceinline__ void rotate(float v0, float v1, float c, float s, float& r0, float& r1) {
#pragma clang fp contract(off)
    r0 = round_to_f16(v0 * c - v1 * s);
    r1 = round_to_f16(v0 * s + v1 * c);
}

// one thread per (token, head, pair)
__global__ __launch_bounds__(256) void rope_kernel(uint16_t* q, uint16_t* k, int n_heads, int n_kv, int hd,
                                                   int start_pos, int N, int q_stride, int k_stride, RopeFreq fr,
                                                   int neox, const int* pos_dev) {
    const int h2 = hd / 2;
    const int64_t per_tok = (int64_t)(n_heads + n_kv) * h2;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= per_tok * N) return;
    const int t = (int)(gid / per_tok);
    const int r = (int)(gid % per_tok);
    const int head = r / h2, i = r % h2;
    uint16_t* p = head < n_heads ? q + (int64_t)t * q_stride + (int64_t)head * hd
                                 : k + (int64_t)t * k_stride + (int64_t)(head - n_heads) * hd;
    const int p0 = pos_dev ? *pos_dev : start_pos;
    const float ang = (float)(p0 + t) * fr.f[i];
    float s, c;
    sincosf(ang, &s, &c);
    const int i0 = neox ? i : 2 * i, i1 = neox ? i + h2 : 2 * i + 1;
    float r0, r1;
    rotate(f16_bits_to_f32(p[i0]), f16_bits_to_f32(p[i1]), c, s, r0, r1);
    p[i0] = f32_to_f16_bits(r0);
    p[i1] = f32_to_f16_bits(r1);
}

hipError_t rope_launch(uint16_t* q, uint16_t* k, int n_heads, int n_kv, int head_dim, int start_pos, int N,
                       int q_stride, int k_stride, const RopeFreq& fr, bool neox, hipStream_t st,
                       const int* pos_dev) {
    const int64_t total = (int64_t)(n_heads + n_kv) * (head_dim / 2) * N;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, q, k, n_heads, n_kv,
                       head_dim, start_pos, N, q_stride, k_stride, fr, neox ? 1 : 0, pos_dev);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Fused attention front for N tokens: one wave per (token, slot), slots =
// n_heads q heads, n_kv k heads, n_kv v heads.  Lane i < hd/2 holds the
// rotary pair i (both elements), so the norm is one wave reduction and the
// rotation needs no data exchange.  The fp16 roundings of the unfused
// sequence are kept: normed value -> fp16 (rmsnorm output), rotated ->
// fp16 (rope output), then the KV quantiser reads those fp16 values.
// Replaces decode.cu:1441-1478 (q/k norm, rope_inplace, fp16_to_int8 x2)
// and the per-token loop of decode.cu:1806-1842.
__global__ __launch_bounds__(256) void qk_post_kernel(QKPostArgs a) {
    // every scalar argument requested at one point (one batch of scalar
    // loads), then the wave's global loads -- its head's pair, the norm
    // weights, the position -- before any arithmetic that waits for them
    asm volatile("" :: "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.q_norm), "s"(a.k_norm), "s"(a.k_dst), "s"(a.v_dst),
                 "s"(a.k_scales), "s"(a.v_scales), "s"(a.kv_stride), "s"(a.n_heads), "s"(a.n_kv), "s"(a.head_dim),
                 "s"(a.cache_head_dim), "s"(a.start_pos), "s"(a.N), "s"(a.eps), "s"(a.norm_fp32), "s"(a.neox),
                 "s"(a.kv_int8), "s"(a.q_in_stride), "s"(a.kv_in_stride), "s"(a.pos_dev));
    const int hd = a.head_dim;
    const int slots = a.n_heads + 2 * a.n_kv;
    const int gw = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);   // wave-uniform: scalar
    const int l = threadIdx.x & 63;
    if (gw >= slots * a.N) return;                      // whole wave exits together
    const int t = gw / slots, slot = gw % slots;
    const int kind = slot < a.n_heads ? 0 : (slot < a.n_heads + a.n_kv ? 1 : 2);   // q, k, v
    const int head = kind == 0 ? slot : (kind == 1 ? slot - a.n_heads : slot - a.n_heads - a.n_kv);
    const int64_t qs = a.q_in_stride ? a.q_in_stride : (int64_t)a.n_heads * hd;
    const int64_t ks = a.kv_in_stride ? a.kv_in_stride : (int64_t)a.n_kv * hd;
    const uint16_t* src = kind == 0 ? a.q + t * qs + (int64_t)head * hd
                                    : (kind == 1 ? a.k : a.v) + t * ks + (int64_t)head * hd;
    const void* norm = kind < 2 ? (kind == 0 ? a.q_norm : a.k_norm) : nullptr;
    const bool act = l < hd / 2;
    int i0, i1;
    front_idx(hd, a.neox != 0, l, i0, i1);
    const int j0 = act ? i0 : 0, j1 = act ? i1 : 0;    // lanes past the pairs read element 0
    // raw loads first (all in flight together), conversions after
    const uint16_t x0 = src[j0], x1 = src[j1];
    uint32_t wr0 = 0, wr1 = 0;
    if (norm) {
        if (a.norm_fp32) { wr0 = ((const uint32_t*)norm)[j0]; wr1 = ((const uint32_t*)norm)[j1]; }
        else { wr0 = ((const uint16_t*)norm)[j0]; wr1 = ((const uint16_t*)norm)[j1]; }
    }
    const float fq = a.fr.f[act ? l : 0];
    const int pd = a.pos_dev ? *a.pos_dev : 0;
    __builtin_amdgcn_sched_barrier(0);
    const float v0i = act ? f16_bits_to_f32(x0) : 0.0f, v1i = act ? f16_bits_to_f32(x1) : 0.0f;
    float v0 = v0i, v1 = v1i, w0 = 0.0f, w1 = 0.0f;
    if (norm && act) {
        if (a.norm_fp32) { w0 = __builtin_bit_cast(float, wr0); w1 = __builtin_bit_cast(float, wr1); }
        else { w0 = f16_bits_to_f32((uint16_t)wr0); w1 = f16_bits_to_f32((uint16_t)wr1); }
    }
    const int p0 = a.pos_dev ? __builtin_amdgcn_readfirstlane(pd) : a.start_pos;
    const int64_t r0 = a.pos_dev ? p0 : 0;            // cache row of token 0 relative to k_dst / v_dst
    const int pos = p0 + t;
    front_finish(a, kind, head, t, r0, pos, l, act, i0, i1, v0, v1, w0, w1, fq, qs, ks);
}

hipError_t qk_post_launch(const QKPostArgs& a, hipStream_t st) {
    const int64_t waves = (int64_t)(a.n_heads + 2 * a.n_kv) * a.N;
    if (waves <= 0) return hipSuccess;
    hipLaunchKernelGGL(qk_post_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Embedding rows: dst[t][hidden] = dequant(W row tokens[t]).  Each thread
// produces 8 consecutive weights of one 256-weight super-block (one 16-byte
// store); a 256-thread workgroup covers 8 super-blocks.
__device__ __forceinline__ void q4k_sc_min(const uint8_t* q, int j, int& d, int& m) {
    if (j < 4) { d = q[j] & 63; m = q[j + 4] & 63; }
    else { d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4); m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
}

template <int TYPE>
__global__ __launch_bounds__(256) void embed_kernel(uint16_t* __restrict__ dst, const uint8_t* __restrict__ W,
                                                    const int32_t* __restrict__ tokens, int token0, int N, int nb,
                                                    int vocab) {
#pragma clang fp contract(off)
    const int64_t g = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);      // (token, super-block)
    if (g >= (int64_t)N * nb) return;
    const int t = (int)(g / nb), b = (int)(g % nb);
    const int tok = tokens ? tokens[t] : token0;
    const int i = (threadIdx.x & 31) * 8;                                // first weight of this thread
    float val[8];
    if (vocab > 0 && (tok < 0 || tok >= vocab)) {                         // id out of range: zero row
#pragma unroll
        for (int e = 0; e < 8; e++) val[e] = 0.0f;
    } else if (TYPE == 12) {
        const uint8_t* blk = W + ((int64_t)tok * nb + b) * 144;
        const float dall = f16_bits_to_f32(blk[0] | (blk[1] << 8));
        const float dmin = f16_bits_to_f32(blk[2] | (blk[3] << 8));
        const int il = i >> 6, l64 = i & 63, l32 = l64 & 31;
        int sc, mn;
        q4k_sc_min(blk + 4, 2 * il + (l64 >= 32), sc, mn);
        const uint8_t* qs = blk + 16 + 32 * il + l32;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int qv = l64 < 32 ? (qs[e] & 0xF) : (qs[e] >> 4);
            val[e] = dall * (float)sc * (float)qv - dmin * (float)mn;
        }
    } else if (TYPE == 13) {      // the engine's host Q5_K row dequant, decode.cu:230-266
        const uint8_t* blk = W + ((int64_t)tok * nb + b) * 176;
        const float dall = f16_bits_to_f32(blk[0] | (blk[1] << 8));
        const float dmin = f16_bits_to_f32(blk[2] | (blk[3] << 8));
        const int il = i >> 6, l64 = i & 63, l32 = l64 & 31, hi = l64 >= 32;
        int sc, mn;
        q4k_sc_min(blk + 4, 2 * il + hi, sc, mn);
        const float d1 = dall * (float)sc, dm1 = dmin * (float)mn;
        const uint8_t* qs = blk + 48 + 32 * il + l32;
        const uint8_t* qh = blk + 16 + l32;
        const int ub = 2 * il + hi;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int qv = (hi ? (qs[e] >> 4) : (qs[e] & 0xF)) + (((qh[e] >> ub) & 1) ? 16 : 0);
            val[e] = d1 * (float)qv - dm1;
        }
    } else {
        const uint8_t* blk = W + ((int64_t)tok * nb + b) * 210;
        const float d = f16_bits_to_f32(blk[208] | (blk[209] << 8));
        const int hb = i >> 7, local = i & 127, lane = local & 31, quarter = local >> 5;
        const uint8_t* ql = blk + hb * 64;
        const uint8_t* qh = blk + 128 + hb * 32;
        const int8_t* scs = (const int8_t*)(blk + 192) + hb * 8;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int ln = lane + e, is = ln >> 4;
            const int lo = (quarter & 1) ? ql[ln + 32] : ql[ln];
            const int qv = ((quarter >> 1) ? (lo >> 4) : (lo & 0xF)) | (((qh[ln] >> (2 * quarter)) & 3) << 4);
            val[e] = d * (float)scs[is + 2 * quarter] * (float)(qv - 32);
        }
    }
    u32x4v o;
#pragma unroll
    for (int e = 0; e < 4; e++)
        o[e] = (uint32_t)f32_to_f16_bits(val[2 * e]) | ((uint32_t)f32_to_f16_bits(val[2 * e + 1]) << 16);
    *(u32x4v*)(dst + (int64_t)t * nb * 256 + (int64_t)b * 256 + i) = o;
}

hipError_t embed_launch(uint16_t* dst, const void* W, int type, const int32_t* tokens, int token0, int N, int hidden,
                        int vocab, hipStream_t st) {
    const int nb = hidden / 256;
    const int64_t groups = (int64_t)N * nb;
    if (groups <= 0) return hipSuccess;
    const dim3 g((unsigned)((groups + 7) / 8));
    if (type == 12) hipLaunchKernelGGL((embed_kernel<12>), g, dim3(256), 0, st, dst, (const uint8_t*)W, tokens, token0, N, nb, vocab);
    else if (type == 13) hipLaunchKernelGGL((embed_kernel<13>), g, dim3(256), 0, st, dst, (const uint8_t*)W, tokens, token0, N, nb, vocab);
    else hipLaunchKernelGGL((embed_kernel<14>), g, dim3(256), 0, st, dst, (const uint8_t*)W, tokens, token0, N, nb, vocab);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Greedy argmax over fp32 logits: the lowest index of the largest finite
// value (0 when none is finite), i.e. the host loop of sample_greedy.  Two
// launches: AM_BLOCKS workgroups each reduce a contiguous chunk (float4
// loads over the aligned body) to one (value, index) candidate in a
// file-scope device array, then one wave merges the candidates in index
// order.  Calls on one device share that array: they must be serialised
// (one stream), like the library's other scratch users.
constexpr int AM_BLOCKS = 128, AM_THREADS = 256;
__device__ float g_am_val[AM_BLOCKS];
__device__ int g_am_idx[AM_BLOCKS];

__device__ __forceinline__ void arg_better(float v, int i, float& bv, int& bi) {
    if (isfinite(v) && (v > bv || (v == bv && i < bi))) { bv = v; bi = i; }
}
__device__ __forceinline__ void arg_merge(float ov, int oi, float& bv, int& bi) {
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

// the wave's best (value, index) in every lane: DPP steps within each
// 16-lane row, then the four row winners (arg_merge is a total order, so
// the merge order does not change the result)
__device__ __forceinline__ void wave_arg_merge(float& bv, int& bi) {
#define JLLM_AM_STEP(C) arg_merge(dpp_mov_f<C>(bv), __builtin_amdgcn_mov_dpp(bi, C, 0xF, 0xF, false), bv, bi)
    JLLM_AM_STEP(0xB1);
    JLLM_AM_STEP(0x4E);
    JLLM_AM_STEP(0x141);
    JLLM_AM_STEP(0x140);
#undef JLLM_AM_STEP
    float v0 = readlane_f(bv, 0), v1 = readlane_f(bv, 16), v2 = readlane_f(bv, 32), v3 = readlane_f(bv, 48);
    int i0 = __builtin_amdgcn_readlane(bi, 0), i1 = __builtin_amdgcn_readlane(bi, 16);
    int i2 = __builtin_amdgcn_readlane(bi, 32), i3 = __builtin_amdgcn_readlane(bi, 48);
    arg_merge(v1, i1, v0, i0);
    arg_merge(v3, i3, v2, i2);
    arg_merge(v2, i2, v0, i0);
    bv = v0;
    bi = i0;
}

__global__ __launch_bounds__(AM_THREADS) void argmax_part_kernel(const float* __restrict__ x, int n, int chunk) {
    __shared__ float sv[AM_THREADS / 64];
    __shared__ int si[AM_THREADS / 64];
    const int t = threadIdx.x;
    const int b0 = blockIdx.x * chunk, b1 = min(n, b0 + chunk);      // chunk is a multiple of 4
    float bv = -INFINITY;
    int bi = INT_MAX;
    if (((uintptr_t)x & 15) == 0) {
        const int q1 = b0 + ((b1 - b0) & ~3);
        for (int j = b0 + 4 * t; j < q1; j += 4 * AM_THREADS) {
            const float4 f = *(const float4*)(x + j);
            arg_better(f.x, j, bv, bi);
            arg_better(f.y, j + 1, bv, bi);
            arg_better(f.z, j + 2, bv, bi);
            arg_better(f.w, j + 3, bv, bi);
        }
        for (int j = q1 + t; j < b1; j += AM_THREADS) arg_better(x[j], j, bv, bi);
    } else {
        for (int j = b0 + t; j < b1; j += AM_THREADS) arg_better(x[j], j, bv, bi);
    }
    wave_arg_merge(bv, bi);
    if ((t & 63) == 0) { sv[t >> 6] = bv; si[t >> 6] = bi; }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < AM_THREADS / 64; w++) arg_merge(sv[w], si[w], bv, bi);
        g_am_val[blockIdx.x] = bv;
        g_am_idx[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(int32_t* out, int nblocks) {
    const int t = threadIdx.x;
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int b = t; b < nblocks; b += 64) arg_merge(g_am_val[b], g_am_idx[b], bv, bi);
    wave_arg_merge(bv, bi);
    if (t == 0) out[0] = bi == INT_MAX ? 0 : bi;
}

hipError_t argmax_launch(int32_t* out, const float* x, int n, hipStream_t st) {
    if (n <= 0) return hipErrorInvalidValue;
    // chunks of a multiple of 4 elements (16-byte aligned starts when x is)
    int chunk = (n + AM_BLOCKS - 1) / AM_BLOCKS;
    chunk = (chunk + 3) & ~3;
    const int nblocks = (n + chunk - 1) / chunk;
    hipLaunchKernelGGL(argmax_part_kernel, dim3(nblocks), dim3(AM_THREADS), 0, st, x, n, chunk);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(64), 0, st, out, nblocks);
    return hipGetLastError();
}

}  // namespace jllm_hip
