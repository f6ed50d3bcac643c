// qk_front.h -- the per-head step of the attention front (the fused q/k-post
// kernel): one wave, one head;
// lane i < head_dim/2 holds the rotary pair (i, i + hd/2) (neox) or (2i,
// 2i+1).  Optional RMSNorm (one wave reduction), rounding to fp16 (the
// rmsnorm output), RoPE, rounding to fp16 (the rope output) -- the
// arithmetic of fused_rmsnorm_residual_kernel (fused_norm.cu:33-101) and
// rope_kernel (rope.cu:322-367) in the order the engine runs them
// (decode.cu:1441-1478).
#pragma once
#include "kq_common.h"
#include "layer_ops.h"

namespace jllm_hip {

__device__ __forceinline__ float front_wave_sum(float v) { return wave_sum(v); }
__device__ __forceinline__ float front_wave_max(float v) { return wave_max(v); }

__device__ __forceinline__ void front_rotate(float v0, float v1, float c, float s, float& r0, float& r1) {
#pragma clang fp contract(off)
    r0 = round_to_f16(v0 * c - v1 * s);
    r1 = round_to_f16(v0 * s + v1 * c);
}

// The pieces of front_pair: the pair's indices, its raw values, the norm
// weights, and the norm + rotation of loaded values.
__device__ __forceinline__ void front_idx(int hd, bool neox, int lane, int& i0, int& i1) {
    const int h2 = hd / 2;
    i0 = neox ? lane : 2 * lane;
    i1 = neox ? lane + h2 : 2 * lane + 1;
}
__device__ __forceinline__ void front_load(const uint16_t* src, bool act, int i0, int i1, float& v0, float& v1) {
    v0 = act ? f16_bits_to_f32(src[i0]) : 0.0f;
    v1 = act ? f16_bits_to_f32(src[i1]) : 0.0f;
}
__device__ __forceinline__ void front_weights(const void* norm, bool norm_fp32, bool act, int i0, int i1, float& w0,
                                              float& w1) {
    w0 = 0.0f; w1 = 0.0f;
    if (norm && act) {
        if (norm_fp32) { w0 = ((const float*)norm)[i0]; w1 = ((const float*)norm)[i1]; }
        else { w0 = f16_bits_to_f32(((const uint16_t*)norm)[i0]); w1 = f16_bits_to_f32(((const uint16_t*)norm)[i1]); }
    }
}
__device__ __forceinline__ void front_apply(bool norm, float w0, float w1, int hd, float eps, bool rot, float c,
                                            float s, float& v0, float& v1) {
#pragma clang fp contract(off)
    if (norm) {
        const float ss = front_wave_sum(v0 * v0 + v1 * v1);
        const float rrms = 1.0f / sqrtf(ss / (float)hd + eps);
        v0 = round_to_f16(v0 * rrms * w0);
        v1 = round_to_f16(v1 * rrms * w1);
    }
    if (rot) front_rotate(v0, v1, c, s, v0, v1);
}

// The lane's pair of one head row src [hd]: loads, normalises (norm != null:
// weights fp32 or fp16) and, when rot, rotates by (c, s).  i0/i1 are the
// pair's element indices; lanes >= hd/2 return zeros.
__device__ __forceinline__ void front_pair(const uint16_t* src, int hd, bool neox, const void* norm, bool norm_fp32,
                                           float eps, bool rot, float c, float s, int lane, float& v0, float& v1,
                                           int& i0, int& i1) {
    const bool act = lane < hd / 2;
    front_idx(hd, neox, lane, i0, i1);
    front_load(src, act, i0, i1, v0, v1);
    float w0, w1;
    front_weights(norm, norm_fp32, act, i0, i1, w0, w1);
    front_apply(norm != nullptr, w0, w1, hd, eps, rot, c, s, v0, v1);
}

// Store the lane's pair into a KV-cache row: int8 with the row's absmax
// scale (fp16_to_int8_kernel, convert.cu:26-69; scale to *sc when sc is
// not null) or fp16 copies.
__device__ __forceinline__ void front_store_kv(void* row, float* sc, bool kv_int8, int hd, float v0, float v1, int i0,
                                               int i1, int lane) {
    const bool act = lane < hd / 2;
    if (kv_int8) {
        const float mx = front_wave_max(fmaxf(fabsf(v0), fabsf(v1)));
        const float scale = mx / 127.0f;
        const float inv = scale > 0.0f ? 127.0f / mx : 0.0f;
        if (act) {
            int q0 = (int)__builtin_rintf(v0 * inv), q1 = (int)__builtin_rintf(v1 * inv);
            q0 = q0 > 127 ? 127 : (q0 < -127 ? -127 : q0);
            q1 = q1 > 127 ? 127 : (q1 < -127 ? -127 : q1);
            ((int8_t*)row)[i0] = (int8_t)q0;
            ((int8_t*)row)[i1] = (int8_t)q1;
        }
        if (lane == 0 && sc) *sc = scale;
    } else if (act) {
        ((uint16_t*)row)[i0] = f32_to_f16_bits(v0);
        ((uint16_t*)row)[i1] = f32_to_f16_bits(v1);
    }
}

// The rest of the attention-front step of one (token t, head) of kind 0 /
// 1 / 2 (q / k / v) once the lane's raw pair values v0, v1 and norm weights
// w0, w1 are in registers: q and k normalised and rotated (position pos,
// frequency fq) and written back as fp16 into a.q / a.k (row strides qs /
// ks), k and v stored into the KV cache at row r0 + t.
__device__ __forceinline__ void front_finish(const QKPostArgs& a, int kind, int head, int t, int64_t r0, int pos,
                                             int l, bool act, int i0, int i1, float v0, float v1, float w0,
                                             float w1, float fq, int64_t qs, int64_t ks) {
    const int hd = a.head_dim;
    const void* norm = kind < 2 ? (kind == 0 ? a.q_norm : a.k_norm) : nullptr;
    float s = 0.0f, c = 1.0f;
    if (kind < 2) sincosf((float)pos * fq, &s, &c);
    front_apply(norm != nullptr, w0, w1, hd, a.eps, kind < 2, c, s, v0, v1);
    if (kind < 2 && act) {
        uint16_t* dq = kind == 0 ? a.q + t * qs + (int64_t)head * hd : a.k + t * ks + (int64_t)head * hd;
        dq[i0] = f32_to_f16_bits(v0);
        dq[i1] = f32_to_f16_bits(v1);
    }
    if (kind == 0) return;
    const int64_t row = (r0 + t) * a.kv_stride + (int64_t)head * a.cache_head_dim;
    void* cache = kind == 1 ? a.k_dst : a.v_dst;
    float* sc = kind == 1 ? a.k_scales : a.v_scales;
    front_store_kv(a.kv_int8 ? (void*)((int8_t*)cache + row) : (void*)((uint16_t*)cache + row),
                   sc ? sc + (r0 + t) * a.n_kv + head : nullptr, a.kv_int8 != 0, hd, v0, v1, i0, i1, l);
}

}  // namespace jllm_hip
