// kq_common.h -- block formats and small device helpers shared by the
// gfx950 kernels (GEMV, MMQ, attention).  wave64 only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jllm_hip {

constexpr int QK_K = 256;
constexpr int Q4K_BYTES = 144;   // u16 d, u16 dmin, u8 scales[12], u8 qs[128]
constexpr int Q6K_BYTES = 210;   // u8 ql[128], u8 qh[64], i8 scales[16], u16 d
constexpr int Q5K_BYTES = 176;   // u16 d, u16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]
constexpr int TYPE_Q4_K = 12;
constexpr int TYPE_Q5_K = 13;
constexpr int TYPE_Q6_K = 14;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);   // v_cvt_f16_f32, RNE
}
__device__ __forceinline__ float round_to_f16(float f) {
    return (float)(_Float16)f;
}
// silu(g) * u in fp32 as the reference's swiglu_kernel evaluates it
// (convert.cu:85-112), no contraction
__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
    return g / (1.0f + expf(-g)) * u;
}
__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t h2_bits(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// byte i (0..11) of the Q4_K scales[12], given as three little-endian words
__device__ __forceinline__ uint32_t sc_byte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (w >> (8 * (i & 3))) & 0xFFu;
}

// 6-bit (scale, min) of sub-block j of a Q4_K super-block (the packing of
// get_scale_min_k4, gemv_q4.cu:185-195).
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                              uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = sc_byte(s0, s1, s2, j) & 63u;
        m  = sc_byte(s0, s1, s2, j + 4) & 63u;
    } else {
        const uint32_t b = sc_byte(s0, s1, s2, j + 4);
        sc = (b & 0xFu) | ((sc_byte(s0, s1, s2, j - 4) >> 6) << 4);
        m  = (b >> 4)   | ((sc_byte(s0, s1, s2, j) >> 6) << 4);
    }
}

// 8 bytes starting at a 2-byte-aligned address, from three aligned dword
// loads.  Reads [floor4(p), floor4(p)+12) which lies inside [p-2, p+10).
__device__ __forceinline__ uint2 load8_a2(const uint8_t* p) {
    const uintptr_t a = (uintptr_t)p;
    const uint32_t* w = (const uint32_t*)(a & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(a & 3) * 8u;
    const uint32_t w0 = __builtin_nontemporal_load(w + 0);
    const uint32_t w1 = __builtin_nontemporal_load(w + 1);
    const uint32_t w2 = __builtin_nontemporal_load(w + 2);
    uint2 r;
    r.x = __builtin_amdgcn_alignbit(w1, w0, sh);
    r.y = __builtin_amdgcn_alignbit(w2, w1, sh);
    return r;
}

// per-byte (v - 32) for bytes v in [0, 63] without cross-byte borrows
__device__ __forceinline__ uint32_t sub32_bytes(uint32_t v) {
    return ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// swap with the neighbouring lane (lane ^ 1) through DPP quad_perm [1,0,3,2]
__device__ __forceinline__ int swap_lane1(int v) {
    return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
}

// Wave64 reductions that stay out of the LDS pipe (a butterfly of
// __shfl_xor is six dependent ds_bpermute round trips): four DPP steps
// (lane ^ 1, lane ^ 2, then the mirrors within 8 and within 16 lanes)
// leave each 16-lane row's result in all its lanes; the four row results
// are read out and combined in a fixed order, so every lane returns the
// same value.  All 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov_f<0xB1>(v);     // quad_perm [1,0,3,2]
    v += dpp_mov_f<0x4E>(v);     // quad_perm [2,3,0,1]
    v += dpp_mov_f<0x141>(v);    // row_half_mirror
    v += dpp_mov_f<0x140>(v);    // row_mirror
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov_f<0xB1>(v));
    v = fmaxf(v, dpp_mov_f<0x4E>(v));
    v = fmaxf(v, dpp_mov_f<0x141>(v));
    v = fmaxf(v, dpp_mov_f<0x140>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// The values of lanes l & 31 and (l & 31) + 32 -- lane l and lane l ^ 32 --
// in every lane, lower half's first (one v_permlane32_swap, no LDS pipe);
// a commutative op of the two equals op(v, __shfl_xor(v, 32)) bit for bit.
__device__ __forceinline__ void wave_halves(float v, float& lo, float& hi) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto s = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    lo = __builtin_bit_cast(float, (unsigned)s[0]);
    hi = __builtin_bit_cast(float, (unsigned)s[1]);
}

template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

}  // namespace jllm_hip
