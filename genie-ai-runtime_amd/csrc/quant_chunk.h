// quant_chunk.h -- the MMQ activation quantiser's per-lane step, shared by
// the quantiser kernels and the kernels that quantise their own output
// (the prefill attention's epilogue, the fused RMSNorm rows).  The
// reference's activation quantiser (quantize_mmq_q8_1_ds4 / _d4,
// mmq_q4k_llama.cu:383-404): d = absmax / 127, q = rint(v / d), the block
// sum in butterfly order.
#pragma once
#include "kq_common.h"

namespace jllm_hip {

typedef uint32_t qc_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t qc_u32x4 __attribute__((ext_vector_type(4)));

// The quantisation of one lane's 8 values v: sub-chunk `sub` (0..3, the
// lane's index within its aligned group of 4 lanes) of 32-value block kb32
// of token col.  All 4 lanes of the group call it together.
template <bool I8>
__device__ __forceinline__ void quant_chunk(const float (&v)[8], int sub, int kb32, int col, int Npad, void* codes,
                                            uint32_t* scl, bool ds4) {
    float amax = 0.0f, t[8];
#pragma unroll
    for (int e = 0; e < 8; e++) { amax = fmaxf(amax, fabsf(v[e])); t[e] = v[e]; }
    // lane ^ 1 and lane ^ 2 within the block's 4 lanes through DPP quad
    // permutes (the same partner values and add order as the shuffles)
    amax = fmaxf(amax, dpp_mov_f<0xB1>(amax));
    amax = fmaxf(amax, dpp_mov_f<0x4E>(amax));
#pragma unroll
    for (int e = 0; e < 8; e++) t[e] += dpp_mov_f<0x4E>(t[e]);       // index bit 4 (lane ^ 2)
#pragma unroll
    for (int e = 0; e < 8; e++) t[e] += dpp_mov_f<0xB1>(t[e]);       // index bit 3 (lane ^ 1)
    const float s2[4] = {t[0] + t[4], t[1] + t[5], t[2] + t[6], t[3] + t[7]};
    const float s1[2] = {s2[0] + s2[2], s2[1] + s2[3]};
    const float sum = s1[0] + s1[1];
    const float d = amax / 127.0f;
    const float dinv = d > 0.0f ? 1.0f / d : 0.0f;
    const int64_t at = ((int64_t)(kb32 >> 3) * Npad + col) * 256 + (kb32 & 7) * 32 + 8 * sub;
    if (I8) {
        uint32_t o[2] = {0u, 0u};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int q = (int)__builtin_rintf(v[e] * dinv);
            o[e >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (e & 3));
        }
        *(qc_u32x2*)((uint8_t*)codes + at) = qc_u32x2{o[0], o[1]};
    } else {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int q0 = (int)__builtin_rintf(v[2 * e] * dinv), q1 = (int)__builtin_rintf(v[2 * e + 1] * dinv);
            o[e] = (uint32_t)f32_to_f16_bits((float)q0) | ((uint32_t)f32_to_f16_bits((float)q1) << 16);
        }
        *(qc_u32x4*)((uint16_t*)codes + at) = qc_u32x4{o[0], o[1], o[2], o[3]};
    }
    if (sub == 0)
        scl[(int64_t)kb32 * Npad + col] =
            ds4 ? ((uint32_t)f32_to_f16_bits(d) | ((uint32_t)f32_to_f16_bits(sum) << 16)) : __builtin_bit_cast(uint32_t, d);
}

}  // namespace jllm_hip
