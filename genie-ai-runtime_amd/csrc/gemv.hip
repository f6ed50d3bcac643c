// gemv.hip -- Q4_K / Q5_K / Q6_K decode GEMV for gfx950 (wave64).
//
// Two arithmetic modes, matching the reference dispatcher's defaults
// (gemv_q4.cu:1245-1616):
//   * MMVQ: the fp16 activation is quantised to q8_1 (32-value blocks,
//     gemv_q4.cu:445-466) and dotted as int8 (v_dot4_i32_i8) against the
//     weight codes, one exact int32 per 32-weight Q4_K sub-block or per
//     16-weight Q6_K group, then scaled in fp32 (gemv_q4.cu:474-618).
//   * float dequant: weights dequantised in registers and dotted with the
//     fp16 activation in fp32 (gemv_q4.cu:266-398).  The only mode of Q5_K,
//     as in the reference (gemv_q4.cu:318-363).
//
// Layout of the work (streaming kernel below): the rows of a launch are
// split between waves; each wave streams its rows' bytes (contiguous in
// memory) in rounds of 4 KiB -- every lane loads 16-byte chunks, so a wave's
// load instruction covers 1 KiB of consecutive bytes -- through registers
// into its own LDS buffer, from which one quad of lanes per super-block does
// the arithmetic.  The activation is staged once per workgroup in LDS (for
// MMVQ quantised there, so no q8_1 buffer and no extra launch).
#include "kq_common.h"
#include "gemv.h"
#include <algorithm>

// Native clang vector types (not HIP's struct-based uint4 & co.), so that
// values in them stay in registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 u32x4_make(uint32_t a, uint32_t b, uint32_t c, uint32_t d) { return u32x4{a, b, c, d}; }
__device__ __forceinline__ u32x2 u32x2_make(uint32_t a, uint32_t b) { return u32x2{a, b}; }

namespace jllm_hip {

constexpr int GEMV_THREADS = 256;

// ---- activation staging -------------------------------------------------

// Quantise 32 fp16 values to q8_1 with 8 cooperating lanes (4 values each):
// d = amax/127, q = rn(v*(1/d)) clamped to +-127, s = d*sum(q)  (the
// arithmetic of quantize_q8_1_kernel, gemv_q4.cu:445-466).  Returns the 4
// packed codes; d and the partial sums via the out-parameters.
__device__ __forceinline__ uint32_t quant_q8_1_x4(u32x2 raw, float& d_out, int& sumq_all, int& sumq_half) {
    float v[4];
    v[0] = f16_bits_to_f32(raw.x & 0xFFFFu); v[1] = f16_bits_to_f32(raw.x >> 16);
    v[2] = f16_bits_to_f32(raw.y & 0xFFFFu); v[3] = f16_bits_to_f32(raw.y >> 16);
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint32_t packed = 0;
    int sumq = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int q = (int)__builtin_rintf(v[i] * id);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        sumq += q;
        packed |= ((uint32_t)q & 0xFFu) << (8 * i);
    }
    sumq += __shfl_xor(sumq, 1, 64);
    sumq += __shfl_xor(sumq, 2, 64);
    sumq_half = sumq;                          // sum over this lane's 16-value half
    sumq += __shfl_xor(sumq, 4, 64);
    sumq_all = sumq;
    d_out = d;
    return packed;
}

// Index of the 16-value group n (natural order) in the Q6_K lane order
// [block][half h][l-half][quarter g], so that a lane reads its four groups
// with one 16-byte LDS load.
__device__ __forceinline__ int q6_group_slot(int n) {
    const int b = n >> 4, r = n & 15;
    const int h = r >> 3, g = (r & 7) >> 1, lh = r & 1;
    return b * 16 + h * 8 + lh * 4 + g;
}

// x index -> LDS half index: 8 halves of padding after every 128, so that the
// quads' reads 256 B apart land in different banks.
//
// Staged activation in LDS (gemv_lds_bytes):
//   MMVQ : q8 codes i8 [K] | d8 f32 [K/32] | s8 f32 [K/32] (both rounded
//          through fp16 like the block_q8_1 fields) | per-16 code sums i32
//          [K/16] in Q6_K lane order (q6_group_slot)
//   float: x f16 [K + K/16] (xpad) | per-32 sums f32 [K/32] | 32 * per-16
//          sums f32 [K/16] in Q6_K lane order
__device__ __forceinline__ int xpad(int k) { return k + ((k >> 7) << 3); }

// ---- block slices ------------------------------------------------------------

// Quad lane layout: 4 lanes per super-block; lane q (0..3) owns 64 weights.
//   Q4_K: qs bytes [32q, 32q+32): low nibbles = sub-block 2q, high = 2q+1.
//   Q6_K: half h = q/2 of the block, positions l0..l0+15 (l0 = 16*(q&1)) of
//         each 32-wide quarter g = 0..3: elements h*128 + 32g + l0 + [0,16).
//   Q5_K: as Q4_K (qs bytes [32q, 32q+32)), plus all 32 qh bytes, of which
//         the lane uses bits 2q (low nibbles) and 2q+1 (high nibbles).
// One register layout for all types (Q4_K / Q5_K use a = header, b/c = qs,
// Q5_K h0/h1 = qh).
// Q6_K blocks are only 2-byte aligned: their pieces are read dword-aligned
// from up to 2 bytes early (sh = 16 when so) and realigned with a funnel
// shift.
struct Raw { u32x4 a, b, c; uint32_t a4, b4, c4; u32x2 sc; uint32_t sc2, d, sh; u32x4 h0, h1; };
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ u32x4 realign16(const u32x4& v, uint32_t w4, uint32_t sh) {
    return u32x4_make(__builtin_amdgcn_alignbit(v.y, v.x, sh), __builtin_amdgcn_alignbit(v.z, v.y, sh),
                      __builtin_amdgcn_alignbit(v.w, v.z, sh), __builtin_amdgcn_alignbit(w4, v.w, sh));
}

// ---- per-lane constants ------------------------------------------------------

// Q4_K: bit positions of the 6-bit (scale, min) of sub-blocks 2q and 2q+1
// (the packing of get_scale_min_k4, gemv_q4.cu:185-195).  For sub-block j < 4
// both fields are the low 6 bits of scales[j] / scales[j+4]; for j >= 4 the
// low 4 bits come from scales[j+4] (low / high nibble) and the top 2 bits
// from bits 6-7 of scales[j-4] / scales[j].
struct Q4Consts {
    bool hi;               // sub-blocks 4..7
    uint32_t w_lo, w_hi;   // field widths of the low / high part (6,0) or (4,2)
    uint32_t o_sc0, o_m0, o_top0;   // bit offsets for sub-block 2q
};

__device__ __forceinline__ Q4Consts q4_consts(int q) {
    Q4Consts c;
    c.hi = q >= 2;
    c.w_lo = c.hi ? 4u : 6u;
    c.w_hi = c.hi ? 2u : 0u;
    const int jj = c.hi ? 2 * q - 4 : 2 * q;
    c.o_sc0 = 8u * jj;
    c.o_m0 = 8u * jj + (c.hi ? 4u : 0u);
    c.o_top0 = 8u * jj + 6u;
    return c;
}

// (scale, min) of sub-block 2q + t; the fields of sub-block 2q+1 sit 8 bits
// above those of 2q.
__device__ __forceinline__ void q4_scales(const Q4Consts& c, const u32x4& hdr, int t, uint32_t& sc, uint32_t& m) {
    const uint32_t a_sc = c.hi ? hdr.w : hdr.y;   // scales[8..11] : scales[0..3]
    const uint32_t a_m = c.hi ? hdr.w : hdr.z;    // scales[8..11] : scales[4..7]
    const uint32_t d = 8u * (uint32_t)t;
    sc = __builtin_amdgcn_ubfe(a_sc, c.o_sc0 + d, c.w_lo) | (__builtin_amdgcn_ubfe(hdr.y, c.o_top0 + d, c.w_hi) << 4);
    m  = __builtin_amdgcn_ubfe(a_m,  c.o_m0 + d,  c.w_lo) | (__builtin_amdgcn_ubfe(hdr.z, c.o_top0 + d, c.w_hi) << 4);
}

// Q6_K lane slice with the pieces realigned (see Raw)
__device__ __forceinline__ Raw q6_realign(const Raw& r) {
    Raw o = r;
    o.a = realign16(r.a, r.a4, r.sh);
    o.b = realign16(r.b, r.b4, r.sh);
    o.c = realign16(r.c, r.c4, r.sh);
    o.sc = u32x2_make(__builtin_amdgcn_alignbit(r.sc.y, r.sc.x, r.sh), __builtin_amdgcn_alignbit(r.sc2, r.sc.y, r.sh));
    return o;
}

// 6-bit codes (bytes 0..63) of quarter g of a realigned Q6_K lane slice, 4 words
__device__ __forceinline__ void q6_codes(const Raw& r, int g, uint32_t out[4]) {
    const uint32_t src[4] = {(g & 1) ? r.b.x : r.a.x, (g & 1) ? r.b.y : r.a.y,
                             (g & 1) ? r.b.z : r.a.z, (g & 1) ? r.b.w : r.a.w};
    const uint32_t hq[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t lo = g >= 2 ? (src[i] >> 4) : src[i];
        const uint32_t hb = g == 3 ? (hq[i] >> 2) : (hq[i] << (4 - 2 * g));
        out[i] = (lo & 0x0F0F0F0Fu) | (hb & 0x30303030u);
    }
}

__device__ __forceinline__ float q6_scale_f(const Raw& r, int q, int g) {
    const int idx = (q & 1) + 2 * g;                       // 0..7 within scales[8h..8h+8)
    const uint32_t w = idx < 4 ? r.sc.x : r.sc.y;
    return (float)(int)(int8_t)(uint8_t)(w >> (8 * (idx & 3)));
}

// ---- per-block lane arithmetic -----------------------------------------------

// MMVQ Q4_K: two exact int32 sub-block dots (the 32-weight dots of
// dot_q4k_row_q8_1), combined as dall*sum_j(sc_j*dot_j*d8_j) - dmin*sum_j(m_j*s8_j).
template <int TYPE> __device__ float mmvq_block(const Raw& r, int b, int q, const Q4Consts& c, const uint8_t* lds, int K);

template <>
__device__ __forceinline__ float mmvq_block<TYPE_Q4_K>(const Raw& r, int b, int q, const Q4Consts& c, const uint8_t* lds, int K) {
    const int8_t* s_q = (const int8_t*)lds;
    const float* s_d8 = (const float*)(lds + K);
    const float* s_s8 = s_d8 + K / 32;
    const int sb = b * 8 + 2 * q;
    const u32x4 x0 = *(const u32x4*)(s_q + sb * 32), x1 = *(const u32x4*)(s_q + sb * 32 + 16);
    const u32x4 y0 = *(const u32x4*)(s_q + sb * 32 + 32), y1 = *(const u32x4*)(s_q + sb * 32 + 48);
    const f32x2 d8 = *(const f32x2*)(s_d8 + sb), s8 = *(const f32x2*)(s_s8 + sb);
    const uint32_t M = 0x0F0F0F0Fu;
    const uint32_t w[8] = {r.b.x, r.b.y, r.b.z, r.b.w, r.c.x, r.c.y, r.c.z, r.c.w};
    const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const uint32_t xh[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
    int dl = 0, dh = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        dl = sdot4(w[i] & M, xl[i], dl);
        dh = sdot4((w[i] >> 4) & M, xh[i], dh);
    }
    uint32_t sc0, m0, sc1, m1;
    q4_scales(c, r.a, 0, sc0, m0);
    q4_scales(c, r.a, 1, sc1, m1);
    // |dot| <= 32*15*127 and sc <= 63: the products fit the full-rate 24-bit multiply exactly
    const float a = (float)__mul24(dl, (int)sc0) * d8.x + (float)__mul24(dh, (int)sc1) * d8.y;
    const float mm = (float)m0 * s8.x + (float)m1 * s8.y;
    const float dall = f16_bits_to_f32(r.a.x & 0xFFFFu), dmin = f16_bits_to_f32(r.a.x >> 16);
    return dall * a - dmin * mm;
}

// MMVQ Q6_K: per 16-weight group an exact int32 dot of the raw 6-bit codes,
// minus 32*sum(q8) (so the offset of 32 is applied exactly in int), times the
// int8 scale; then d8 and d in fp32.
template <>
__device__ __forceinline__ float mmvq_block<TYPE_Q6_K>(const Raw& raw, int b, int q, const Q4Consts&, const uint8_t* lds, int K) {
    const Raw r = q6_realign(raw);
    const int8_t* s_q = (const int8_t*)lds;
    const float* s_d8 = (const float*)(lds + K);
    const int* s_sx = (const int*)(s_d8 + 2 * (K / 32));
    const int h = q >> 1, l0 = 16 * (q & 1);
    const f32x4 d8 = *(const f32x4*)(s_d8 + b * 8 + 4 * h);
    const i32x4 sx = *(const i32x4*)(s_sx + b * 16 + h * 8 + (q & 1) * 4);
    const float d8v[4] = {d8.x, d8.y, d8.z, d8.w};
    const int sxv[4] = {sx.x, sx.y, sx.z, sx.w};
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        uint32_t cw[4];
        q6_codes(r, g, cw);
        const u32x4 xv = *(const u32x4*)(s_q + b * 256 + h * 128 + 32 * g + l0);
        int dot = sdot4(cw[0], xv.x, 0);
        dot = sdot4(cw[1], xv.y, dot); dot = sdot4(cw[2], xv.z, dot); dot = sdot4(cw[3], xv.w, dot);
        dot -= 32 * sxv[g];
        acc += (float)dot * q6_scale_f(r, q, g) * d8v[g];
    }
    return f16_bits_to_f32(r.d) * acc;
}

// fp16 code pairs as subnormal halves: byte pair (b0, b1) of w -> halves
// with bit patterns b0 and b1, i.e. values b*2^-24 (exact).
__device__ __forceinline__ uint32_t pair01(uint32_t w) { return __builtin_amdgcn_perm(w, w, 0x0C010C00u); }
__device__ __forceinline__ uint32_t pair23(uint32_t w) { return __builtin_amdgcn_perm(w, w, 0x0C030C02u); }

// float dequant Q4_K: sum_j (dall*sc_j*q - dmin*m_j) * x over the lane's two
// sub-blocks, evaluated as dall*sc_j*sum(q*x) - dmin*m_j*sum(x) with sum(q*x)
// from fp16 dot products of the codes (as subnormal halves) with x.
template <int TYPE> __device__ float f16_block(const Raw& r, int b, int q, const Q4Consts& c, const uint8_t* lds, int K);

template <>
__device__ __forceinline__ float f16_block<TYPE_Q4_K>(const Raw& r, int b, int q, const Q4Consts& c, const uint8_t* lds, int K) {
    const uint16_t* s_x = (const uint16_t*)lds;
    const float* s_x32 = (const float*)(lds + 2 * K + K / 8);
    const int k0 = xpad(b * 256 + 64 * q);
    const uint32_t w[8] = {r.b.x, r.b.y, r.b.z, r.b.w, r.c.x, r.c.y, r.c.z, r.c.w};
    float sl = 0.0f, sh = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const u32x4 xa = *(const u32x4*)(s_x + k0 + 4 * i);        // x[k0+4i .. +8)
        const u32x4 xb = *(const u32x4*)(s_x + k0 + 32 + 4 * i);   // high-nibble partners
        const uint32_t p0 = pair01(w[i]), p1 = pair23(w[i]), p2 = pair01(w[i + 1]), p3 = pair23(w[i + 1]);
        sl = fdot2(p0 & 0x000F000Fu, xa.x, sl); sl = fdot2(p1 & 0x000F000Fu, xa.y, sl);
        sl = fdot2(p2 & 0x000F000Fu, xa.z, sl); sl = fdot2(p3 & 0x000F000Fu, xa.w, sl);
        sh = fdot2(p0 & 0x00F000F0u, xb.x, sh); sh = fdot2(p1 & 0x00F000F0u, xb.y, sh);
        sh = fdot2(p2 & 0x00F000F0u, xb.z, sh); sh = fdot2(p3 & 0x00F000F0u, xb.w, sh);
    }
    uint32_t sc0, m0, sc1, m1;
    q4_scales(c, r.a, 0, sc0, m0);
    q4_scales(c, r.a, 1, sc1, m1);
    const f32x2 xs = *(const f32x2*)(s_x32 + b * 8 + 2 * q);
    const float dall = f16_bits_to_f32(r.a.x & 0xFFFFu), dmin = f16_bits_to_f32(r.a.x >> 16);
    const float a = (float)sc0 * (sl * 16777216.0f) + (float)sc1 * (sh * 1048576.0f);
    const float mm = (float)m0 * xs.x + (float)m1 * xs.y;
    return dall * a - dmin * mm;
}

// float dequant Q5_K: as Q4_K with 5-bit codes (nibble | qh bit << 4) built
// as bytes, then dotted with x as subnormal halves.
template <>
__device__ __forceinline__ float f16_block<TYPE_Q5_K>(const Raw& r, int b, int q, const Q4Consts& c, const uint8_t* lds, int K) {
    const uint16_t* s_x = (const uint16_t*)lds;
    const float* s_x32 = (const float*)(lds + 2 * K + K / 8);
    const int k0 = xpad(b * 256 + 64 * q);
    const uint32_t w[8] = {r.b.x, r.b.y, r.b.z, r.b.w, r.c.x, r.c.y, r.c.z, r.c.w};
    const uint32_t hq[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
    const uint32_t s0 = 2u * (uint32_t)q;
    float sl = 0.0f, sh = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const u32x4 xa = *(const u32x4*)(s_x + k0 + 4 * i);        // x[k0+4i .. +8)
        const u32x4 xb = *(const u32x4*)(s_x + k0 + 32 + 4 * i);   // high-nibble partners
        const uint32_t lo0 = (w[i] & 0x0F0F0F0Fu) | (((hq[i] >> s0) & 0x01010101u) << 4);
        const uint32_t lo1 = (w[i + 1] & 0x0F0F0F0Fu) | (((hq[i + 1] >> s0) & 0x01010101u) << 4);
        const uint32_t hi0 = ((w[i] >> 4) & 0x0F0F0F0Fu) | (((hq[i] >> (s0 + 1)) & 0x01010101u) << 4);
        const uint32_t hi1 = ((w[i + 1] >> 4) & 0x0F0F0F0Fu) | (((hq[i + 1] >> (s0 + 1)) & 0x01010101u) << 4);
        sl = fdot2(pair01(lo0), xa.x, sl); sl = fdot2(pair23(lo0), xa.y, sl);
        sl = fdot2(pair01(lo1), xa.z, sl); sl = fdot2(pair23(lo1), xa.w, sl);
        sh = fdot2(pair01(hi0), xb.x, sh); sh = fdot2(pair23(hi0), xb.y, sh);
        sh = fdot2(pair01(hi1), xb.z, sh); sh = fdot2(pair23(hi1), xb.w, sh);
    }
    uint32_t sc0, m0, sc1, m1;
    q4_scales(c, r.a, 0, sc0, m0);
    q4_scales(c, r.a, 1, sc1, m1);
    const f32x2 xs = *(const f32x2*)(s_x32 + b * 8 + 2 * q);
    const float dall = f16_bits_to_f32(r.a.x & 0xFFFFu), dmin = f16_bits_to_f32(r.a.x >> 16);
    const float a = ((float)sc0 * sl + (float)sc1 * sh) * 16777216.0f;
    const float mm = (float)m0 * xs.x + (float)m1 * xs.y;
    return dall * a - dmin * mm;
}

// float dequant Q6_K: per 16-weight group sum((code-32)*x) = sum(code*x) - 32*sum(x)
// with sum(code*x) from fp16 dot products of the codes as subnormal halves.
template <>
__device__ __forceinline__ float f16_block<TYPE_Q6_K>(const Raw& raw, int b, int q, const Q4Consts&, const uint8_t* lds, int K) {
    const Raw r = q6_realign(raw);
    const uint16_t* s_x = (const uint16_t*)lds;
    const float* s_x16 = (const float*)(lds + 2 * K + K / 8) + K / 32;
    const int h = q >> 1, l0 = 16 * (q & 1);
    const f32x4 xs = *(const f32x4*)(s_x16 + b * 16 + h * 8 + (q & 1) * 4);
    const float xsv[4] = {xs.x, xs.y, xs.z, xs.w};
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        uint32_t cw[4];
        q6_codes(r, g, cw);
        const uint16_t* xp = s_x + xpad(b * 256 + h * 128) + 32 * g + l0;
        const u32x4 xa = *(const u32x4*)xp, xb = *(const u32x4*)(xp + 8);
        float s = fdot2(pair01(cw[0]), xa.x, 0.0f);
        s = fdot2(pair23(cw[0]), xa.y, s); s = fdot2(pair01(cw[1]), xa.z, s); s = fdot2(pair23(cw[1]), xa.w, s);
        s = fdot2(pair01(cw[2]), xb.x, s); s = fdot2(pair23(cw[2]), xb.y, s);
        s = fdot2(pair01(cw[3]), xb.z, s); s = fdot2(pair23(cw[3]), xb.w, s);
        acc += (s * 16777216.0f - xsv[g]) * q6_scale_f(r, q, g);
    }
    return f16_bits_to_f32(r.d) * acc;
}

// Row result: fp32, fp16, or fp16 of fp16(W x) + residual (the residual row
// staged in LDS).
template <int OUT>
__device__ __forceinline__ void store_row(const GemvSeg& s, int r, float acc, const uint16_t* res_lds, int lrow) {
    if (OUT == OUT_F32) {
        ((float*)s.y)[r] = acc;
    } else if (OUT == OUT_HALF) {
        ((uint16_t*)s.y)[r] = f32_to_f16_bits(acc);
    } else {   // y = half(half(W x) + residual), gemv_q4.cu:1001-1004
        const float proj = round_to_f16(acc);
        ((uint16_t*)s.y)[r] = f32_to_f16_bits(proj + f16_bits_to_f32(res_lds[lrow]));
    }
}

template <bool MMVQ, int TYPE>
__device__ __forceinline__ float block_dot(const Raw& r, int b, int q, const Q4Consts& c, const uint8_t* lds, int K) {
    static_assert(!(MMVQ && TYPE == TYPE_Q5_K), "Q5_K has no MMVQ mode");
    if constexpr (MMVQ) return mmvq_block<TYPE>(r, b, q, c, lds, K);
    else return f16_block<TYPE>(r, b, q, c, lds, K);
}

// ---- streaming kernel ----------------------------------------------------
//
// All segments of a launch share K, so their rows form one sequence of
// rows x nb blocks.  The waves of the grid (4 per workgroup, up to 4
// workgroups per CU) split the Q4_K rows and the Q6_K rows between them in
// proportion to bytes; a wave's rows are contiguous bytes per segment and are
// streamed in rounds of up to 4 KiB: each lane loads 4 aligned 16-byte chunks
// (buffer loads: chunks past the round's end are not fetched), two rounds
// ahead of the one being computed, and the wave moves a round into its own
// LDS buffer -- no workgroup barrier in the loop.  A round is computed with
// one quad per block (the per-block arithmetic above, reading the block from
// LDS); the quad's sum lands in the block's slot, and at the end each row
// adds its nb slots in block order and is stored.  The activation and the
// residual rows are loaded before any weight bytes, behind a barrier, so
// that they do not queue behind the CU's weight traffic.

// threads per workgroup: 256, or 512 for a launch under 12 MB (one
// workgroup of 8 waves per CU stages the activation once per CU: QKV triple
// 6.05 -> 5.7 us, with RMSNorm 6.85 -> 6.5 us)
constexpr int ST_T = 256;
constexpr int ST_T_SMALL = 512;

// lane ^ 1 and lane ^ 2 through DPP quad_perm (no LDS round trip)
__device__ __forceinline__ int dpp_x1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int dpp_x2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ float dpp_x1(float v) { return __builtin_bit_cast(float, dpp_x1(__builtin_bit_cast(int, v))); }
__device__ __forceinline__ float dpp_x2(float v) { return __builtin_bit_cast(float, dpp_x2(__builtin_bit_cast(int, v))); }

// q8_1 of one 8-value chunk c of x (4 lanes per 32-value block): d = amax/127,
// q = rn(v*(1/d)) clamped to +-127, s = d*sum(q) (quantize_q8_1_kernel,
// gemv_q4.cu:445-466), into the MMVQ staging layout.
__device__ __forceinline__ void xstage_q8_1(const u32x4& raw, int c, int K, uint8_t* lds) {
    int8_t* s_q = (int8_t*)lds;
    float* s_d8 = (float*)(lds + K);
    float* s_s8 = s_d8 + K / 32;
    int* s_sx = (int*)(s_s8 + K / 32);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; i++) { v[2 * i] = f16_bits_to_f32(w[i] & 0xFFFFu); v[2 * i + 1] = f16_bits_to_f32(w[i] >> 16); }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, dpp_x1(amax));
    amax = fmaxf(amax, dpp_x2(amax));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint32_t p0 = 0, p1 = 0;
    int sumq = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int q = (int)__builtin_rintf(v[i] * id);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        sumq += q;
        if (i < 4) p0 |= ((uint32_t)q & 0xFFu) << (8 * i);
        else       p1 |= ((uint32_t)q & 0xFFu) << (8 * (i - 4));
    }
    const int shalf = sumq + dpp_x1(sumq);
    const int sall = shalf + dpp_x2(shalf);
    if (c < K / 8) {
        *(u32x2*)(s_q + 8 * c) = u32x2_make(p0, p1);
        const int blk = c >> 2, sub = c & 3;
        if (sub == 0) {
            s_d8[blk] = round_to_f16(d);
            s_s8[blk] = round_to_f16(d * (float)sall);
        }
        if ((sub & 1) == 0) s_sx[q6_group_slot(blk * 2 + (sub >> 1))] = shalf;
    }
}

// fp16 copy and sums of one 8-value chunk, into the float staging layout.
__device__ __forceinline__ void xstage_f16(const u32x4& a, int c, int K, uint8_t* lds) {
    uint16_t* s_x = (uint16_t*)lds;
    float* s_x32 = (float*)(lds + 2 * K + K / 8);
    float* s_x16 = s_x32 + K / 32;
    const uint32_t one = 0x3C003C00u;
    float s = fdot2(a.x, one, 0.0f);
    s = fdot2(a.y, one, s); s = fdot2(a.z, one, s); s = fdot2(a.w, one, s);
    const float s16 = s + dpp_x1(s);
    const float s32 = s16 + dpp_x2(s16);
    if (c < K / 8) {
        *(u32x4*)(s_x + xpad(8 * c)) = a;
        if ((c & 1) == 0) s_x16[q6_group_slot(c >> 1)] = 32.0f * s16;
        if ((c & 3) == 0) s_x32[c >> 2] = s32;
    }
}

// Standalone q8_1 quantiser in the reference's AoS block layout
// (block_q8_1 {u16 d, u16 s, i8 qs[32]}, gemv_q4.cu:434-466).
__global__ __launch_bounds__(GEMV_THREADS)
void quantize_q8_1_aos_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ y, int K) {
    const int t = blockIdx.x * GEMV_THREADS + threadIdx.x;
    const int n = (K / 32) * 8;
    const bool live = t < n;
    const int blk = live ? t >> 3 : 0, sub = t & 7;
    const u32x2 raw = live ? *(const u32x2*)(x + blk * 32 + sub * 4) : u32x2_make(0, 0);
    float d; int sall, shalf;
    const uint32_t packed = quant_q8_1_x4(raw, d, sall, shalf);
    if (!live) return;
    uint8_t* out = y + (int64_t)blk * 36;
    *(uint32_t*)(out + 4 + 4 * sub) = packed;
    if (sub == 0) *(uint32_t*)out = (uint32_t)f32_to_f16_bits(d) | ((uint32_t)f32_to_f16_bits(d * (float)sall) << 16);
}

// ---- host launchers ----------------------------------------------------

size_t gemv_lds_bytes(bool mmvq, int K) {
    return mmvq ? (size_t)K + (size_t)(K / 32) * 8 + (size_t)(K / 16) * 4
                : (size_t)K * 2 + (size_t)(K / 8) + (size_t)(K / 32) * 4 + (size_t)(K / 16) * 4;
}

static int device_cus() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 256;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
        return n;
    }();
    return cus;
}

// The rows [r0, r1) (segment-relative) a wave owns inside one segment, its
// first slot and its rounds.
// The blocks [b0, b0 + nblk) of one segment (b0 counted from the segment's
// first block) that a wave streams, the workgroup slot of its first block
// and its number of rounds.
struct Piece { int b0, nblk, slot0, rounds; };

// A round: up to WGeom::NBLK blocks of one piece (contiguous bytes).
struct RoundDesc {
    const uint8_t* base;   // 16-byte-aligned start of the round's bytes
    int nrec;              // bytes to fetch (multiple of 16; 0 for no round)
    int delta;             // offset of the first block in the fetched bytes
    int nblk;              // blocks in the round
    int col0;              // block column of the first block
    int slot0;             // slot of the first block
};

template <int TYPE>
constexpr int block_bytes() { return TYPE == TYPE_Q4_K ? Q4K_BYTES : (TYPE == TYPE_Q5_K ? Q5K_BYTES : Q6K_BYTES); }

template <int TYPE, int L>
struct WGeom {
    static constexpr int BB = block_bytes<TYPE>();
    static constexpr int BYTES = 64 * 16 * L;                                  // one wave's round
    // Q4_K / Q5_K blocks are 16-byte multiples (rounds start aligned); a Q6_K
    // round may start up to 14 bytes into its first 16-byte chunk
    static constexpr int NFIT = TYPE == TYPE_Q6_K ? (BYTES - 14) / BB : BYTES / BB;
    // whole passes of the 16 quads: a round of 19 Q6_K blocks would leave 13
    // of 16 quads idle in its second pass (measured: lm_head 74 -> 61 us)
    static constexpr int NBLK = NFIT >= 16 ? NFIT / 16 * 16 : NFIT;
};

template <int TYPE, int L>
__device__ __forceinline__ RoundDesc round_desc(const StreamArgs& a, const Piece (&pc)[3], int k) {
    constexpr int BB = WGeom<TYPE, L>::BB, NB = WGeom<TYPE, L>::NBLK;
    const int nb = a.nb;
    RoundDesc d;
    d.base = a.seg[0].W; d.nrec = 0; d.delta = 0; d.nblk = 0; d.col0 = 0; d.slot0 = 0;
    int r = k;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        if (r >= 0 && r < pc[i].rounds) {
            const int f = r * NB;                                   // block offset in the piece
            d.nblk = min(NB, pc[i].nblk - f);
            const uint8_t* start = a.seg[i].W + ((int64_t)pc[i].b0 + f) * BB;
            d.delta = (int)((uintptr_t)start & 15u);
            d.base = start - d.delta;
            d.nrec = (d.delta + d.nblk * BB + 15) & ~15;
            d.col0 = (int)((uint32_t)(pc[i].b0 + f) % (uint32_t)nb);     // non-negative: unsigned division
            d.slot0 = pc[i].slot0 + f;
        }
        r -= pc[i].rounds;
    }
    return d;
}

#ifndef JLLM_GEMV_CPOL
#define JLLM_GEMV_CPOL 2   // nt: the weights are streamed once (measured 5 % faster than the default policy)
#endif
template <int L>
__device__ __forceinline__ void issue_round(const RoundDesc& d, u32x4 (&v)[L], int lane) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)d.base, (short)0, d.nrec, 0x00020000);
#pragma unroll
    for (int i = 0; i < L; i++) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane + 64 * i) * 16, 0, JLLM_GEMV_CPOL);
}

template <int L>
__device__ __forceinline__ void write_round(uint8_t* buf, const u32x4 (&v)[L], int lane) {
#pragma unroll
    for (int i = 0; i < L; i++) *(u32x4*)(buf + (lane + 64 * i) * 16) = v[i];
}

// Raw lane slice of the block at byte offset `off` of an LDS round buffer
// (16-byte aligned).  Same register layout as load_raw.
template <int TYPE>
__device__ __forceinline__ void load_raw_lds(const uint8_t* buf, int off, int q, Raw& r) {
    if (TYPE == TYPE_Q4_K) {
        const uint8_t* blk = buf + off;          // 16-byte aligned
        r.a = *(const u32x4*)blk;
        r.b = *(const u32x4*)(blk + 16 + 32 * q);
        r.c = *(const u32x4*)(blk + 32 + 32 * q);
    } else if (TYPE == TYPE_Q5_K) {
        const uint8_t* blk = buf + off;          // 16-byte aligned
        r.a = *(const u32x4*)blk;
        r.h0 = *(const u32x4*)(blk + 16);
        r.h1 = *(const u32x4*)(blk + 32);
        r.b = *(const u32x4*)(blk + 48 + 32 * q);
        r.c = *(const u32x4*)(blk + 64 + 32 * q);
    } else {
        const int h = q >> 1, l0 = 16 * (q & 1);
        r.sh = (uint32_t)(off & 2) * 8u;
        const uint8_t* b4 = buf + (off & ~3);    // dword-aligned, up to 2 bytes before the block
        const u32x4_a4 ta = *(const u32x4_a4*)(b4 + h * 64 + l0);
        const u32x4_a4 tb = *(const u32x4_a4*)(b4 + h * 64 + 32 + l0);
        const u32x4_a4 tc = *(const u32x4_a4*)(b4 + 128 + h * 32 + l0);
        r.a = u32x4_make(ta.x, ta.y, ta.z, ta.w); r.a4 = *(const uint32_t*)(b4 + h * 64 + l0 + 16);
        r.b = u32x4_make(tb.x, tb.y, tb.z, tb.w); r.b4 = *(const uint32_t*)(b4 + h * 64 + 32 + l0 + 16);
        r.c = u32x4_make(tc.x, tc.y, tc.z, tc.w); r.c4 = *(const uint32_t*)(b4 + 128 + h * 32 + l0 + 16);
        const u32x2_a4 t = *(const u32x2_a4*)(b4 + 192 + 8 * h);
        r.sc = u32x2_make(t.x, t.y);
        r.sc2 = *(const uint32_t*)(b4 + 192 + 8 * h + 8);
        r.d = *(const uint16_t*)(buf + off + 208);
    }
}

__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_x1(v);
    return v + dpp_x2(v);
}

// One quad per block: quad j (0..15) of the wave takes blocks j, j+16, ... of
// the round; the quad sum of a block lands in its slot.
template <bool MMVQ, int TYPE>
__device__ __forceinline__ void compute_round(const RoundDesc& d, const uint8_t* buf, const uint8_t* xlds,
                                              float* slots, int K, int nb, int lane) {
    constexpr int BB = block_bytes<TYPE>();
    const int quad = lane >> 2, q = lane & 3;
    const Q4Consts c = q4_consts(q);
    int col = d.col0 + quad;
    while (col >= nb) col -= nb;
    const int step = 16 % nb;
    for (int i = quad; i < d.nblk; i += 16) {
        Raw r;
        load_raw_lds<TYPE>(buf, d.delta + i * BB, q, r);
        const float v = quad_sum(block_dot<MMVQ, TYPE>(r, col, q, c, xlds, K));
        if (q == 0) slots[d.slot0 + i] = v;
        col += step;
        if (col >= nb) col -= nb;
    }
}

// Rows of a workgroup: workgroups [0, wg_split) serve the first-class rows,
// the rest the Q6_K rows; each class's rows are split evenly.
__device__ __forceinline__ void wg_rows(const StreamArgs& a, int wg, int& g0, int& g1, bool& q4) {
    q4 = wg < a.wg_split;
    const int w = q4 ? wg : wg - a.wg_split;
    const int q = q4 ? a.rows_q[0] : a.rows_q[1], rr = q4 ? a.rows_r[0] : a.rows_r[1];
    g0 = (q4 ? 0 : a.row_split) + w * q + min(w, rr);
    g1 = g0 + q + (w < rr ? 1 : 0);
}

// The workgroup's rows [g0, g1) as one sequence of blocks (OUT_SWIGLU: the
// gate rows' blocks, then the up rows'), cut into T/64 equal contiguous
// ranges, one per wave; the wave's range as up to three pieces, one per
// segment it touches.  Slots are indexed by the block's place in the
// workgroup sequence.
template <int TYPE, int L, int OUT, int T>
__device__ __forceinline__ int make_pieces(const StreamArgs& a, int g0, int g1, int wv, bool ilv, Piece (&pc)[3]) {
    constexpr int NB = WGeom<TYPE, L>::NBLK;
    const int nb = a.nb, nrow = g1 - g0;
    const int seq = nrow * nb * (OUT == OUT_SWIGLU ? 2 : 1);
    // a.ilv: the pieces are the whole workgroup's (its rounds are dealt to
    // the waves round-robin, see wave_body); else the wave's own range
    const int j0 = ilv ? 0 : (int)((int64_t)seq * wv / (T / 64));
    const int j1 = ilv ? seq : (int)((int64_t)seq * (wv + 1) / (T / 64));
    int nr = 0;
#pragma unroll
    for (int s = 0; s < 3; s++) {
        int ra, rb, o, first;          // chunk: rows [ra, rb) of the sequence order, sequence offset o, first segment row
        if (OUT == OUT_SWIGLU) {
            ra = s < 2 ? g0 : g1; rb = g1; o = s == 1 ? nrow * nb : 0; first = g0;
        } else {
            ra = max(g0, a.row_off[s]); rb = max(min(g1, a.row_off[s + 1]), ra);
            o = (ra - g0) * nb; first = ra - a.row_off[s];
        }
        const int lo = max(j0, o), hi = min(j1, o + (rb - ra) * nb);
        pc[s].nblk = hi > lo ? hi - lo : 0;
        pc[s].b0 = first * nb + (lo - o);
        pc[s].slot0 = lo;
        pc[s].rounds = (pc[s].nblk + NB - 1) / NB;
        nr += pc[s].rounds;
    }
    if (ilv) nr = nr > wv ? (nr - wv + (T / 64) - 1) / (T / 64) : 0;   // this wave's share
    return nr;
}

// ---- activation prologues (applied to an 8-value chunk held in registers)

__device__ __forceinline__ float sumsq8(const u32x4& a) {
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float v0 = f16_bits_to_f32(w[i] & 0xFFFFu), v1 = f16_bits_to_f32(w[i] >> 16);
        s += v0 * v0 + v1 * v1;
    }
    return s;
}

// half(v * rrms * w) for the 8 values of a chunk; weights: two 16-byte
// words of fp32 (w_fp32) or one of fp16 (in w0)
__device__ __forceinline__ u32x4 rms8(const u32x4& a, float rrms, int w_fp32, const u32x4& w0, const u32x4& w1) {
#pragma clang fp contract(off)
    float wv[8];
    if (w_fp32) {
        const uint32_t ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) wv[i] = __builtin_bit_cast(float, ww[i]);
    } else {
        const uint32_t hw[4] = {w0.x, w0.y, w0.z, w0.w};
#pragma unroll
        for (int i = 0; i < 4; i++) { wv[2 * i] = f16_bits_to_f32(hw[i] & 0xFFFFu); wv[2 * i + 1] = f16_bits_to_f32(hw[i] >> 16); }
    }
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float v0 = f16_bits_to_f32(w[i] & 0xFFFFu), v1 = f16_bits_to_f32(w[i] >> 16);
        o[i] = (uint32_t)f32_to_f16_bits(v0 * rrms * wv[2 * i]) | ((uint32_t)f32_to_f16_bits(v1 * rrms * wv[2 * i + 1]) << 16);
    }
    return u32x4_make(o[0], o[1], o[2], o[3]);
}

#ifdef JLLM_GEMV_TRACE
// debug build only: per-wave timestamps (s_memrealtime, 100 MHz) of the last launch
__device__ uint64_t g_gemv_trace[8192 * 8];
__device__ uint64_t g_gemv_rtrace[4096 * 48];
#define GT_MARK(i) do { tr[i] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define GT_MARK(i) do { } while (0)
#endif

// One wave's rows: rounds stream through two register stages and the wave's
// own LDS buffer; the slots of its rows are added up and stored at the end.
// Both weight types run the same two workgroup barriers (activation staging).
template <bool MMVQ, int OUT, int TYPE, int L, int NX, int PRE, int T>
__device__ __forceinline__ void wave_body(const StreamArgs& a, uint8_t* lds, int g0, int g1, int lane, int wv,
                                          uint16_t* res_lds) {
    const int nb = a.nb, K = a.K;
#ifdef JLLM_GEMV_TRACE
    uint64_t tr[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#endif
    GT_MARK(0);
#ifdef JLLM_GEMV_TRACE
    tr[7] = ((uint64_t)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32) | (uint64_t)__builtin_amdgcn_s_getreg((31 << 11) | 4);
#endif
    Piece pc[3];
    // the residual forms with K <= 8 T (one activation chunk per lane) may
    // deal rounds round-robin; the other kernels compile without the choice
    // (a runtime branch in every kernel measured 0.15-0.25 us slower for the
    // launches that do not use it)
    const bool ilv = OUT == OUT_ADD && NX == 1 && a.ilv;
    const int nr = make_pieces<TYPE, L, OUT, T>(a, g0, g1, wv, ilv, pc);
    // the descriptor of this wave's round k
    auto RD = [&](int k) { return round_desc<TYPE, L>(a, pc, ilv ? wv + k * (T / 64) : k); };
    u32x4 R0[L], R1[L];
    {
        // activation (and residual) loads first, on every wave, then a barrier,
        // then the weight loads: the CU's memory pipeline returns them first
        const int nch = K / 8;
        u32x4 xv[NX];
        u32x4 nwv[PRE == PRE_RMS ? 2 * NX : 1];     // RMSNorm weights of the lane's chunks, loaded with x
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int c = (int)threadIdx.x + T * i;
            xv[i] = *(const u32x4*)(a.x + 8 * (c < nch ? c : 0));
            if (PRE == PRE_RMS) {
                const int cc = c < nch ? c : 0;
                if (a.pre.nw_fp32) {
                    nwv[2 * i] = *((const u32x4*)a.pre.nw + 2 * cc);
                    nwv[2 * i + 1] = *((const u32x4*)a.pre.nw + 2 * cc + 1);
                } else {
                    nwv[2 * i] = *((const u32x4*)a.pre.nw + cc);
                    nwv[2 * i + 1] = u32x4_make(0u, 0u, 0u, 0u);
                }
            }
        }
        uint16_t rv = 0;
        const int nres = OUT == OUT_ADD ? g1 - g0 : 0;   // the workgroup's rows, nres <= T
        if (OUT == OUT_ADD && (int)threadIdx.x < nres) rv = a.seg[0].res[g0 + threadIdx.x];
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue_round<L>(RD(0), R0, lane);
        issue_round<L>(RD(1), R1, lane);
        __builtin_amdgcn_sched_barrier(0);
        GT_MARK(1);
        if (PRE == PRE_RMS) {
            // sum of squares of the whole activation (K <= NX * T * 8 here):
            // lanes, then waves through LDS (the first words of the block
            // slots, not written before the staging barrier below; the round
            // buffers may already be receiving weights)
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < NX; i++) {
                const int c = (int)threadIdx.x + T * i;
                if (c < nch) ss += sumsq8(xv[i]);
            }
            ss = wave_sum(ss);
            float* red = (float*)(lds + a.xlds_bytes + (T / 64) * (64 * 16 * L));
            if (lane == 0) red[wv] = ss;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            float tot = 0.0f;
#pragma unroll
            for (int w = 0; w < (T / 64); w++) tot += red[w];
            const float rrms = 1.0f / sqrtf(tot / (float)K + a.pre.eps);
#pragma unroll
            for (int i = 0; i < NX; i++) {
                const int c = (int)threadIdx.x + T * i;
                if (T * i + 64 * wv < nch && c < nch) xv[i] = rms8(xv[i], rrms, a.pre.nw_fp32, nwv[2 * i], nwv[2 * i + 1]);
            }
        }
        // staging and, below, the row sums also at raised wave priority
        // (decode 685 -> 687 tok/s)
        __builtin_amdgcn_s_setprio(1);
        // (a wave whose chunks all lie beyond K skips the staging arithmetic: uniform branch)
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int c = (int)threadIdx.x + T * i;
            if (T * i + 64 * wv >= nch) continue;
            if (MMVQ) xstage_q8_1(xv[i], c, K, lds);
            else      xstage_f16(xv[i], c, K, lds);
        }
        // K beyond NX chunks per lane (K > 10240): the rest after the weights
        for (int c0 = NX * T; c0 < nch; c0 += NX * T) {
#pragma unroll
            for (int i = 0; i < NX; i++) {
                const int c = c0 + (int)threadIdx.x + T * i;
                xv[i] = *(const u32x4*)(a.x + 8 * (c < nch ? c : 0));
            }
#pragma unroll
            for (int i = 0; i < NX; i++) {
                const int c = c0 + (int)threadIdx.x + T * i;
                if (c0 + T * i + 64 * wv >= nch) continue;
                if (MMVQ) xstage_q8_1(xv[i], c, K, lds);
                else      xstage_f16(xv[i], c, K, lds);
            }
        }
        if (OUT == OUT_ADD && (int)threadIdx.x < nres) res_lds[threadIdx.x] = rv;
        __builtin_amdgcn_s_setprio(0);
    }
    // LDS-only barrier: the weight loads in flight are not waited for
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    GT_MARK(2);
    const uint8_t* xlds = lds;
    uint8_t* buf = lds + a.xlds_bytes + wv * (64 * 16 * L);
    float* slots = (float*)(lds + a.xlds_bytes + (T / 64) * (64 * 16 * L));    // the workgroup's block slots
    // Round r travels in register stage r mod 2.  Step k: compute round k
    // from the wave's LDS buffer, move round k+1 from its registers into the
    // buffer, and reuse those registers for round k+3 (round k+2 stays in
    // flight in the other stage).  Descriptors are recomputed where needed
    // (scalar arithmetic) rather than kept per stage.
    write_round<L>(buf, R0, lane);
    __builtin_amdgcn_wave_barrier();
    GT_MARK(3);
    issue_round<L>(RD(2), R0, lane);
    auto step = [&](int k, u32x4 (&nxt)[L]) {
#ifdef JLLM_GEMV_TRACE
        const int64_t gw = (int64_t)blockIdx.x * (T / 64) + wv;
        const bool rt = gw < 4096 && k < 16 && lane == 0;
        if (rt) g_gemv_rtrace[gw * 48 + k * 3] = __builtin_amdgcn_s_memrealtime();
#endif
        // the round's arithmetic at raised wave priority: a wave whose
        // round has landed computes it ahead of waves still waiting (same
        // arithmetic; gate/up pair 8.65 -> 8.51 us, decode 679 -> 683 tok/s)
        __builtin_amdgcn_s_setprio(1);
        compute_round<MMVQ, TYPE>(RD(k), buf, xlds, slots, K, nb, lane);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_wave_barrier();
#ifdef JLLM_GEMV_TRACE
        if (rt) g_gemv_rtrace[gw * 48 + k * 3 + 1] = __builtin_amdgcn_s_memrealtime();
#endif
        write_round<L>(buf, nxt, lane);
        __builtin_amdgcn_wave_barrier();
#ifdef JLLM_GEMV_TRACE
        if (rt) g_gemv_rtrace[gw * 48 + k * 3 + 2] = __builtin_amdgcn_s_memrealtime();
#endif
        issue_round<L>(RD(k + 3), nxt, lane);
    };
    int k = 0;
    for (; k + 2 <= nr; k += 2) {
        step(k, R1);
        step(k + 1, R0);
    }
    if (k < nr) step(k, R1);
    GT_MARK(4);
    // every wave's slots are written: LDS-only barrier (no wait on global loads)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_s_setprio(1);
    // rows: 8 lanes per row add the row's slots (lane j the blocks b = j mod 8,
    // in order), then a fixed butterfly; T / 8 rows per pass
    const int nrow = g1 - g0, j = lane & 7, rg = (int)threadIdx.x >> 3;
    if (OUT == OUT_SWIGLU) {
        for (int t0 = 0; t0 < nrow; t0 += T / 8) {
            const int t = t0 + rg;
            float vg = 0.0f, vu = 0.0f;
            if (t < nrow) {
                const float* p = slots + t * nb;
                const float* q = slots + (nrow + t) * nb;
                for (int b = j; b < nb; b += 8) { vg += p[b]; vu += q[b]; }
            }
            vg += dpp_x1(vg); vu += dpp_x1(vu);
            vg += dpp_x2(vg); vu += dpp_x2(vu);
            // the other quad of the 8 lanes (every lane of a quad holds its sum)
            vg += dpp_mov_f<0x141>(vg); vu += dpp_mov_f<0x141>(vu);
            if (j == 0 && t < nrow) {
                // half(silu(g) * u) of the half-rounded pair outputs (swiglu_kernel, convert.cu:85-112)
#pragma clang fp contract(off)
                const float g = round_to_f16(vg), u = round_to_f16(vu);
                ((uint16_t*)a.seg[0].y)[g0 + t] = f32_to_f16_bits(g / (1.0f + expf(-g)) * u);
            }
        }
        GT_MARK(6);
#ifdef JLLM_GEMV_TRACE
        {
            uint64_t tv = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) if (lane == i) tv = tr[i];
            const int64_t gwt = (int64_t)blockIdx.x * (T / 64) + wv;
            if (lane < 8 && gwt < 8192) g_gemv_trace[gwt * 8 + lane] = tv;
        }
#endif
        return;
    }
    GT_MARK(5);
    for (int t0 = 0; t0 < nrow; t0 += T / 8) {
        const int t = t0 + rg;
        float v = 0.0f;
        if (t < nrow) {
            const float* p = slots + t * nb;
            for (int b = j; b < nb; b += 8) v += p[b];
        }
        v += dpp_x1(v);
        v += dpp_x2(v);
        v += dpp_mov_f<0x141>(v);      // the other quad of the 8 lanes (row_half_mirror)
        if (j == 0 && t < nrow) {
            const int g = g0 + t;
            const int sg = g >= a.row_off[1] ? (g >= a.row_off[2] ? 2 : 1) : 0;
            store_row<OUT>(a.seg[sg], g - a.row_off[sg], v, res_lds, t);
        }
    }
    GT_MARK(6);
#ifdef JLLM_GEMV_TRACE
    {
        uint64_t tv = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) if (lane == i) tv = tr[i];
        const int64_t gwt = (int64_t)blockIdx.x * (T / 64) + wv;
        if (lane < 8 && gwt < 8192) g_gemv_trace[gwt * 8 + lane] = tv;
    }
#endif
}

// Pin a uniform value into SGPRs here (kernel-argument loads are otherwise
// issued lazily, one dependent round trip at a time).
template <class T>
__device__ __forceinline__ void pin_sgpr(const T& v) { asm volatile("" :: "s"(v)); }

// TA: the type of the first row class (Q4_K or Q5_K); the second is Q6_K.
template <bool MMVQ, int OUT, int L, int NX, int PRE, int TA, int T>
__global__ __launch_bounds__(T) __attribute__((amdgpu_waves_per_eu(4)))
void gemv_stream_kernel(StreamArgs a_in) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    StreamArgs a = a_in;
    // every argument the kernel needs in SGPRs, requested at one point: one
    // batch of scalar loads and one wait (separate requests serialise into
    // one round trip each, ~0.1 us apiece at the start of the kernel)
    asm volatile("" :: "s"(a.seg[0].W), "s"(a.seg[1].W), "s"(a.seg[2].W), "s"(a.seg[0].y), "s"(a.seg[1].y),
                 "s"(a.seg[2].y), "s"(a.row_off[0]), "s"(a.row_off[1]), "s"(a.row_off[2]), "s"(a.row_off[3]),
                 "s"(a.x), "s"(a.K), "s"(a.nb), "s"(a.xlds_bytes), "s"(a.row_split), "s"(a.wg_split),
                 "s"(a.slots_per_wg), "s"(a.rows_q[0]), "s"(a.rows_q[1]), "s"(a.rows_r[0]), "s"(a.rows_r[1]));
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int g0, g1;
    bool q4;
    wg_rows(a, blockIdx.x, g0, g1, q4);
    uint16_t* res_lds = (uint16_t*)(lds + a.xlds_bytes + (T / 64) * (64 * 16 * L) + 4 * a.slots_per_wg);
    // (both bodies hold the same workgroup barriers; a workgroup serves one class)
    if constexpr (OUT == OUT_SWIGLU) {
        wave_body<MMVQ, OUT, TA, L, NX, PRE, T>(a, lds, g0, g1, lane, wv, res_lds);
    } else {
        if (q4) wave_body<MMVQ, OUT, TA, L, NX, PRE, T>(a, lds, g0, g1, lane, wv, res_lds);
        else    wave_body<MMVQ, OUT, TYPE_Q6_K, L, NX, PRE, T>(a, lds, g0, g1, lane, wv, res_lds);
    }
}

template <bool MMVQ, int OUT, int L, int NX, int PRE, int TA, int T>
static hipError_t launch_s(const StreamArgs& a, int grid, size_t lds, hipStream_t st) {
    static const hipError_t attr = hipFuncSetAttribute((const void*)gemv_stream_kernel<MMVQ, OUT, L, NX, PRE, TA, T>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((gemv_stream_kernel<MMVQ, OUT, L, NX, PRE, TA, T>), dim3(grid), dim3(T), lds, st, a);
    return hipGetLastError();
}

template <bool MMVQ, int OUT, int L, int PRE, int TA, int T>
static hipError_t launch_nx_t(const StreamArgs& a, int grid, size_t lds, hipStream_t st) {
    const int nch = a.K / 8;
    if (nch <= T) return launch_s<MMVQ, OUT, L, 1, PRE, TA, T>(a, grid, lds, st);
    if constexpr (PRE == PRE_RMS) {
        return launch_s<MMVQ, OUT, L, 2, PRE, TA, T>(a, grid, lds, st);
    } else {
        if (nch <= 2 * T) return launch_s<MMVQ, OUT, L, 2, PRE, TA, T>(a, grid, lds, st);
        return launch_s<MMVQ, OUT, L, 5, PRE, TA, T>(a, grid, lds, st);
    }
}

// Q5_K rows exist only in float mode
template <bool MMVQ, int OUT, int L, int PRE = PRE_NONE>
static hipError_t launch_nx(const StreamArgs& a, int grid, size_t lds, hipStream_t st, bool q5, int threads) {
    if constexpr (MMVQ) {
        if (q5) return hipErrorInvalidValue;
        return threads == ST_T_SMALL ? launch_nx_t<true, OUT, L, PRE, TYPE_Q4_K, ST_T_SMALL>(a, grid, lds, st)
                                     : launch_nx_t<true, OUT, L, PRE, TYPE_Q4_K, ST_T>(a, grid, lds, st);
    } else {
        if (q5) return threads == ST_T_SMALL ? launch_nx_t<false, OUT, L, PRE, TYPE_Q5_K, ST_T_SMALL>(a, grid, lds, st)
                                             : launch_nx_t<false, OUT, L, PRE, TYPE_Q5_K, ST_T>(a, grid, lds, st);
        return threads == ST_T_SMALL ? launch_nx_t<false, OUT, L, PRE, TYPE_Q4_K, ST_T_SMALL>(a, grid, lds, st)
                                     : launch_nx_t<false, OUT, L, PRE, TYPE_Q4_K, ST_T>(a, grid, lds, st);
    }
}

static constexpr size_t LDS_CU = 160 * 1024;
// Workgroups per CU by launch size (measured on MI355X, graphs of 36 layers):
// 2 (8 waves per CU) for a decode-layer matrix -- fewer waves reach the CU
// sooner and each streams more rounds (gate/up pair with RMSNorm + SwiGLU
// 11.1 -> 9.3 us, down 8.95 -> 8.35 us against 4 per CU); 1 under 12 MB
// (QKV triple 6.4 -> 6.05 us, O 6.05 -> 5.7 us); 4 above 64 MB (the
// lm_head, 63 -> 61 us).
#ifndef JLLM_GEMV_WG_PER_CU
#define JLLM_GEMV_WG_PER_CU 2
#endif
#ifndef JLLM_GEMV_WG_PER_CU_BIG
#define JLLM_GEMV_WG_PER_CU_BIG 4
#endif
#ifndef JLLM_GEMV_WG_PER_CU_SMALL
#define JLLM_GEMV_WG_PER_CU_SMALL 1
#endif
#ifndef JLLM_GEMV_ROUND_KB
#define JLLM_GEMV_ROUND_KB 4
#endif
constexpr int ST_L = JLLM_GEMV_ROUND_KB;   // 16-byte chunks per lane per round (KiB per wave round)

hipError_t gemv_launch(const GemvArgs& in, bool mmvq, int out_kind, hipStream_t st) {
    if (out_kind == OUT_ADD && in.nseg != 1) return hipErrorInvalidValue;
    const bool sw = out_kind == OUT_SWIGLU;
    if (sw && (in.nseg != 2 || in.seg[0].type != in.seg[1].type || in.seg[0].M != in.seg[1].M ||
               (in.seg[0].type != TYPE_Q4_K && in.seg[0].type != TYPE_Q5_K)))
        return hipErrorInvalidValue;
    bool has4 = false, has5 = false;
    for (int i = 0; i < in.nseg; i++) {
        has4 |= in.seg[i].type == TYPE_Q4_K && in.seg[i].M > 0;
        has5 |= in.seg[i].type == TYPE_Q5_K && in.seg[i].M > 0;
    }
    if (has5 && mmvq) return hipErrorInvalidValue;
    if (has4 && has5 && !sw) {
        // one launch per first-class type: the Q5_K (and Q6_K) rows, then the Q4_K rows
        GemvArgs p = in, r = in;
        p.nseg = r.nseg = 0;
        for (int i = 0; i < in.nseg; i++) {
            if (in.seg[i].type == TYPE_Q4_K) r.seg[r.nseg++] = in.seg[i];
            else p.seg[p.nseg++] = in.seg[i];
        }
        const hipError_t e = gemv_launch(p, mmvq, out_kind, st);
        return e != hipSuccess ? e : gemv_launch(r, mmvq, out_kind, st);
    }
    const int ta = has5 ? TYPE_Q5_K : TYPE_Q4_K;
    StreamArgs a;
    a.K = in.K;
    a.x = in.x;
    a.nb = in.K / QK_K;
    // first-class (Q4_K or Q5_K) segments first, then Q6_K (stable); unused slots are empty
    int n = 0;
    for (int i = 0; i < in.nseg; i++) if (in.seg[i].type == ta) a.seg[n++] = in.seg[i];
    const int nseg4 = n;
    for (int i = 0; i < in.nseg; i++) if (in.seg[i].type == TYPE_Q6_K) a.seg[n++] = in.seg[i];
    if (n == 0) return hipSuccess;
    for (int i = n; i < 3; i++) { a.seg[i] = a.seg[n - 1]; a.seg[i].M = 0; }
    a.row_off[0] = 0;
    for (int i = 0; i < 3; i++) a.row_off[i + 1] = a.row_off[i] + a.seg[i].M;
    a.swiglu = sw;
    // OUT_SWIGLU: the row sequence is the M row pairs (two rows' slots per pair)
    const int64_t rows4 = sw ? in.seg[0].M : a.row_off[nseg4], rows6 = sw ? 0 : a.row_off[3] - rows4;
    const int64_t slot_rows = sw ? 2 : 1;
    if (rows4 + rows6 <= 0) return hipSuccess;
    a.row_split = (int)rows4;
    const int64_t bytes4 = rows4 * a.nb * (has5 ? Q5K_BYTES : Q4K_BYTES), bytes6 = rows6 * a.nb * Q6K_BYTES;
    a.xlds_bytes = (int)((gemv_lds_bytes(mmvq, a.K) + 15) & ~(size_t)15);
    const int64_t wbytes = bytes4 + bytes6;
    // 512 threads (the same waves per CU in half the workgroups) where it
    // measured faster: under 12 MB, above 64 MB (lm_head 62 -> 61 us) and in
    // between for every product except the residual form from 16 MB up
    // (gate/up pair 9.3-9.6 -> 9.0-9.2 us, RMSNorm + gate/up + SwiGLU 8.59 ->
    // 8.52 us, Q4_K down + residual (14 MB) 7.07 -> 6.84 us; Q6_K down +
    // residual (20 MB) 8.19 -> 8.33 us, so 256 there)
    const bool mid_plain = out_kind != OUT_ADD || wbytes < ((int64_t)16 << 20);
    int threads = (wbytes < ((int64_t)12 << 20) || wbytes > ((int64_t)64 << 20) || mid_plain) ? ST_T_SMALL : ST_T;
    // (8 waves' round buffers and a large activation may not fit one CU's LDS: then 4 waves)
    if (threads == ST_T_SMALL &&
        (size_t)a.xlds_bytes + (size_t)(ST_T_SMALL / 64) * (64 * 16 * ST_L) + 16384 > LDS_CU)
        threads = ST_T;
    const size_t wbuf = (size_t)(threads / 64) * (size_t)(64 * 16 * ST_L);
    // JLLM_GEMV_WG_PER_CU workgroups per CU when LDS allows, split between
    // the classes by bytes; a workgroup takes a contiguous row range
    int64_t grid = 0;
    int64_t w4 = 0, w6 = 0, max_rows = 0;
    auto split = [&](int64_t g) {
        const int64_t w = g;
        if (rows6 == 0) { w4 = w; w6 = 0; }
        else if (rows4 == 0) { w4 = 0; w6 = w; }
        else {
            w4 = (w * bytes4 + (bytes4 + bytes6) / 2) / (bytes4 + bytes6);
            w4 = w4 < 1 ? 1 : (w4 > w - 1 ? w - 1 : w4);
            w6 = w - w4;
        }
        max_rows = std::max(w4 ? (rows4 + w4 - 1) / w4 : 0, w6 ? (rows6 + w6 - 1) / w6 : 0);
    };
    auto lds_of = [&]() {
        const size_t res = out_kind == OUT_ADD ? (size_t)max_rows * 2 : 0;
        return (size_t)a.xlds_bytes + wbuf + (size_t)4 * std::max<int64_t>(slot_rows * max_rows * a.nb, 16) + res;
    };
    // (the residual rows of a workgroup are staged one per lane)
    auto fits = [&](int per_cu) { return (size_t)per_cu * lds_of() <= LDS_CU && !(out_kind == OUT_ADD && max_rows > threads); };
    int per_cu0 = wbytes > ((int64_t)64 << 20) ? JLLM_GEMV_WG_PER_CU_BIG
                      : (wbytes < ((int64_t)12 << 20) ? JLLM_GEMV_WG_PER_CU_SMALL : JLLM_GEMV_WG_PER_CU);
    if (threads == ST_T_SMALL && wbytes >= ((int64_t)12 << 20)) per_cu0 /= 2;     // same waves per CU
    for (int per_cu = per_cu0; per_cu >= 1 && grid == 0; per_cu--) {
        split((int64_t)device_cus() * per_cu);
        if (fits(per_cu)) grid = (int64_t)device_cus() * per_cu;
    }
    if (grid == 0) {      // rows too many for one resident grid: more workgroups, in several waves
        grid = device_cus();
        split(grid);
        while (!fits(1)) {
            if (grid > (int64_t)1 << 24) return hipErrorInvalidValue;
            split(grid *= 2);
        }
    }
    a.wg_split = (int)w4;
    a.rows_q[0] = w4 > 0 ? (int)(rows4 / w4) : 0; a.rows_r[0] = w4 > 0 ? (int)(rows4 % w4) : 0;
    a.rows_q[1] = w6 > 0 ? (int)(rows6 / w6) : 0; a.rows_r[1] = w6 > 0 ? (int)(rows6 % w6) : 0;
    a.slots_per_wg = (int)std::max<int64_t>(slot_rows * max_rows * a.nb, 16);   // >= 16: the RMSNorm staging's wave sums
    {
        // Rounds dealt round-robin (residual forms only) when a wave's own
        // range would hold at most two rounds: measured (graphs of 36 layers)
        // O + residual, Q4_K 2560 x 4096, 5.46 -> 4.79 us; QKV triple
        // unchanged; with ~6 rounds per wave it costs (gate/up pair 8.8 ->
        // 9.0 us, Q6_K down 8.21 -> 8.37 us)
        const int nbk = WGeom<TYPE_Q6_K, ST_L>::NBLK;     // 16 blocks per round for every type
        const int64_t per_wave = (int64_t)a.slots_per_wg / (threads / 64);
        a.ilv = per_wave <= 2 * nbk ? 1 : 0;
    }
    const size_t lds = lds_of();
    const int g = (int)grid;
    a.pre = in.pre;
    if (in.pre.kind == PRE_RMS) {      // the sum of squares needs the whole x in the first staging pass
        if (a.K > 2 * threads * 8) return hipErrorInvalidValue;
        if (mmvq && out_kind == OUT_HALF) return launch_nx<true, OUT_HALF, ST_L, PRE_RMS>(a, g, lds, st, has5, threads);
        if (mmvq && out_kind == OUT_F32)  return launch_nx<true, OUT_F32, ST_L, PRE_RMS>(a, g, lds, st, has5, threads);
        if (!mmvq && out_kind == OUT_F32) return launch_nx<false, OUT_F32, ST_L, PRE_RMS>(a, g, lds, st, has5, threads);
        if (!mmvq && out_kind == OUT_HALF) return launch_nx<false, OUT_HALF, ST_L, PRE_RMS>(a, g, lds, st, has5, threads);
        if (mmvq && sw) return launch_nx<true, OUT_SWIGLU, ST_L, PRE_RMS>(a, g, lds, st, has5, threads);
        if (!mmvq && sw) return launch_nx<false, OUT_SWIGLU, ST_L, PRE_RMS>(a, g, lds, st, has5, threads);
        return hipErrorInvalidValue;
    }
    if (sw) {
        if (mmvq) return launch_nx<true, OUT_SWIGLU, ST_L>(a, g, lds, st, has5, threads);
        return launch_nx<false, OUT_SWIGLU, ST_L>(a, g, lds, st, has5, threads);
    }
    if (mmvq) {
        if (out_kind == OUT_HALF) return launch_nx<true, OUT_HALF, ST_L>(a, g, lds, st, has5, threads);
        if (out_kind == OUT_F32)  return launch_nx<true, OUT_F32, ST_L>(a, g, lds, st, has5, threads);
        return launch_nx<true, OUT_ADD, ST_L>(a, g, lds, st, has5, threads);
    }
    if (out_kind == OUT_HALF) return launch_nx<false, OUT_HALF, ST_L>(a, g, lds, st, has5, threads);
    if (out_kind == OUT_F32)  return launch_nx<false, OUT_F32, ST_L>(a, g, lds, st, has5, threads);
    return launch_nx<false, OUT_ADD, ST_L>(a, g, lds, st, has5, threads);
}

#ifdef JLLM_GEMV_TRACE
extern "C" int jllm_hip_gemv_trace_read(uint64_t* host, int n) {
    if (n < 0) return -1;
    if (n > 8192 * 8) n = 8192 * 8;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_gemv_trace), (size_t)n * 8, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
extern "C" int jllm_hip_gemv_rtrace_read(uint64_t* host) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_gemv_rtrace), (size_t)4096 * 48 * 8, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif

hipError_t quantize_q8_1_aos_launch(const uint16_t* x, void* y, int K, hipStream_t st) {
    const int n = (K / 32) * 8;
    hipLaunchKernelGGL(quantize_q8_1_aos_kernel, dim3((n + GEMV_THREADS - 1) / GEMV_THREADS),
                       dim3(GEMV_THREADS), 0, st, x, (uint8_t*)y, K);
    return hipGetLastError();
}

}  // namespace jllm_hip
