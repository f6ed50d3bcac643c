// gemv.hip -- Q4_K / Q6_K decode GEMV for gfx950 (wave64).
//
// Two arithmetic modes, matching the reference dispatcher's defaults
// (gemv_q4.cu:1245-1616):
//   * MMVQ: the fp16 activation is quantised to q8_1 (32-value blocks,
//     gemv_q4.cu:445-466) and dotted as int8 (v_dot4_i32_i8) against the
//     weight codes, one exact int32 per 32-weight Q4_K sub-block or per
//     4-weight Q6_K group, then scaled in fp32 (gemv_q4.cu:474-618).
//   * float dequant: weights dequantised in registers and dotted with the
//     fp16 activation in fp32 (gemv_q4.cu:266-398).
//
// Layout of the work: every workgroup (256 lanes) first stages the whole
// activation vector in LDS -- for MMVQ it quantises it there, so no q8_1
// scratch buffer and no separate quantiser launch are needed.  Then groups
// of LPR lanes own one output row; inside a group, each 8-lane octet streams
// one super-block per step (Q4_K: two 16 B loads per lane, Q6_K: three
// 8 B loads per lane), so a wave's load instruction touches whole 144/210 B
// blocks.  Rows are reduced with lane shuffles at the end.
#include "kq_common.h"
#include "gemv.h"

#ifndef JLLM_GEMV_NT
#define JLLM_GEMV_NT 0
#endif
// Weight loads: streaming (non-temporal) or ordinary cached loads.
#if JLLM_GEMV_NT
#define WLOAD(p) __builtin_nontemporal_load(p)
#else
#define WLOAD(p) (*(p))
#endif

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

// MMVQ staging: q8 codes [K] | d8 fp32 [K/32] | s8 fp32 [K/32] | q6 group
// code sums int [K/16] (lane order).
__device__ __forceinline__ void stage_q8_1(const uint16_t* __restrict__ x, int K, uint8_t* lds) {
    int8_t* s_q = (int8_t*)lds;
    float* s_d8 = (float*)(lds + K);
    float* s_s8 = s_d8 + K / 32;
    int* s_sx = (int*)(s_s8 + K / 32);
    const int n = (K / 32) * 8;
    for (int t = threadIdx.x; t < n; t += GEMV_THREADS) {
        const int blk = t >> 3, sub = t & 7;
        const u32x2 raw = *(const u32x2*)(x + blk * 32 + sub * 4);
        float d; int sall, shalf;
        const uint32_t packed = quant_q8_1_x4(raw, d, sall, shalf);
        *(uint32_t*)(s_q + blk * 32 + sub * 4) = packed;
        if (sub == 0) {
            // s = d*sum(q) rounded through fp16 like the stored block_q8_1 field
            s_d8[blk] = round_to_f16(d);
            s_s8[blk] = round_to_f16(d * (float)sall);
        }
        if ((sub & 3) == 0) s_sx[q6_group_slot(blk * 2 + (sub >> 2))] = shalf;
    }
}

// x index -> LDS half index: 8 halves of padding after every 128, so that the
// quads' reads 256 B apart land in different banks.
__device__ __forceinline__ int xpad(int k) { return k + ((k >> 7) << 3); }

// float staging: x fp16 [K + K/16 padded] | per-32 fp32 sums [K/32] |
// 32 * per-16 fp32 sums [K/16] (Q6_K lane order).
__device__ __forceinline__ void stage_f16(const uint16_t* __restrict__ x, int K, uint8_t* lds) {
    uint16_t* s_x = (uint16_t*)lds;
    float* s_x32 = (float*)(lds + 2 * K + K / 8);
    float* s_x16 = s_x32 + K / 32;
    const int n = K / 16;
    const uint32_t one = 0x3C003C00u;
    for (int t = threadIdx.x; t < n; t += GEMV_THREADS) {
        const u32x4 a = *(const u32x4*)(x + t * 16);
        const u32x4 b = *(const u32x4*)(x + t * 16 + 8);
        *(u32x4*)(s_x + xpad(t * 16)) = a;
        *(u32x4*)(s_x + xpad(t * 16) + 8) = b;
        float s = 0.0f;
        s = fdot2(a.x, one, s); s = fdot2(a.y, one, s); s = fdot2(a.z, one, s); s = fdot2(a.w, one, s);
        s = fdot2(b.x, one, s); s = fdot2(b.y, one, s); s = fdot2(b.z, one, s); s = fdot2(b.w, one, s);
        s_x16[q6_group_slot(t)] = 32.0f * s;
        const float s2 = s + __shfl_xor(s, 1, 64);
        if ((t & 1) == 0) s_x32[t >> 1] = s2;
    }
}

// ---- raw weight loads ------------------------------------------------------

// Quad lane layout: 4 lanes per super-block; lane q (0..3) owns 64 weights.
//   Q4_K: qs bytes [32q, 32q+32): low nibbles = sub-block 2q, high = 2q+1.
//   Q6_K: half h = q/2 of the block, positions l0..l0+15 (l0 = 16*(q&1)) of
//         each 32-wide quarter g = 0..3: elements h*128 + 32g + l0 + [0,16).
// One register layout for both types (Q4_K uses a = header, b/c = qs) so a
// wave can keep prefetched blocks of either type in the same registers.
// Q6_K pieces are loaded dword-aligned from 2 bytes early when the block is
// only 2-byte aligned (sh = 16); the funnel shift that realigns them is
// applied at use, so no load has to be waited for before the next is issued.
struct Raw { u32x4 a, b, c; uint32_t a4, b4, c4; u32x2 sc; uint32_t sc2, d, sh; };
template <int TYPE> struct RawT { Raw r; };
typedef RawT<TYPE_Q4_K> RawQ4;
typedef RawT<TYPE_Q6_K> RawQ6;

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ u32x4 ld_nt16(const uint8_t* p) {
    const u32x4 v = WLOAD((const u32x4*)p);
    return u32x4_make(v.x, v.y, v.z, v.w);
}

// A piece of a Q6_K block that starts at a 2-byte-aligned address p: load the
// dword-aligned window [p - pad, p - pad + 20) (pad = p & 2), realign later.
__device__ __forceinline__ void ld16_window(const uint8_t* p, u32x4& v, uint32_t& w4) {
    const uint8_t* base = p - ((uintptr_t)p & 3u);   // keeps the global address space
    const u32x4_a4 t = WLOAD((const u32x4_a4*)base);
    v = u32x4_make(t.x, t.y, t.z, t.w);
    w4 = WLOAD((const uint32_t*)(base + 16));
}

__device__ __forceinline__ u32x4 realign16(const u32x4& v, uint32_t w4, uint32_t sh) {
    return u32x4_make(__builtin_amdgcn_alignbit(v.y, v.x, sh), __builtin_amdgcn_alignbit(v.z, v.y, sh),
                      __builtin_amdgcn_alignbit(v.w, v.z, sh), __builtin_amdgcn_alignbit(w4, v.w, sh));
}

template <int TYPE>
__device__ __forceinline__ void load_raw(const uint8_t* __restrict__ blk, int q, Raw& r) {
    if (TYPE == TYPE_Q4_K) {
        r.a = ld_nt16(blk);                  // d, dmin, scales[12]
        r.b = ld_nt16(blk + 16 + 32 * q);
        r.c = ld_nt16(blk + 32 + 32 * q);
    } else {
        const int h = q >> 1, l0 = 16 * (q & 1);
        r.sh = (uint32_t)((uintptr_t)blk & 2u) * 8u;
        ld16_window(blk + h * 64 + l0, r.a, r.a4);        // ql, quarters 0 / 2
        ld16_window(blk + h * 64 + 32 + l0, r.b, r.b4);   // ql, quarters 1 / 3
        ld16_window(blk + 128 + h * 32 + l0, r.c, r.c4);  // qh
        const uint8_t* sb = blk + 192 + 8 * h - ((uintptr_t)blk & 3u);
        const u32x2_a4 t = WLOAD((const u32x2_a4*)sb);
        r.sc = u32x2_make(t.x, t.y);
        r.sc2 = WLOAD((const uint32_t*)(sb + 8));
        r.d = WLOAD((const uint16_t*)(blk + 208));
    }
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
    const float a = (float)(dl * (int)sc0) * d8.x + (float)(dh * (int)sc1) * d8.y;
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

template <int OUT>
__device__ __forceinline__ void store_row(const GemvSeg& s, int r, float acc) {
    if (OUT == OUT_F32) {
        ((float*)s.y)[r] = acc;
    } else if (OUT == OUT_HALF) {
        ((uint16_t*)s.y)[r] = f32_to_f16_bits(acc);
    } else {   // y = half(half(W x) + residual), gemv_q4.cu:1001-1004
        const float proj = round_to_f16(acc);
        ((uint16_t*)s.y)[r] = f32_to_f16_bits(proj + f16_bits_to_f32(s.res[r]));
    }
}

__device__ __forceinline__ float row_reduce(float v, int lpr) {
    if (lpr > 32) v += __shfl_xor(v, 32, 64);
    if (lpr > 16) v += __shfl_xor(v, 16, 64);
    if (lpr > 8)  v += __shfl_xor(v, 8, 64);
    if (lpr > 4)  v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 1, 64);
    return v;
}

// Work of one wave: a sequence of row groups (rpw = 64/lpr rows of one
// segment each, so the weight type is wave-uniform), each split into `spg`
// steps of U blocks per lane.  Quad qi of a row owns the contiguous blocks
// [qi*per_q, (qi+1)*per_q); per_q is even for Q6_K so that all quads of a
// wave touch blocks of the same 4-byte alignment at every step.
struct WaveWork {
    int grp0, gstride, ngrp_end;   // groups grp0, grp0+gstride, ... < ngrp_end
    int spg;                       // steps per group
};

struct StepPos {
    const uint8_t* blk0;  // address of the step's first block (clamped to a valid block)
    const uint8_t* blk1;  // address of the step's second block (clamped)
    int s;                // wave-uniform segment
    int r;                // row within the segment
    bool live;            // row exists
    bool v0, v1;          // the two blocks belong to this lane
    int b_first;          // block index of the first block
};

// grp is wave-uniform; it is made explicitly so (readfirstlane) so that the
// segment lookups below are scalar loads from the kernel arguments.  Block
// addresses are clamped to valid blocks of the matrix so that every lane
// issues the same loads (exact wait counts, no branches around loads); the
// data of blocks that are not the lane's is never used.
template <int TYPE>
__device__ __forceinline__ StepPos step_pos(const GemvArgs& a, int grp, int step, int lane, int lpr, int rpw,
                                            int qi, int per_q, int nb) {
    constexpr int BB = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    StepPos p;
    grp = __builtin_amdgcn_readfirstlane(grp);
    const int s = grp >= a.gend[0] ? (grp >= a.gend[1] ? 2 : 1) : 0;
    const int gstart = s == 0 ? 0 : a.gend[s - 1];
    p.s = s;
    p.r = (grp - gstart) * rpw + lane / lpr;
    p.live = p.r < a.seg[s].M;
    const int q0 = qi * per_q;
    const int b_end = min(q0 + per_q, nb);
    p.b_first = q0 + step * 2;
    p.v0 = p.live && p.b_first < b_end;
    p.v1 = p.live && p.b_first + 1 < b_end;
    const uint8_t* rowp = a.seg[s].W + (int64_t)(p.live ? p.r : 0) * nb * BB;
    p.blk0 = rowp + (int64_t)(p.v0 ? p.b_first : 0) * BB;
    p.blk1 = rowp + (int64_t)(p.v1 ? p.b_first + 1 : 0) * BB;
    return p;
}

template <bool MMVQ, int TYPE>
__device__ __forceinline__ float block_dot(const Raw& r, int b, int q, const Q4Consts& c, const uint8_t* lds, int K) {
    return MMVQ ? mmvq_block<TYPE>(r, b, q, c, lds, K) : f16_block<TYPE>(r, b, q, c, lds, K);
}

template <bool MMVQ, int TYPE>
__device__ __forceinline__ float compute_step(const StepPos& p, int q, const Q4Consts& c,
                                              const uint8_t* lds, int K, const Raw& r0, const Raw& r1) {
    float acc = 0.0f;
    if (p.v0) acc += block_dot<MMVQ, TYPE>(r0, p.b_first, q, c, lds, K);
    __builtin_amdgcn_sched_barrier(0);
    if (p.v1) acc += block_dot<MMVQ, TYPE>(r1, p.b_first + 1, q, c, lds, K);
    return acc;
}

#ifndef JLLM_GEMV_WAVES_PER_EU
#define JLLM_GEMV_WAVES_PER_EU 2
#endif

// The waves of the workgroups assigned to one weight type walk that type's
// row groups [g_begin, g_end) grid-stride; steps of two blocks per lane run
// through a two-stage register pipeline (loads of step i+1 in flight while
// step i is computed).  The first step is issued before x is staged.
template <bool MMVQ, int OUT, int TYPE>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, uint8_t* lds, int g_begin, int g_end,
                                          int wg, int nwg) {
    const int K = a.K, nb = K / QK_K, lpr = a.lpr;
    const int rpw = 64 / lpr;
    const int lane = threadIdx.x & 63;
    const int qi = (lane & (lpr - 1)) >> 2, q = lane & 3;
    const int wave0 = g_begin + __builtin_amdgcn_readfirstlane((wg * GEMV_THREADS + threadIdx.x) >> 6);
    const int nwaves = nwg * (GEMV_THREADS / 64);
    const Q4Consts c = q4_consts(q);
    const int per_q = a.per_q;
    const int spg = (per_q + 1) / 2;
    const int my_groups = wave0 < g_end ? (g_end - wave0 + nwaves - 1) / nwaves : 0;
    const int total = my_groups * spg;

    Raw A0, A1, B0, B1;
    StepPos pa, pb;
    if (total > 0) {
        pa = step_pos<TYPE>(a, wave0, 0, lane, lpr, rpw, qi, per_q, nb);
        load_raw<TYPE>(pa.blk0, q, A0);
        load_raw<TYPE>(pa.blk1, q, A1);
    }
    if (MMVQ) stage_q8_1(a.x, K, lds);
    else      stage_f16(a.x, K, lds);
    __syncthreads();

    float acc = 0.0f;
    auto finish = [&](const StepPos& p, int i) {
        if ((i % spg) == spg - 1) {
            const float v = row_reduce(acc, lpr);
            if (p.live && (threadIdx.x & (lpr - 1)) == 0) store_row<OUT>(a.seg[p.s], p.r, v);
            acc = 0.0f;
        }
    };
    for (int i = 0; i < total; i += 2) {
        if (i + 1 < total) {
            pb = step_pos<TYPE>(a, wave0 + ((i + 1) / spg) * nwaves, (i + 1) % spg, lane, lpr, rpw, qi, per_q, nb);
            load_raw<TYPE>(pb.blk0, q, B0);
            load_raw<TYPE>(pb.blk1, q, B1);
        }
        acc += compute_step<MMVQ, TYPE>(pa, q, c, lds, K, A0, A1);
        finish(pa, i);
        if (i + 1 >= total) break;
        if (i + 2 < total) {
            pa = step_pos<TYPE>(a, wave0 + ((i + 2) / spg) * nwaves, (i + 2) % spg, lane, lpr, rpw, qi, per_q, nb);
            load_raw<TYPE>(pa.blk0, q, A0);
            load_raw<TYPE>(pa.blk1, q, A1);
        }
        acc += compute_step<MMVQ, TYPE>(pb, q, c, lds, K, B0, B1);
        finish(pb, i + 1);
    }
}

// Segments are ordered Q4_K first; workgroups [0, wg_split) serve the Q4_K
// row groups [0, g_split), the rest serve the Q6_K groups [g_split, gend[2]).
template <bool MMVQ, int OUT>
__global__ __launch_bounds__(GEMV_THREADS) __attribute__((amdgpu_waves_per_eu(JLLM_GEMV_WAVES_PER_EU)))
void gemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if ((int)blockIdx.x < a.wg_split) gemv_body<MMVQ, OUT, TYPE_Q4_K>(a, lds, 0, a.g_split, blockIdx.x, a.wg_split);
    else gemv_body<MMVQ, OUT, TYPE_Q6_K>(a, lds, a.g_split, a.gend[2], blockIdx.x - a.wg_split, gridDim.x - a.wg_split);
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

#ifndef JLLM_GEMV_WAVES_PER_CU
#define JLLM_GEMV_WAVES_PER_CU 12
#endif

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

// Lanes per row: one quad per row unless the row groups are too few to give
// every resident wave two of them; then more quads share each row.
static int pick_lpr(int64_t rows, int nb, int64_t resident_waves) {
    int lpr = 4;
    while (lpr < 64 && lpr < 4 * nb && rows * lpr / 64 < 2 * resident_waves) lpr *= 2;
    return lpr;
}

template <bool MMVQ, int OUT>
static hipError_t launch_k(const GemvArgs& a, int grid, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((gemv_kernel<MMVQ, OUT>), dim3(grid), dim3(GEMV_THREADS), lds, st, a);
    return hipGetLastError();
}

hipError_t gemv_launch(const GemvArgs& a_in, bool mmvq, int out_kind, int lpr_override, hipStream_t st) {
    GemvArgs a = a_in;
    // Q4_K segments first (stable), then Q6_K; unused slots are empty copies.
    {
        GemvSeg tmp[3];
        int n = 0;
        for (int i = 0; i < a.nseg; i++) if (a.seg[i].type == TYPE_Q4_K) tmp[n++] = a.seg[i];
        for (int i = 0; i < a.nseg; i++) if (a.seg[i].type != TYPE_Q4_K) tmp[n++] = a.seg[i];
        for (int i = 0; i < a.nseg; i++) a.seg[i] = tmp[i];
    }
    int64_t rows = 0;
    for (int i = 0; i < a.nseg; i++) rows += a.seg[i].M;
    for (int i = a.nseg; i < 3; i++) { a.seg[i] = a.seg[a.nseg - 1]; a.seg[i].M = 0; }
    if (rows <= 0) return hipSuccess;
    const int nb = a.K / QK_K;
    const int waves_per_cu = JLLM_GEMV_WAVES_PER_CU;
    const int64_t resident = (int64_t)device_cus() * waves_per_cu;
    const int lpr = lpr_override ? lpr_override : pick_lpr(rows, nb, resident);
    const int rpw = 64 / lpr, nq = lpr / 4;
    int g = 0;
    for (int i = 0; i < 3; i++) { g += (a.seg[i].M + rpw - 1) / rpw; a.gend[i] = g; }
    a.lpr = lpr;
    bool any_q6 = false;
    for (int i = 0; i < a.nseg; i++) any_q6 |= a.seg[i].type == TYPE_Q6_K;
    int per_q = (nb + nq - 1) / nq;
    if (any_q6 && nq > 1 && (per_q & 1)) per_q++;
    a.per_q = per_q;
    int g4 = 0;
    int64_t bytes4 = 0, bytes6 = 0;
    for (int i = 0; i < 3; i++) {
        if (a.seg[i].type == TYPE_Q4_K) { g4 = a.gend[i]; bytes4 += (int64_t)a.seg[i].M * nb * Q4K_BYTES; }
        else bytes6 += (int64_t)a.seg[i].M * nb * Q6K_BYTES;
    }
    a.g_split = g4;
    const int64_t waves = g < resident ? g : resident;
    int grid = (int)((waves + 3) / 4);
    if (bytes4 > 0 && bytes6 > 0) {
        // split the workgroups in proportion to the bytes each type streams
        if (grid < 2) grid = 2;
        int w4 = (int)((grid * bytes4 + (bytes4 + bytes6) / 2) / (bytes4 + bytes6));
        w4 = w4 < 1 ? 1 : (w4 > grid - 1 ? grid - 1 : w4);
        const int gq4 = (g4 + 3) / 4, gq6 = (g - g4 + 3) / 4;        // WGs needed at one group per wave
        if (w4 > gq4) w4 = gq4;
        if (grid - w4 > gq6) grid = w4 + gq6;
        a.wg_split = w4;
    } else {
        a.wg_split = bytes4 > 0 ? grid : 0;
    }
    const size_t lds = gemv_lds_bytes(mmvq, a.K);
    if (mmvq) {
        if (out_kind == OUT_HALF) return launch_k<true, OUT_HALF>(a, grid, lds, st);
        if (out_kind == OUT_F32)  return launch_k<true, OUT_F32>(a, grid, lds, st);
        return launch_k<true, OUT_ADD>(a, grid, lds, st);
    }
    if (out_kind == OUT_HALF) return launch_k<false, OUT_HALF>(a, grid, lds, st);
    if (out_kind == OUT_F32)  return launch_k<false, OUT_F32>(a, grid, lds, st);
    return launch_k<false, OUT_ADD>(a, grid, lds, st);
}

hipError_t quantize_q8_1_aos_launch(const uint16_t* x, void* y, int K, hipStream_t st) {
    const int n = (K / 32) * 8;
    hipLaunchKernelGGL(quantize_q8_1_aos_kernel, dim3((n + GEMV_THREADS - 1) / GEMV_THREADS),
                       dim3(GEMV_THREADS), 0, st, x, (uint8_t*)y, K);
    return hipGetLastError();
}

}  // namespace jllm_hip
