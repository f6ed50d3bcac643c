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

namespace jllm_hip {

constexpr int GEMV_THREADS = 256;

// ---- activation staging -------------------------------------------------

// Quantise 32 fp16 values to q8_1 with 8 cooperating lanes (4 values each):
// d = amax/127, q = rn(v*(1/d)) clamped to +-127, s = d*sum(q).
// Returns the 4 packed codes; d/s via ds_out (valid on every lane).
__device__ __forceinline__ uint32_t quant_q8_1_x4(uint2 raw, uint32_t& ds_out) {
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
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) sumq += __shfl_xor(sumq, o, 64);
    ds_out = (uint32_t)f32_to_f16_bits(d) | ((uint32_t)f32_to_f16_bits(d * (float)sumq) << 16);
    return packed;
}

// q8_1 in LDS as SoA: codes s_q[K] then (d,s) words s_ds[K/32]
__device__ __forceinline__ void stage_q8_1(const uint16_t* __restrict__ x, int K,
                                           int8_t* s_q, uint32_t* s_ds) {
    const int n = (K / 32) * 8;
    for (int t = threadIdx.x; t < n; t += GEMV_THREADS) {
        const int blk = t >> 3, sub = t & 7;
        const uint2 raw = *(const uint2*)(x + blk * 32 + sub * 4);
        uint32_t ds;
        const uint32_t packed = quant_q8_1_x4(raw, ds);
        *(uint32_t*)(s_q + blk * 32 + sub * 4) = packed;
        if (sub == 0) s_ds[blk] = ds;
    }
}

// fp16 x in LDS plus the fp32 sum of every 16-value chunk (for the Q4_K min term)
__device__ __forceinline__ void stage_f16(const uint16_t* __restrict__ x, int K,
                                          uint16_t* s_x, float* s_xs) {
    const int n = K / 16;
    for (int t = threadIdx.x; t < n; t += GEMV_THREADS) {
        const uint4 a = *(const uint4*)(x + t * 16);
        const uint4 b = *(const uint4*)(x + t * 16 + 8);
        *(uint4*)(s_x + t * 16) = a;
        *(uint4*)(s_x + t * 16 + 8) = b;
        const uint32_t one = 0x3C003C00u;
        float s = 0.0f;
        s = fdot2(a.x, one, s); s = fdot2(a.y, one, s); s = fdot2(a.z, one, s); s = fdot2(a.w, one, s);
        s = fdot2(b.x, one, s); s = fdot2(b.y, one, s); s = fdot2(b.z, one, s); s = fdot2(b.w, one, s);
        s_xs[t] = s;
    }
}

// ---- per-block lane work -------------------------------------------------

// MMVQ, Q4_K: octet lane o8 holds qs bytes [16*o8, 16*o8+16): low nibbles are
// 16 weights of sub-block 2*il, high nibbles 16 weights of sub-block 2*il+1
// (il = o8/2).  The pair (o8, o8^1) completes both 32-weight int32 dots; lane
// with part 0 applies the fp32 epilogue of the low sub-block, part 1 the high.
__device__ __forceinline__ float q4k_mmvq_block(const uint8_t* __restrict__ blk, int b, int o8,
                                                const int8_t* s_q, const uint32_t* s_ds) {
    const uint4 hdr = *(const uint4*)blk;
    const uint4 q = *(const uint4*)(blk + 16 + 16 * o8);
    const int il = o8 >> 1, part = o8 & 1;
    const int j0 = 2 * il;
    const uint4 xl = *(const uint4*)(s_q + (b * 8 + j0) * 32 + 16 * part);
    const uint4 xh = *(const uint4*)(s_q + (b * 8 + j0 + 1) * 32 + 16 * part);
    const uint32_t M = 0x0F0F0F0Fu;
    int dl = sdot4(q.x & M, xl.x, 0);
    dl = sdot4(q.y & M, xl.y, dl); dl = sdot4(q.z & M, xl.z, dl); dl = sdot4(q.w & M, xl.w, dl);
    int dh = sdot4((q.x >> 4) & M, xh.x, 0);
    dh = sdot4((q.y >> 4) & M, xh.y, dh); dh = sdot4((q.z >> 4) & M, xh.z, dh); dh = sdot4((q.w >> 4) & M, xh.w, dh);
    const int recv = swap_lane1(part ? dl : dh);
    const int dot = (part ? dh : dl) + recv;
    const int j = j0 + part;
    uint32_t sc, m;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, m);
    const uint32_t ds = s_ds[b * 8 + j];
    const float dall = f16_bits_to_f32(hdr.x & 0xFFFFu), dmin = f16_bits_to_f32(hdr.x >> 16);
    const float d8 = f16_bits_to_f32(ds & 0xFFFFu), s8 = f16_bits_to_f32(ds >> 16);
    return dall * (float)sc * (d8 * (float)dot) - dmin * (float)m * s8;
}

// Q6_K lane slice: octet lane o8 -> half h = o8/4 of the block, positions
// l0..l0+7 (l0 = 8*(o8&3)) of each of the four 32-wide quarters g, i.e.
// elements h*128 + 32*g + l0 + [0,8).  v[g] holds the 8 raw 6-bit codes.
struct Q6Slice { uint2 v[4]; uint2 sc; float d; };

__device__ __forceinline__ Q6Slice q6k_load_slice(const uint8_t* __restrict__ blk, int o8) {
    const int h = o8 >> 2, l0 = 8 * (o8 & 3);
    const uint2 qa = load8_a2(blk + h * 64 + l0);
    const uint2 qb = load8_a2(blk + h * 64 + 32 + l0);
    const uint2 qh = load8_a2(blk + 128 + h * 32 + l0);
    Q6Slice s;
    s.sc = load8_a2(blk + 192 + 8 * h);
    s.d = f16_bits_to_f32(*(const uint16_t*)(blk + 208));
    const uint32_t M4 = 0x0F0F0F0Fu, M2 = 0x03030303u;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const uint2 src = (g & 1) ? qb : qa;
        const int ns = (g >= 2) ? 4 : 0;
        s.v[g].x = ((src.x >> ns) & M4) | (((qh.x >> (2 * g)) & M2) << 4);
        s.v[g].y = ((src.y >> ns) & M4) | (((qh.y >> (2 * g)) & M2) << 4);
    }
    return s;
}

__device__ __forceinline__ int q6_scale(const Q6Slice& s, int o8, int g) {
    const int idx = ((o8 & 3) >> 1) + 2 * g;                 // 0..7 within scales[8h..8h+8)
    const uint32_t w = idx < 4 ? s.sc.x : s.sc.y;
    return (int)(int8_t)((w >> (8 * (idx & 3))) & 0xFFu);
}

__device__ __forceinline__ float q6k_mmvq_block(const uint8_t* __restrict__ blk, int b, int o8,
                                                const int8_t* s_q, const uint32_t* s_ds) {
    const Q6Slice s = q6k_load_slice(blk, o8);
    const int h = o8 >> 2, l0 = 8 * (o8 & 3);
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int qb = b * 8 + 4 * h + g;
        const uint2 xv = *(const uint2*)(s_q + qb * 32 + l0);
        const int dot = sdot4(sub32_bytes(s.v[g].x), xv.x, sdot4(sub32_bytes(s.v[g].y), xv.y, 0));
        const float d8 = f16_bits_to_f32(s_ds[qb] & 0xFFFFu);
        acc += s.d * (float)q6_scale(s, o8, g) * (d8 * (float)dot);
    }
    return acc;
}

// float dequant, Q4_K: same lane slice as the MMVQ path.  Codes become exact
// fp16 values by OR-ing them into the mantissa of 1024.0 and subtracting
// 1024 (high nibbles land as 16*q, undone by a 1/16 factor on the scale).
__device__ __forceinline__ float q4k_f16_block(const uint8_t* __restrict__ blk, int b, int o8,
                                               const uint16_t* s_x, const float* s_xs) {
    const uint4 hdr = *(const uint4*)blk;
    const uint4 q = *(const uint4*)(blk + 16 + 16 * o8);
    const int il = o8 >> 1, part = o8 & 1;
    const int j0 = 2 * il;
    const int k_lo = b * 256 + 64 * il + 16 * part;
    const uint4 xa = *(const uint4*)(s_x + k_lo), xb = *(const uint4*)(s_x + k_lo + 8);
    const uint4 ya = *(const uint4*)(s_x + k_lo + 32), yb = *(const uint4*)(s_x + k_lo + 40);
    const uint32_t xl[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    const uint32_t xh[8] = {ya.x, ya.y, ya.z, ya.w, yb.x, yb.y, yb.z, yb.w};
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    const half2_t bias = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    float sl = 0.0f, sh = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t p01 = __builtin_amdgcn_perm(qw[i], qw[i], 0x0C010C00u);
        const uint32_t p23 = __builtin_amdgcn_perm(qw[i], qw[i], 0x0C030C02u);
        const uint32_t l01 = h2_bits(as_h2((p01 & 0x000F000Fu) | 0x64006400u) + bias);
        const uint32_t l23 = h2_bits(as_h2((p23 & 0x000F000Fu) | 0x64006400u) + bias);
        const uint32_t h01 = h2_bits(as_h2((p01 & 0x00F000F0u) | 0x64006400u) + bias);
        const uint32_t h23 = h2_bits(as_h2((p23 & 0x00F000F0u) | 0x64006400u) + bias);
        sl = fdot2(l01, xl[2 * i], sl); sl = fdot2(l23, xl[2 * i + 1], sl);
        sh = fdot2(h01, xh[2 * i], sh); sh = fdot2(h23, xh[2 * i + 1], sh);
    }
    uint32_t sc1, m1, sc2, m2;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, j0, sc1, m1);
    q4k_scale_min(hdr.y, hdr.z, hdr.w, j0 + 1, sc2, m2);
    const float dall = f16_bits_to_f32(hdr.x & 0xFFFFu), dmin = f16_bits_to_f32(hdr.x >> 16);
    const float xs_lo = s_xs[k_lo >> 4], xs_hi = s_xs[(k_lo + 32) >> 4];
    return (dall * (float)sc1) * sl - (dmin * (float)m1) * xs_lo
         + (dall * (float)sc2 * 0.0625f) * sh - (dmin * (float)m2) * xs_hi;
}

__device__ __forceinline__ float q6k_f16_block(const uint8_t* __restrict__ blk, int b, int o8,
                                               const uint16_t* s_x) {
    const Q6Slice s = q6k_load_slice(blk, o8);
    const int h = o8 >> 2, l0 = 8 * (o8 & 3);
    const half2_t bias = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const uint4 xv = *(const uint4*)(s_x + b * 256 + h * 128 + 32 * g + l0);
        const uint32_t w0 = s.v[g].x, w1 = s.v[g].y;
        const uint32_t a0 = h2_bits(as_h2(__builtin_amdgcn_perm(w0, w0, 0x0C010C00u) | 0x64006400u) + bias);
        const uint32_t a1 = h2_bits(as_h2(__builtin_amdgcn_perm(w0, w0, 0x0C030C02u) | 0x64006400u) + bias);
        const uint32_t a2 = h2_bits(as_h2(__builtin_amdgcn_perm(w1, w1, 0x0C010C00u) | 0x64006400u) + bias);
        const uint32_t a3 = h2_bits(as_h2(__builtin_amdgcn_perm(w1, w1, 0x0C030C02u) | 0x64006400u) + bias);
        float sg = fdot2(a0, xv.x, 0.0f);
        sg = fdot2(a1, xv.y, sg); sg = fdot2(a2, xv.z, sg); sg = fdot2(a3, xv.w, sg);
        acc += (s.d * (float)q6_scale(s, o8, g)) * sg;
    }
    return acc;
}

template <bool MMVQ, int TYPE>
__device__ __forceinline__ float row_partial(const uint8_t* __restrict__ rowp, int nb, int oct, int noct,
                                             int o8, const void* lds_a, const void* lds_b) {
    float acc = 0.0f;
    constexpr int BB = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;

    for (int b = oct; b < nb; b += noct) {
        const uint8_t* blk = rowp + (int64_t)b * BB;
        if (MMVQ) {
            if (TYPE == TYPE_Q4_K) acc += q4k_mmvq_block(blk, b, o8, (const int8_t*)lds_a, (const uint32_t*)lds_b);
            else                   acc += q6k_mmvq_block(blk, b, o8, (const int8_t*)lds_a, (const uint32_t*)lds_b);
        } else {
            if (TYPE == TYPE_Q4_K) acc += q4k_f16_block(blk, b, o8, (const uint16_t*)lds_a, (const float*)lds_b);
            else                   acc += q6k_f16_block(blk, b, o8, (const uint16_t*)lds_a);
        }
    }
    return acc;
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

template <bool MMVQ, int LPR, int OUT, int T0, int T1, int T2>
__global__ __launch_bounds__(GEMV_THREADS)
void gemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int K = a.K;
    void* lds_a = lds;
    void* lds_b = lds + (MMVQ ? K : 2 * K);
    if (MMVQ) stage_q8_1(a.x, K, (int8_t*)lds_a, (uint32_t*)lds_b);
    else      stage_f16(a.x, K, (uint16_t*)lds_a, (float*)lds_b);
    __syncthreads();

    constexpr int RPW = 64 / LPR, NOCT = LPR / 8;
    const int lane = threadIdx.x & 63;
    const int wave = (blockIdx.x * GEMV_THREADS + threadIdx.x) >> 6;
    const int row = wave * RPW + lane / LPR;
    if (row >= a.total_rows) return;
    const int lir = lane % LPR, oct = lir >> 3, o8 = lane & 7;
    const int nb = K / QK_K;

    int s = 0, r = row;
    if (r >= a.seg[0].M) { r -= a.seg[0].M; s = 1; if (r >= a.seg[1].M) { r -= a.seg[1].M; s = 2; } }
    const GemvSeg& sg = a.seg[s];
    float acc;
    if (s == 0) {
        acc = row_partial<MMVQ, T0>(sg.W + (int64_t)r * nb * (T0 == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES), nb, oct, NOCT, o8, lds_a, lds_b);
    } else if (s == 1) {
        acc = row_partial<MMVQ, T1>(sg.W + (int64_t)r * nb * (T1 == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES), nb, oct, NOCT, o8, lds_a, lds_b);
    } else {
        acc = row_partial<MMVQ, T2>(sg.W + (int64_t)r * nb * (T2 == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES), nb, oct, NOCT, o8, lds_a, lds_b);
    }
    acc = group_sum<LPR>(acc);
    if (lir == 0) store_row<OUT>(sg, r, acc);
}

// Standalone q8_1 quantiser in the reference's AoS block layout
// (block_q8_1 {u16 d, u16 s, i8 qs[32]}, gemv_q4.cu:434-466).
__global__ __launch_bounds__(GEMV_THREADS)
void quantize_q8_1_aos_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ y, int K) {
    const int t = blockIdx.x * GEMV_THREADS + threadIdx.x;
    const int n = (K / 32) * 8;
    const bool live = t < n;
    const int blk = live ? t >> 3 : 0, sub = t & 7;
    const uint2 raw = live ? *(const uint2*)(x + blk * 32 + sub * 4) : make_uint2(0, 0);
    uint32_t ds;
    const uint32_t packed = quant_q8_1_x4(raw, ds);
    if (!live) return;
    uint8_t* out = y + (int64_t)blk * 36;
    *(uint32_t*)(out + 4 + 4 * sub) = packed;
    if (sub == 0) *(uint32_t*)out = ds;
}

// ---- host launchers ----------------------------------------------------

static int pick_lpr(int rows) {
    if (rows >= 32768) return 8;
    if (rows >= 16384) return 16;
    if (rows >= 8192) return 32;
    return 64;
}

size_t gemv_lds_bytes(bool mmvq, int K) {
    return mmvq ? (size_t)K + (size_t)(K / 32) * 4 : (size_t)K * 2 + (size_t)(K / 16) * 4;
}

template <bool MMVQ, int OUT, int T0, int T1, int T2>
static hipError_t launch_typed(const GemvArgs& a, int lpr, hipStream_t st) {
    const size_t lds = gemv_lds_bytes(MMVQ, a.K);
    const int64_t waves = ((int64_t)a.total_rows * lpr + 63) / 64;
    const int grid = (int)((waves + 3) / 4);
    switch (lpr) {
        case 8:  hipLaunchKernelGGL((gemv_kernel<MMVQ, 8, OUT, T0, T1, T2>), dim3(grid), dim3(GEMV_THREADS), lds, st, a); break;
        case 16: hipLaunchKernelGGL((gemv_kernel<MMVQ, 16, OUT, T0, T1, T2>), dim3(grid), dim3(GEMV_THREADS), lds, st, a); break;
        case 32: hipLaunchKernelGGL((gemv_kernel<MMVQ, 32, OUT, T0, T1, T2>), dim3(grid), dim3(GEMV_THREADS), lds, st, a); break;
        default: hipLaunchKernelGGL((gemv_kernel<MMVQ, 64, OUT, T0, T1, T2>), dim3(grid), dim3(GEMV_THREADS), lds, st, a); break;
    }
    return hipGetLastError();
}

template <bool MMVQ, int OUT>
static hipError_t launch_out(const GemvArgs& a, int lpr, hipStream_t st) {
    const int t0 = a.seg[0].type;
    const int t1 = a.nseg > 1 ? a.seg[1].type : t0;
    const int t2 = a.nseg > 2 ? a.seg[2].type : t1;
    const int code = (t0 == TYPE_Q6_K) * 4 + (t1 == TYPE_Q6_K) * 2 + (t2 == TYPE_Q6_K);
    constexpr int A = TYPE_Q4_K, B = TYPE_Q6_K;
    switch (code) {
        case 0: return launch_typed<MMVQ, OUT, A, A, A>(a, lpr, st);
        case 1: return launch_typed<MMVQ, OUT, A, A, B>(a, lpr, st);
        case 2: return launch_typed<MMVQ, OUT, A, B, A>(a, lpr, st);
        case 3: return launch_typed<MMVQ, OUT, A, B, B>(a, lpr, st);
        case 4: return launch_typed<MMVQ, OUT, B, A, A>(a, lpr, st);
        case 5: return launch_typed<MMVQ, OUT, B, A, B>(a, lpr, st);
        case 6: return launch_typed<MMVQ, OUT, B, B, A>(a, lpr, st);
        default: return launch_typed<MMVQ, OUT, B, B, B>(a, lpr, st);
    }
}

hipError_t gemv_launch(const GemvArgs& a_in, bool mmvq, int out_kind, int lpr_override, hipStream_t st) {
    GemvArgs a = a_in;
    a.total_rows = 0;
    for (int i = 0; i < a.nseg; i++) a.total_rows += a.seg[i].M;
    for (int i = a.nseg; i < 3; i++) { a.seg[i] = a.seg[a.nseg - 1]; a.seg[i].M = 0; }
    if (a.total_rows <= 0) return hipSuccess;
    const int lpr = lpr_override ? lpr_override : pick_lpr(a.total_rows);
    if (mmvq) {
        if (out_kind == OUT_HALF) return launch_out<true, OUT_HALF>(a, lpr, st);
        if (out_kind == OUT_F32)  return launch_out<true, OUT_F32>(a, lpr, st);
        return launch_out<true, OUT_ADD>(a, lpr, st);
    }
    if (out_kind == OUT_HALF) return launch_out<false, OUT_HALF>(a, lpr, st);
    if (out_kind == OUT_F32)  return launch_out<false, OUT_F32>(a, lpr, st);
    return launch_out<false, OUT_ADD>(a, lpr, st);
}

hipError_t quantize_q8_1_aos_launch(const uint16_t* x, void* y, int K, hipStream_t st) {
    const int n = (K / 32) * 8;
    hipLaunchKernelGGL(quantize_q8_1_aos_kernel, dim3((n + GEMV_THREADS - 1) / GEMV_THREADS),
                       dim3(GEMV_THREADS), 0, st, x, (uint8_t*)y, K);
    return hipGetLastError();
}

}  // namespace jllm_hip
