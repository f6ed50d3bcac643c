// mmq.hip -- int8 MFMA prefill GEMM for Q4_K / Q6_K weights on gfx950.
//
// y[t][r] = sum_k x[t][k] * W[r][k] for N tokens, M weight rows, with the
// activation quantised to q8_1 in 32-value blocks and every 32-weight (Q4_K)
// or 16-weight (Q6_K) group dotted EXACTLY in int32 by the matrix cores,
// then scaled in fp32 -- the arithmetic of the reference's default prefill
// path (mmq_q4k_llama.cu:92-453, mmq_q6k_llama.cu:71-483, SM 8.x branch):
//   Q4_K: sum += half(d*sc_j) * d8_j * C_j ;  sum += half(-dmin*m_j) * sumx_j
//   Q6_K: per 128-half, tmp += float(C_g0*sc_g0 + C_g1*sc_g1) * d8 (per 32),
//         sum += tmp * d.
//
// Matrix-core mapping: one v_mfma_i32_32x32x32_i8 per (32 rows, 32 tokens,
// Q4_K sub-block) -- K = 32 is exactly one sub-block, so each accumulator
// holds one reference int32 dot; Q6_K uses v_mfma_i32_32x32x16_i8 per 16-group.
// A workgroup computes a 128-row x 64-token tile: per super-block it stages
// the 128 weight blocks and the 64 tokens' q8 codes in LDS (row strides
// padded so the per-lane 16-byte reads are bank-conflict free), each wave
// owns 32 rows x 64 tokens.  Tiles are ordered row-major and handed out so
// that each XCD (blockIdx % 8) works on a contiguous range of row tiles,
// keeping a weight tile in one L2.
#include "kq_common.h"
#include "mmq.h"

namespace jllm_hip {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4m __attribute__((ext_vector_type(4)));
typedef float f32x4m __attribute__((ext_vector_type(4)));

constexpr int MMQ_THREADS = 256;
constexpr int TM = 128;                 // rows per tile
constexpr int TN = MMQ_TILE_N;          // tokens per tile
constexpr int A4_STRIDE = 144;          // LDS bytes per staged Q4_K row block
constexpr int A6_STRIDE = 272;          // LDS bytes per decoded Q6_K row (256 codes + pad)
constexpr int B_STRIDE = 272;           // LDS bytes per token (256 codes + pad)

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

// ---------------------------------------------------------------------------
// tile scheduling

__device__ __forceinline__ int xcd_tile(int bid, int tiles) {
    const int full = tiles - tiles % 8;
    if (bid >= full) return bid;
    return (bid % 8) * (full / 8) + bid / 8;
}

// ---------------------------------------------------------------------------
// B staging (shared by both weight types): the tile's 64 tokens x 256 codes
// of one super-block (two 128-value q8 blocks per token) and their per-32
// scales.  DS4: d8 and sum; D4: d8 only.
template <bool DS4>
__device__ __forceinline__ void stage_b(const uint8_t* __restrict__ q8, int Npad, int col0, int b,
                                        uint8_t* sB, float* sD8, float* sSX) {
    const int t = threadIdx.x;
#pragma unroll
    for (int it = 0; it < (TN * 16) / MMQ_THREADS; it++) {
        const int c = it * MMQ_THREADS + t;          // chunk: token c/16, 16-byte piece c%16
        const int tok = c >> 4, piece = c & 15, half = piece >> 3;
        const uint8_t* src = q8 + ((int64_t)(2 * b + half) * Npad + col0 + tok) * 144 + 16 + (piece & 7) * 16;
        *(u32x4m*)(sB + tok * B_STRIDE + piece * 16) = *(const u32x4m*)src;
    }
    if (t < TN * 2) {                                // 64 tokens x 2 q8 blocks: scales
        const int tok = t >> 1, half = t & 1;
        const u32x4m w = *(const u32x4m*)(q8 + ((int64_t)(2 * b + half) * Npad + col0 + tok) * 144);
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int j = half * 4 + s;
            if (DS4) {
                sD8[j * TN + tok] = f16_bits_to_f32(ww[s] & 0xFFFFu);
                sSX[j * TN + tok] = f16_bits_to_f32(ww[s] >> 16);
            } else {
                sD8[j * TN + tok] = __builtin_bit_cast(float, ww[s]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_K

template <int OUT>
__global__ __launch_bounds__(MMQ_THREADS, 2)
void mmq_q4k_kernel(void* __restrict__ y, const uint8_t* __restrict__ W, const uint8_t* __restrict__ q8,
                    int M, int N, int K, int Npad) {
    __shared__ __attribute__((aligned(16))) uint8_t sA[TM * A4_STRIDE];
    __shared__ __attribute__((aligned(16))) float sDA[8 * TM];     // half(d*sc) per [j][row]
    __shared__ __attribute__((aligned(16))) float sMA[8 * TM];     // half(-dmin*m) per [j][row]
    __shared__ __attribute__((aligned(16))) uint8_t sB[TN * B_STRIDE];
    __shared__ __attribute__((aligned(16))) float sD8[8 * TN];
    __shared__ __attribute__((aligned(16))) float sSX[8 * TN];

    const int nb = K / QK_K;
    const int n_rt = (M + TM - 1) / TM, n_tt = Npad / TN;
    const int tile = xcd_tile(blockIdx.x, n_rt * n_tt);
    const int row0 = (tile / n_tt) * TM, col0 = (tile % n_tt) * TN;
    const int t = threadIdx.x, w = t >> 6, l = t & 63, li = l & 31, g = l >> 5;

    float acc[2][16];
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[nt][v] = 0.0f;

    for (int b = 0; b < nb; b++) {
        // stage the 128 weight blocks (rows past M re-read the last row)
        for (int c = t; c < TM * 9; c += MMQ_THREADS) {
            const int row = c / 9, piece = c % 9;
            const int R = min(row0 + row, M - 1);
            *(u32x4m*)(sA + row * A4_STRIDE + piece * 16) =
                *(const u32x4m*)(W + ((int64_t)R * nb + b) * Q4K_BYTES + piece * 16);
        }
        if (t < TM) {    // per-row sub-block scales, rounded to half as the reference does
            const int R = min(row0 + t, M - 1);
            const u32x4m h = *(const u32x4m*)(W + ((int64_t)R * nb + b) * Q4K_BYTES);
            const float d = f16_bits_to_f32(h.x & 0xFFFFu), dmin = f16_bits_to_f32(h.x >> 16);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint32_t sc, m;
                q4k_scale_min(h.y, h.z, h.w, j, sc, m);
                sDA[j * TM + t] = round_to_f16(d * (float)sc);
                sMA[j * TM + t] = round_to_f16(-dmin * (float)m);
            }
        }
        stage_b<true>(q8, Npad, col0, b, sB, sD8, sSX);
        __syncthreads();

#pragma unroll 1
        for (int jj = 0; jj < 4; jj++) {
            // A: 16 packed bytes = the lane's 16 K positions of sub-blocks 2jj (low
            // nibbles) and 2jj+1 (high nibbles) for row 32w + li
            const u32x4m a = *(const u32x4m*)(sA + (32 * w + li) * A4_STRIDE + 16 + 32 * jj + 16 * g);
            const u32x4m M4 = {0x0F0F0F0Fu, 0x0F0F0F0Fu, 0x0F0F0F0Fu, 0x0F0F0F0Fu};
            const i32x4 alo = __builtin_bit_cast(i32x4, a & M4);
            const i32x4 ahi = __builtin_bit_cast(i32x4, (a >> 4) & M4);
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const int j = 2 * jj + p;
                i32x16 C[2];
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const i32x4 bv = *(const i32x4*)(sB + (32 * nt + li) * B_STRIDE + 32 * j + 16 * g);
                    const i32x16 zero = {};
                    C[nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(p ? ahi : alo, bv, zero, 0, 0, 0);
                }
                // rows of this lane's accumulators: 32w + 8m + 4g + (0..3)
                f32x4m da[4], ma[4];
#pragma unroll
                for (int m4 = 0; m4 < 4; m4++) {
                    da[m4] = *(const f32x4m*)(sDA + j * TM + 32 * w + 8 * m4 + 4 * g);
                    ma[m4] = *(const f32x4m*)(sMA + j * TM + 32 * w + 8 * m4 + 4 * g);
                }
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const float db = sD8[j * TN + 32 * nt + li], sx = sSX[j * TN + 32 * nt + li];
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        if (OUT == 2) continue;
                        const float dav = da[v >> 2][v & 3], mav = ma[v >> 2][v & 3];
                        acc[nt][v] += dav * db * (float)C[nt][v];
                        acc[nt][v] += mav * sx;
                    }
                    if (OUT == 2) {   // raw dots [N][M][K/32]
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const int r = row0 + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3);
                            const int tok = col0 + 32 * nt + li;
                            if (r < M && tok < N)
                                ((int*)y)[((int64_t)tok * M + r) * (K / 32) + b * 8 + j] = C[nt][v];
                        }
                    }
                }
            }
        }
        __syncthreads();
    }
    if (OUT == 2) return;
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int tok = col0 + 32 * nt + li;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = row0 + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3);
            if (r < M && tok < N) {
                if (OUT == 1) ((float*)y)[(int64_t)tok * M + r] = acc[nt][v];
                else          ((uint16_t*)y)[(int64_t)tok * M + r] = f32_to_f16_bits(acc[nt][v]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q6_K

typedef float f32x4q6 __attribute__((ext_vector_type(4)));

template <int OUT>
__global__ __launch_bounds__(MMQ_THREADS, 2)
void mmq_q6k_kernel(void* __restrict__ y, const uint8_t* __restrict__ W, const uint8_t* __restrict__ q8,
                    int M, int N, int K, int Npad) {
    __shared__ __attribute__((aligned(16))) uint8_t sA[TM * A6_STRIDE];   // decoded codes q-32 (int8)
    __shared__ __attribute__((aligned(16))) int sSC[16 * TM];             // int8 scales per [group][row]
    __shared__ __attribute__((aligned(16))) float sDA[TM];                // d per row
    __shared__ __attribute__((aligned(16))) uint8_t sB[TN * B_STRIDE];
    __shared__ __attribute__((aligned(16))) float sD8[8 * TN];

    const int nb = K / QK_K;
    const int n_rt = (M + TM - 1) / TM, n_tt = Npad / TN;
    const int tile = xcd_tile(blockIdx.x, n_rt * n_tt);
    const int row0 = (tile / n_tt) * TM, col0 = (tile % n_tt) * TN;
    const int t = threadIdx.x, w = t >> 6, l = t & 63, li = l & 31, g = l >> 5;

    float acc[2][16];
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[nt][v] = 0.0f;

    for (int b = 0; b < nb; b++) {
        // decode: unit = (row, 16-element group n16) -> 16 codes; elements
        // e = 16*n16 + i share the half h, quarter qq and 16 consecutive l.
        for (int u = t; u < TM * 16; u += MMQ_THREADS) {
            const int row = u >> 4, n16 = u & 15;
            const int R = min(row0 + row, M - 1);
            const uint8_t* blk = W + ((int64_t)R * nb + b) * Q6K_BYTES;
            const int e0 = 16 * n16, h = e0 >> 7, ph = e0 & 127, qq = ph >> 5, l0 = ph & 31;
            const uint8_t* pl = blk + 64 * h + l0 + 32 * (qq & 1);
            const uint8_t* ph2 = blk + 128 + 32 * h + l0;
            const uint32_t sh = (uint32_t)((uintptr_t)blk & 2u) * 8u;
            const uint8_t* bl = pl - ((uintptr_t)pl & 3u);
            const uint8_t* bh = ph2 - ((uintptr_t)ph2 & 3u);
            uint32_t ql[4], qh[4];
            {
                const uint32_t* s0 = (const uint32_t*)bl;
                const uint32_t* s1 = (const uint32_t*)bh;
                uint32_t a[5], c[5];
#pragma unroll
                for (int k = 0; k < 5; k++) { a[k] = s0[k]; c[k] = s1[k]; }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    ql[k] = __builtin_amdgcn_alignbit(a[k + 1], a[k], sh);
                    qh[k] = __builtin_amdgcn_alignbit(c[k + 1], c[k], sh);
                }
            }
            u32x4m codes;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t lo = ((qq >= 2 ? (ql[k] >> 4) : ql[k]) & 0x0F0F0F0Fu);
                const uint32_t hb = (qh[k] >> (2 * qq)) & 0x03030303u;
                const uint32_t v = lo | (hb << 4);
                codes[k] = ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;   // bytewise v - 32
            }
            *(u32x4m*)(sA + row * A6_STRIDE + 16 * n16) = codes;
        }
        if (t < TM) {
            const int R = min(row0 + t, M - 1);
            const uint8_t* blk = W + ((int64_t)R * nb + b) * Q6K_BYTES;
#pragma unroll
            for (int gi = 0; gi < 16; gi++) sSC[gi * TM + t] = (int)(int8_t)blk[192 + gi];
            sDA[t] = f16_bits_to_f32(*(const uint16_t*)(blk + 208));
        }
        stage_b<false>(q8, Npad, col0, b, sB, sD8, nullptr);
        __syncthreads();

        f32x4q6 dA[4];
#pragma unroll
        for (int m4 = 0; m4 < 4; m4++) dA[m4] = *(const f32x4q6*)(sDA + 32 * w + 8 * m4 + 4 * g);
#pragma unroll 1
        for (int hh = 0; hh < 2; hh++) {
            float tmp[2][16];
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int v = 0; v < 16; v++) tmp[nt][v] = 0.0f;
#pragma unroll 1
            for (int s = 0; s < 4; s++) {
                const int j = 4 * hh + s;                          // 32-wide block within the super-block
                const int64_t a0 = *(const int64_t*)(sA + (32 * w + li) * A6_STRIDE + 32 * j + 8 * g);
                const int64_t a1 = *(const int64_t*)(sA + (32 * w + li) * A6_STRIDE + 32 * j + 16 + 8 * g);
                i32x4 sc0[4], sc1[4];
#pragma unroll
                for (int m4 = 0; m4 < 4; m4++) {
                    sc0[m4] = *(const i32x4*)(sSC + (2 * j) * TM + 32 * w + 8 * m4 + 4 * g);
                    sc1[m4] = *(const i32x4*)(sSC + (2 * j + 1) * TM + 32 * w + 8 * m4 + 4 * g);
                }
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const int64_t b0 = *(const int64_t*)(sB + (32 * nt + li) * B_STRIDE + 32 * j + 8 * g);
                    const int64_t b1 = *(const int64_t*)(sB + (32 * nt + li) * B_STRIDE + 32 * j + 16 + 8 * g);
                    const i32x16 zero = {};
                    const i32x16 C0 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a0, b0, zero, 0, 0, 0);
                    const i32x16 C1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a1, b1, zero, 0, 0, 0);
                    const float db = sD8[j * TN + 32 * nt + li];
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        if (OUT == 2) {
                            const int r = row0 + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3);
                            const int tok = col0 + 32 * nt + li;
                            if (r < M && tok < N) {
                                int* o = (int*)y + ((int64_t)tok * M + r) * (K / 16) + b * 16 + 2 * j;
                                o[0] = C0[v]; o[1] = C1[v];
                            }
                        } else {
                            const int iv = C0[v] * sc0[v >> 2][v & 3] + C1[v] * sc1[v >> 2][v & 3];
                            tmp[nt][v] += (float)iv * db;
                        }
                    }
                }
            }
            if (OUT != 2) {
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[nt][v] += tmp[nt][v] * dA[v >> 2][v & 3];
            }
        }
        __syncthreads();
    }
    if (OUT == 2) return;
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int tok = col0 + 32 * nt + li;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = row0 + 32 * w + 8 * (v >> 2) + 4 * g + (v & 3);
            if (r < M && tok < N) {
                if (OUT == 1) ((float*)y)[(int64_t)tok * M + r] = acc[nt][v];
                else          ((uint16_t*)y)[(int64_t)tok * M + r] = f32_to_f16_bits(acc[nt][v]);
            }
        }
    }
}

hipError_t mmq_launch(void* y, const uint8_t* W, int type, const void* q8, int M, int N, int K, int Npad,
                      int out_kind, hipStream_t st) {
    const int tiles = ((M + TM - 1) / TM) * (Npad / TN);
    const uint8_t* q = (const uint8_t*)q8;
    if (type == TYPE_Q4_K) {
        if (out_kind == 0) hipLaunchKernelGGL(mmq_q4k_kernel<0>, dim3(tiles), dim3(MMQ_THREADS), 0, st, y, W, q, M, N, K, Npad);
        else if (out_kind == 1) hipLaunchKernelGGL(mmq_q4k_kernel<1>, dim3(tiles), dim3(MMQ_THREADS), 0, st, y, W, q, M, N, K, Npad);
        else hipLaunchKernelGGL(mmq_q4k_kernel<2>, dim3(tiles), dim3(MMQ_THREADS), 0, st, y, W, q, M, N, K, Npad);
    } else {
        if (out_kind == 0) hipLaunchKernelGGL(mmq_q6k_kernel<0>, dim3(tiles), dim3(MMQ_THREADS), 0, st, y, W, q, M, N, K, Npad);
        else if (out_kind == 1) hipLaunchKernelGGL(mmq_q6k_kernel<1>, dim3(tiles), dim3(MMQ_THREADS), 0, st, y, W, q, M, N, K, Npad);
        else hipLaunchKernelGGL(mmq_q6k_kernel<2>, dim3(tiles), dim3(MMQ_THREADS), 0, st, y, W, q, M, N, K, Npad);
    }
    return hipGetLastError();
}

}  // namespace jllm_hip
