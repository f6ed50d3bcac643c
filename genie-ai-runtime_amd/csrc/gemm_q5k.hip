// gemm_q5k.hip -- batched (prefill) GEMM for Q5_K weights on gfx950.
//
// y[t][r] = sum_k x[t][k] * W[r][k], N tokens x M rows, with the arithmetic
// of the reference's Q5_K batched path (gemm_quant_batched_q5k_kernel,
// gemv_q4.cu:1703-1762): weights dequantised in fp32 as
// dall*sc_j*q - dmin*m_j (q = nibble + 16*qh bit, 0..31) and dotted with the
// fp16 activation in fp32 -- no activation quantisation.  The same sum is
// regrouped per super-block as
//     dall * sum_j sc_j * sum_{k in j} q_k x_k  -  dmin * sum_j m_j * X_j
// (X_j = sum of x over sub-block j):
//   * sc_j * q_k <= 63 * 31 = 1953 is an integer exact in fp16, x is fp16, so
//     v_mfma_f32_32x32x16_f16 forms every product exactly and adds them in
//     fp32 -- one MFMA chain per super-block for the first term;
//   * the min term is one more K = 16 MFMA per super-block: A = the eight
//     6-bit mins (exact) twice, B = X_j / 32 split into fp16 hi + lo
//     (|X - 32(hi + lo)| <= 2^-22 |X|), so it too is fp32-accurate;
//   * dall and dmin (per row and super-block) scale the two MFMA results in
//     fp32, two fma per output element and super-block.
// The result equals the reference's up to fp32 summation order.
//
// Tiling: a workgroup computes 128 rows x 64 tokens (4 waves, each 32 rows x
// 64 tokens = two 32x32 tiles).  A lane's weight bytes go straight from
// global memory to its registers (each weight byte is used by one wave
// only); the activation tile of a super-block (64 tokens x 256 fp16) and
// its sub-block sums are staged in LDS, double-buffered, one barrier per
// super-block; the next super-block's loads are in flight while the current
// one computes.
//
// MFMA K order.  Within a sub-block pair il (64 weights), lane group kg
// (lane / 32) takes qs bytes [32 il + 16 kg, +16): their low nibbles are the
// weights 64 il + 16 kg + [0, 16) and their high nibbles 64 il + 32 + 16 kg +
// [0, 16).  The B operand reads x at the same positions, so each MFMA step
// sums 16 matching (weight, x) pairs; the order of the K axis inside an MFMA
// does not change the sum.
#include "kq_common.h"
#include "mmq.h"

namespace jllm_hip {
namespace {

typedef uint32_t u32x4q __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2q __attribute__((ext_vector_type(2)));
typedef _Float16 h8q __attribute__((ext_vector_type(8)));
typedef float f32x16q __attribute__((ext_vector_type(16)));
typedef float f32x4q __attribute__((ext_vector_type(4)));

constexpr int TM = 128, TN = 64, THREADS = 256;
constexpr int XS = QK_K + 8;          // fp16 per staged token row (16 B pad against bank conflicts)

// 8 code bytes (values 0..31) -> 8 fp16 values times the sub-block scale:
// v_perm_b32 pairs each byte with 0x64 (fp16 1024 + byte), a packed
// subtract removes the bias and a packed multiply applies sc (exact).
__device__ __forceinline__ h8q codes_h8(uint32_t w0, uint32_t w1, _Float16 sc) {
    const uint32_t hi = 0x64646464u;
    u32x4q p;
    p.x = __builtin_amdgcn_perm(hi, w0, 0x04010400u);
    p.y = __builtin_amdgcn_perm(hi, w0, 0x04030402u);
    p.z = __builtin_amdgcn_perm(hi, w1, 0x04010400u);
    p.w = __builtin_amdgcn_perm(hi, w1, 0x04030402u);
    const _Float16 b = (_Float16)1024.0f;
    return (__builtin_bit_cast(h8q, p) - h8q{b, b, b, b, b, b, b, b}) * h8q{sc, sc, sc, sc, sc, sc, sc, sc};
}

__device__ __forceinline__ f32x16q mfma16(h8q a, h8q b, f32x16q c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// The lane's weight bytes of one super-block: header (d, dmin, scales),
// qh bytes [16 kg, +16), qs bytes [32 il + 16 kg, +16) for il = 0..3.
struct ARegs { u32x4q hdr, qh, qs[4]; };

__device__ __forceinline__ void load_a(ARegs& a, const uint8_t* blk, int kg) {
    a.hdr = *(const u32x4q*)blk;
    a.qh = *(const u32x4q*)(blk + 16 + 16 * kg);
#pragma unroll
    for (int il = 0; il < 4; il++) a.qs[il] = *(const u32x4q*)(blk + 48 + 32 * il + 16 * kg);
}

// The thread's share of the activation tile: token t >> 2, fp16 values
// [64 q, 64 q + 64) of the super-block (q = t & 3).
struct XRegs { u32x4q v[8]; };

__device__ __forceinline__ void load_x(XRegs& r, const uint16_t* src) {
#pragma unroll
    for (int i = 0; i < 8; i++) r.v[i] = *(const u32x4q*)(src + 8 * i);
}

// Store the thread's 64 values and the two sub-block sums (X/32 as fp16 hi + lo).
__device__ __forceinline__ void commit_x(const XRegs& r, uint16_t* sx, uint16_t* ss, int tok, int q) {
    uint16_t* dst = sx + tok * XS + 64 * q;
#pragma unroll
    for (int i = 0; i < 8; i++) *(u32x4q*)(dst + 8 * i) = r.v[i];
    const uint32_t one = 0x3C003C00u;
    float s[2] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float t = s[i >> 2];
        t = fdot2(r.v[i].x, one, t); t = fdot2(r.v[i].y, one, t);
        t = fdot2(r.v[i].z, one, t); t = fdot2(r.v[i].w, one, t);
        s[i >> 2] = t;
    }
    uint32_t hi = 0, lo = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const float xs = s[h] * 0.03125f;
        const _Float16 fh = (_Float16)xs;
        const _Float16 fl = (_Float16)(xs - (float)fh);
        hi |= (uint32_t)__builtin_bit_cast(uint16_t, fh) << (16 * h);
        lo |= (uint32_t)__builtin_bit_cast(uint16_t, fl) << (16 * h);
    }
    *(uint32_t*)(ss + tok * 16 + 2 * q) = hi;
    *(uint32_t*)(ss + tok * 16 + 8 + 2 * q) = lo;
}

__device__ __forceinline__ int xcd_tile_q5(int bid, int tiles) {
    const int full = tiles - tiles % 8;
    if (bid >= full) return bid;
    return (bid % 8) * (full / 8) + bid / 8;
}

template <int OUT>   // 0: fp16 y [N][M], 1: fp32 y [N][M]
__global__ __launch_bounds__(THREADS, 2)
void gemm_q5k_kernel(void* __restrict__ y, const uint8_t* __restrict__ W, const uint16_t* __restrict__ x,
                     int M, int N, int K, int sps) {
    __shared__ __attribute__((aligned(16))) uint16_t sX[2][TN * XS];
    __shared__ __attribute__((aligned(16))) uint16_t sS[2][TN * 16];     // per token: X/32 hi [8] | lo [8]
    __shared__ __attribute__((aligned(16))) float sD[4][32 * 2];         // per wave and row: dall, 32*dmin

    const int nb = K / QK_K;
    const int sb0 = (int)blockIdx.y * sps, sb1 = min(nb, sb0 + sps);     // split-K range of super-blocks
    const int n_rt = (M + TM - 1) / TM, n_tt = (N + TN - 1) / TN;
    const int tile = xcd_tile_q5(blockIdx.x, n_rt * n_tt);
    const int row0 = (tile / n_tt) * TM, col0 = (tile % n_tt) * TN;
    const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63, li = l & 31, kg = l >> 5;

    const uint8_t* wrow = W + (int64_t)min(row0 + 32 * w + li, M - 1) * nb * Q5K_BYTES;   // rows past M re-read the last
    const int xtok = t >> 2, xq = t & 3;
    const uint16_t* xsrc = x + (int64_t)min(col0 + xtok, N - 1) * K + 64 * xq;            // tokens past N: the last

    f32x16q acc[2];
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[tt][v] = 0.0f;

    ARegs A, An;
    XRegs Xn;
    load_a(A, wrow + (int64_t)sb0 * Q5K_BYTES, kg);
    load_x(Xn, xsrc + sb0 * QK_K);
    commit_x(Xn, sX[0], sS[0], xtok, xq);
    __syncthreads();

#pragma unroll 1
    for (int b = sb0; b < sb1; b++) {
        const int st = (b - sb0) & 1;
        const bool more = b + 1 < sb1;
        if (more) {
            load_a(An, wrow + (int64_t)(b + 1) * Q5K_BYTES, kg);
            load_x(Xn, xsrc + (b + 1) * QK_K);
        }
        // scales and mins of the 8 sub-blocks
        uint32_t sc[8], mn[8];
#pragma unroll
        for (int j = 0; j < 8; j++) q4k_scale_min(A.hdr.y, A.hdr.z, A.hdr.w, j, sc[j], mn[j]);
        f32x16q C[2], Cm[2];
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int v = 0; v < 16; v++) { C[tt][v] = 0.0f; Cm[tt][v] = 0.0f; }
        const uint16_t* xs = sX[st];
        const uint32_t hq[4] = {A.qh.x, A.qh.y, A.qh.z, A.qh.w};
#pragma unroll
        for (int il = 0; il < 4; il++) {
            const uint32_t q[4] = {A.qs[il].x, A.qs[il].y, A.qs[il].z, A.qs[il].w};
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = (q[i] & 0x0F0F0F0Fu) | (((hq[i] >> (2 * il)) & 0x01010101u) << 4);
                hi[i] = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((hq[i] >> (2 * il + 1)) & 0x01010101u) << 4);
            }
            const _Float16 s_lo = (_Float16)(float)sc[2 * il], s_hi = (_Float16)(float)sc[2 * il + 1];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const uint32_t* src = (s >> 1) ? hi : lo;
                const h8q a = codes_h8(src[2 * (s & 1)], src[2 * (s & 1) + 1], (s >> 1) ? s_hi : s_lo);
                const int k = 64 * il + 32 * (s >> 1) + 16 * kg + 8 * (s & 1);
#pragma unroll
                for (int tt = 0; tt < 2; tt++) {
                    const h8q bv = *(const h8q*)(xs + (32 * tt + li) * XS + k);
                    C[tt] = mfma16(a, bv, C[tt]);
                }
            }
        }
        // min term: A = m_0..m_7 in both lane groups, B = X/32 hi (kg 0) / lo (kg 1)
        h8q am;
#pragma unroll
        for (int j = 0; j < 8; j++) am[j] = (_Float16)(float)mn[j];
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const h8q bs = *(const h8q*)(sS[st] + (32 * tt + li) * 16 + 8 * kg);
            Cm[tt] = mfma16(am, bs, Cm[tt]);
        }
        // per-row dall, 32*dmin to the lanes holding the rows' results
        if (kg == 0) {
            sD[w][2 * li] = f16_bits_to_f32(A.hdr.x & 0xFFFFu);
            sD[w][2 * li + 1] = 32.0f * f16_bits_to_f32(A.hdr.x >> 16);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
        for (int v4 = 0; v4 < 4; v4++) {
            const int r = 8 * v4 + 4 * kg;                       // rows r .. r+3 of the wave
            const f32x4q d01 = *(const f32x4q*)&sD[w][2 * r];
            const f32x4q d23 = *(const f32x4q*)&sD[w][2 * r + 4];
            const float da[4] = {d01.x, d01.z, d23.x, d23.z}, dm[4] = {d01.y, d01.w, d23.y, d23.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
#pragma unroll
                for (int tt = 0; tt < 2; tt++) {
                    acc[tt][4 * v4 + e] = fmaf(da[e], C[tt][4 * v4 + e], acc[tt][4 * v4 + e]);
                    acc[tt][4 * v4 + e] = fmaf(-dm[e], Cm[tt][4 * v4 + e], acc[tt][4 * v4 + e]);
                }
            }
        }
        if (more) {
            commit_x(Xn, sX[st ^ 1], sS[st ^ 1], xtok, xq);
            A = An;
        }
        __syncthreads();
    }

#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
        const int tok = col0 + 32 * tt + li;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = row0 + 32 * w + 8 * (v >> 2) + 4 * kg + (v & 3);
            if (r < M && tok < N) {
                if (OUT == 1) ((float*)y)[(int64_t)blockIdx.y * N * M + (int64_t)tok * M + r] = acc[tt][v];
                else          ((uint16_t*)y)[(int64_t)tok * M + r] = f32_to_f16_bits(acc[tt][v]);
            }
        }
    }
}

}  // namespace

hipError_t gemm_q5k_launch(void* y, const uint8_t* W, const uint16_t* x, int M, int N, int K, int out_kind,
                           int splits, hipStream_t st) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (K <= 0 || K % QK_K != 0) return hipErrorInvalidValue;
    const int nb = K / QK_K;
    const int sps = (nb + splits - 1) / splits;
    if (splits < 1 || (splits > 1 && out_kind != 1) || (splits - 1) * sps >= nb) return hipErrorInvalidValue;
    const int64_t tiles = (int64_t)((M + TM - 1) / TM) * ((N + TN - 1) / TN);
    if (tiles > 0x7FFFFFFF) return hipErrorInvalidValue;
    const dim3 grid((unsigned)tiles, splits);
    if (out_kind == 1) hipLaunchKernelGGL(gemm_q5k_kernel<1>, grid, dim3(THREADS), 0, st, y, W, x, M, N, K, sps);
    else               hipLaunchKernelGGL(gemm_q5k_kernel<0>, grid, dim3(THREADS), 0, st, y, W, x, M, N, K, sps);
    return hipGetLastError();
}

}  // namespace jllm_hip
