// attention.hip -- split-K ("flash-decoding") single-query attention over an
// INT8 (or FP16) KV cache, gfx950.
//
// Semantics follow flash_decode_splitk_partial_kernel + flash_decode_reduce_kernel
// (attention.cu:837-969): the key range [0, seq) is cut into n_splits
// contiguous slices of ceil(seq/n_splits) positions; each slice keeps an
// online softmax over 64-key tiles (running max m starting at -FLT_MAX,
// correction expf(m_old - m_new)) and writes the unnormalised (m, l, acc);
// the reduce combines slices with weights e^(m_s - M).  Scores are
// (q . k) * ks[pos][kv_head] * scale, values v * vs[pos][kv_head]; with a
// sliding window, positions < seq - window are excluded (they contribute
// exactly zero in the reference).
//
// MI355X mapping: one workgroup per (KV head, split) computes ALL query
// heads of its GQA group, so each KV byte is read from HBM once.  A 64-key
// tile of K and V (int8 -> 16 KB) is staged in LDS, the next tile's loads
// are in flight while the current one is computed.  Q.K^T and P.V run on
// the matrix cores (v_mfma_f32_32x32x16_f16): int8 keys/values become fp16
// exactly, q is fp16 already, and the fp32 probabilities (times vs) are
// split into a high and a low fp16 part stacked as extra rows of the A
// operand, so the P.V products keep ~22 bits.
#include <float.h>
#include "kq_common.h"
#include "attention.h"

namespace jllm_hip {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));

constexpr int AT_THREADS = 256;
constexpr int AT_TILE = 64;          // keys per tile
constexpr int AT_MAXHD = 128;
constexpr int AT_MAXG = 16;          // max query heads per KV head

// 4 signed int8 (one word) -> 4 exact fp16 values (two words): with u = b ^ 0x80
// in [1, 255], the half with bits 0x6400 + u is 1024 + u, minus 1152 gives b.
__device__ __forceinline__ u32x2a i8x4_to_h4(uint32_t w) {
    const half2_t bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t p01 = __builtin_amdgcn_perm(w, w, 0x0C010C00u);
    const uint32_t p23 = __builtin_amdgcn_perm(w, w, 0x0C030C02u);
    const uint32_t a = (p01 ^ 0x00800080u) + 0x64006400u;
    const uint32_t b = (p23 ^ 0x00800080u) + 0x64006400u;
    return u32x2a{h2_bits(as_h2(a) + bias), h2_bits(as_h2(b) + bias)};
}

template <bool INT8>
__device__ __forceinline__ h8 kv8_to_h8(const uint8_t* p) {
    if (INT8) {
        const u32x2a w = *(const u32x2a*)p;
        const u32x2a lo = i8x4_to_h4(w.x), hi = i8x4_to_h4(w.y);
        return __builtin_bit_cast(h8, u32x4a{lo.x, lo.y, hi.x, hi.y});
    } else {
        return __builtin_bit_cast(h8, *(const u32x4a*)p);
    }
}

int attn_splits(int seq_len, int n_kv) {
    (void)n_kv;
    // one 64-key tile or more per split, at most 32 splits (8 KV heads x 32
    // splits = 256 workgroups, one per CU)
    if (seq_len <= 0) return 1;
    const int tiles = (seq_len + AT_TILE - 1) / AT_TILE;
    return tiles < 32 ? tiles : 32;
}

size_t attn_partials_floats(int n_heads, int n_splits, int head_dim) {
    return (size_t)n_heads * n_splits * 2 + (size_t)n_heads * n_splits * head_dim;
}

template <bool INT8>
__global__ __launch_bounds__(AT_THREADS)
void attn_partial_kernel(AttnArgs a) {
    constexpr int EB = INT8 ? 1 : 2;                             // bytes per cached element
    __shared__ __attribute__((aligned(16))) uint8_t sKV[2][2][AT_TILE * AT_MAXHD * EB];   // [buf][K|V]
    __shared__ float sKS[2][AT_TILE], sVS[2][AT_TILE];
    __shared__ float sS[AT_MAXG][AT_TILE];                       // scores of the tile
    __shared__ __attribute__((aligned(16))) _Float16 sP[2 * AT_MAXG][AT_TILE];   // hi rows | lo rows
    __shared__ float sM[AT_MAXG], sL[AT_MAXG], sCorr[AT_MAXG];

    const int kvh = blockIdx.x, split = blockIdx.y;
    const int G = a.n_heads / a.n_kv, hd = a.head_dim;
    const int t = threadIdx.x, w = t >> 6, l = t & 63, li = l & 31, lg = l >> 5;
    const int kv_dim = a.n_kv * a.cache_head_dim, hoff = kvh * a.cache_head_dim;
    const int lo_pos = a.window > 0 ? max(0, a.seq - a.window) : 0;
    const int span = a.seq - lo_pos;
    const int S = a.n_splits;
    const int per = (span + S - 1) / S;
    const int kv0 = lo_pos + split * per;
    const int kv1 = min(kv0 + per, a.seq);

    // q operand for Q.K^T: rows = heads (G of 32 used), K = d.  Lane (li, lg)
    // holds head li, d in [16*step + 8*lg, +8).
    h8 qa[AT_MAXHD / 16];
#pragma unroll
    for (int st = 0; st < AT_MAXHD / 16; st++) {
        if (st * 16 < hd && li < G)
            qa[st] = __builtin_bit_cast(h8, *(const u32x4a*)(a.q + (int64_t)(kvh * G + li) * hd + 16 * st + 8 * lg));
        else
            qa[st] = h8{};
    }
    if (t < G) { sM[t] = -FLT_MAX; sL[t] = 0.0f; }

    // P.V accumulators: wave w owns the 32-wide d tiles dt = w and w + 4
    constexpr int NDT = AT_MAXHD / 32 / 4;
    f32x16 acc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) acc[i] = f32x16{};

    auto stage = [&](int b, int p0, int n) {
        const int cpr = hd * EB / 16;                            // 16-byte chunks per row
        for (int c = t; c < AT_TILE * cpr; c += AT_THREADS) {
            const int r = c / cpr, piece = c % cpr;
            const int pos = p0 + min(r, n - 1);                  // rows past the tile end repeat the last key
            const int64_t off = ((int64_t)pos * kv_dim + hoff) * EB + piece * 16;
            *(u32x4a*)(sKV[b][0] + r * hd * EB + piece * 16) = *(const u32x4a*)((const uint8_t*)a.k + off);
            *(u32x4a*)(sKV[b][1] + r * hd * EB + piece * 16) = *(const u32x4a*)((const uint8_t*)a.v + off);
        }
        if (t < AT_TILE) {
            const int pos = p0 + min(t, n - 1);
            sKS[b][t] = (INT8 && a.ks) ? a.ks[(int64_t)pos * a.n_kv + kvh] : 1.0f;
            sVS[b][t] = (INT8 && a.vs) ? a.vs[(int64_t)pos * a.n_kv + kvh] : 1.0f;
        }
    };

    int buf = 0;
    if (kv0 < kv1) stage(0, kv0, min(AT_TILE, kv1 - kv0));
    for (int p0 = kv0; p0 < kv1; p0 += AT_TILE) {
        const int n = min(AT_TILE, kv1 - p0);
        __syncthreads();                                   // tile `buf` staged, previous tile consumed
        if (p0 + AT_TILE < kv1) stage(buf ^ 1, p0 + AT_TILE, min(AT_TILE, kv1 - p0 - AT_TILE));

        // 1. scores: waves 0 and 1 take 32 keys each; lane (li, lg) holds heads
        //    8m + 4lg + r of key 32w + li in c[4m + r]
        if (w < 2) {
            f32x16 c = {};
            const uint8_t* krow = sKV[buf][0] + (32 * w + li) * hd * EB;
            for (int st = 0; st < hd / 16; st++) {
                const h8 kb = kv8_to_h8<INT8>(krow + (16 * st + 8 * lg) * EB);
                c = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa[st], kb, c, 0, 0, 0);
            }
            const int key = 32 * w + li;
            const float ksc = sKS[buf][key] * a.scale;
#pragma unroll
            for (int vv = 0; vv < 16; vv++) {
                const int h = 8 * (vv >> 2) + 4 * lg + (vv & 3);
                if (h < G) sS[h][key] = key < n ? c[vv] * ksc : -INFINITY;
            }
        }
        __syncthreads();

        // 2. online softmax: 16 threads per head, 4 keys each
        {
            const int h = t >> 4, sub = t & 15;
            if (h < G) {
                float sc4[4], mx = -FLT_MAX;
#pragma unroll
                for (int i = 0; i < 4; i++) { sc4[i] = sS[h][sub + 16 * i]; mx = fmaxf(mx, sc4[i]); }
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
                const float m_old = sM[h];
                const float m_new = fmaxf(m_old, mx);
                float ps = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int key = sub + 16 * i;
                    const float p = expf(sc4[i] - m_new);
                    ps += p;
                    const float pv = p * sVS[buf][key];
                    const _Float16 hi = (_Float16)pv;
                    sP[h][key] = hi;
                    sP[G + h][key] = (_Float16)(pv - (float)hi);
                }
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) ps += __shfl_xor(ps, o, 64);
                if (sub == 0) {
                    const float corr = expf(m_old - m_new);
                    sM[h] = m_new;
                    sL[h] = sL[h] * corr + ps;
                    sCorr[h] = corr;
                }
            }
        }
        __syncthreads();

        // 3. acc = acc*corr + P.V  (rows: heads 0..G-1 high parts, G..2G-1 low parts)
#pragma unroll
        for (int i = 0; i < NDT; i++) {
            const int dt = w + 4 * i;
            if (dt < hd / 32) {
#pragma unroll
                for (int vv = 0; vv < 16; vv++) {
                    const int r = 8 * (vv >> 2) + 4 * lg + (vv & 3);
                    if (r < 2 * G) acc[i][vv] *= sCorr[r < G ? r : r - G];
                }
                const int d = 32 * dt + li;
                for (int st = 0; st < AT_TILE / 16; st++) {
                    const int k0 = 16 * st + 8 * lg;
                    const h8 pa = li < 2 * G ? *(const h8*)&sP[li][k0] : h8{};
                    h8 vb;
                    if (INT8) {
                        const uint8_t* vcol = sKV[buf][1] + d;
                        uint32_t w0 = 0, w1 = 0;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            w0 |= (uint32_t)vcol[(k0 + e) * hd] << (8 * e);
                            w1 |= (uint32_t)vcol[(k0 + 4 + e) * hd] << (8 * e);
                        }
                        const u32x2a lo = i8x4_to_h4(w0), hi = i8x4_to_h4(w1);
                        vb = __builtin_bit_cast(h8, u32x4a{lo.x, lo.y, hi.x, hi.y});
                    } else {
                        const _Float16* vcol = (const _Float16*)sKV[buf][1] + d;
#pragma unroll
                        for (int e = 0; e < 8; e++) vb[e] = vcol[(k0 + e) * hd];
                    }
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, vb, acc[i], 0, 0, 0);
                }
            }
        }
        buf ^= 1;
    }
    __syncthreads();

    // 4. unnormalised partials: m, l per head; acc = high rows + low rows
    const int pbase = kvh * G;                                 // first global head of this group
    if (t < G) {
        a.part[(int64_t)(pbase + t) * S + split] = sM[t];
        a.part[(int64_t)a.n_heads * S + (int64_t)(pbase + t) * S + split] = sL[t];
    }
    float* sO = (float*)sKV[0][0];                             // reuse: [2G][hd] floats
#pragma unroll
    for (int i = 0; i < NDT; i++) {
        const int dt = w + 4 * i;
        if (dt < hd / 32) {
#pragma unroll
            for (int vv = 0; vv < 16; vv++) {
                const int r = 8 * (vv >> 2) + 4 * lg + (vv & 3);
                if (r < 2 * G) sO[r * hd + 32 * dt + li] = acc[i][vv];
            }
        }
    }
    __syncthreads();
    float* pacc = a.part + (int64_t)a.n_heads * S * 2;
    for (int e = t; e < G * hd; e += AT_THREADS) {
        const int h = e / hd, d = e % hd;
        pacc[((int64_t)(pbase + h) * S + split) * hd + d] = sO[h * hd + d] + sO[(G + h) * hd + d];
    }
}

// out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M), M = max_s m_s
// (flash_decode_reduce_kernel, attention.cu:944-969)
__global__ __launch_bounds__(256)
void attn_reduce_kernel(uint16_t* __restrict__ out, const float* __restrict__ part, int n_heads, int hd, int S) {
    const int h = blockIdx.x;
    const float* pm = part;
    const float* pl = part + (int64_t)n_heads * S;
    const float* pacc = part + (int64_t)n_heads * S * 2;
    float M = -FLT_MAX;
    for (int s = 0; s < S; s++) M = fmaxf(M, pm[h * S + s]);
    float L = 0.0f;
    for (int s = 0; s < S; s++) L += pl[h * S + s] * expf(pm[h * S + s] - M);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.0f;
        for (int s = 0; s < S; s++) acc += pacc[((int64_t)h * S + s) * hd + d] * expf(pm[h * S + s] - M);
        out[h * hd + d] = f32_to_f16_bits(acc * inv);
    }
}

hipError_t attn_launch(const AttnArgs& a, bool kv_int8, hipStream_t st) {
    dim3 grid(a.n_kv, a.n_splits);
    if (kv_int8) hipLaunchKernelGGL(attn_partial_kernel<true>, grid, dim3(AT_THREADS), 0, st, a);
    else         hipLaunchKernelGGL(attn_partial_kernel<false>, grid, dim3(AT_THREADS), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attn_reduce_kernel, dim3(a.n_heads), dim3(128), 0, st, a.out, (const float*)a.part,
                       a.n_heads, a.head_dim, a.n_splits);
    return hipGetLastError();
}

}  // namespace jllm_hip
