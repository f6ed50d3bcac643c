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
typedef float f32x4a __attribute__((ext_vector_type(4)));

constexpr int AT_KEYS = 32;          // keys per tile (one MFMA column block)
constexpr int AT_MAXHD = 128;
constexpr int AT_MAXG = 16;          // max query heads per KV head
constexpr int AT_MAXS = 128;         // max splits

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
    // one wave per (KV head, split), at least 128 keys (four 32-key tiles)
    // per split, at most AT_MAXS splits
    (void)n_kv;
    if (seq_len <= 0) return 1;
    const int s = (seq_len + 127) / 128;
    return s < AT_MAXS ? s : AT_MAXS;
}

size_t attn_partials_floats(int n_heads, int n_splits, int head_dim) {
    return (size_t)n_heads * n_splits * 2 + (size_t)n_heads * n_splits * head_dim;
}

size_t attn_scratch_bytes(int n_heads, int n_splits, int head_dim) {
    return ATTN_COUNTER_BYTES + attn_partials_floats(n_heads, n_splits, head_dim) * sizeof(float);
}

__host__ __device__ size_t attn_lds_bytes(int n_heads, int n_kv, int head_dim) {
    const int G = n_heads / n_kv;
    const size_t tile = (size_t)AT_KEYS * head_dim + 32 * AT_KEYS * 2;   // V tile (int8 max) + P rows
    const size_t outb = (size_t)2 * G * head_dim * 4;
    return (tile * 2 > outb ? tile * 2 : outb) + 96 * 4;              // fp16 V needs 2x; + corr/ks/vs
}

// One wave per (KV head, split).  Lane (li = lane & 31, lg = lane >> 5).
//   Q.K^T : A = q   (rows = query heads of the group, K = d)
//           B = K^T (cols = the tile's 32 keys, K = d); lane group lg
//               covers d in [lg*hd/2, (lg+1)*hd/2), 8 at a time
//   P.V   : A = P'  (rows = heads, high parts then low parts; K = keys)
//           B = V   (cols = 32 d, K = keys) read as columns from LDS
// The K and V rows of the next tile are loaded into registers while the
// current tile is computed.
template <bool INT8>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2)))
void attn_partial_kernel(AttnArgs a) {
    constexpr int EB = INT8 ? 1 : 2;
    constexpr int RW = AT_MAXHD * EB / 2 / 16;          // 16-byte chunks per lane per row half
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int G = a.n_heads / a.n_kv, hd = a.head_dim, half = hd / 2;
    const int l = threadIdx.x, li = l & 31, lg = l >> 5;
    const int kv_dim = a.n_kv * a.cache_head_dim, hoff = kvh * a.cache_head_dim;
    const int lo_pos = a.window > 0 ? max(0, a.seq - a.window) : 0;
    const int span = a.seq - lo_pos;
    const int S = a.n_splits;
    const int per = (span + S - 1) / S;
    const int kv0 = lo_pos + split * per;
    const int kv1 = min(kv0 + per, a.seq);

    uint8_t* sV = smem;                                          // [32 keys][hd] elements
    _Float16* sP = (_Float16*)(smem + AT_KEYS * AT_MAXHD * EB);   // [32 rows][32 keys]
    float* sMisc = (float*)(smem + attn_lds_bytes(a.n_heads, a.n_kv, hd) - 96 * 4);   // corr[32] | ks[32] | vs[32]

    // q operand: lane (head li, lg), step st -> d = lg*half + 8*st + [0, 8)
    h8 qa[AT_MAXHD / 16];
#pragma unroll
    for (int st = 0; st < AT_MAXHD / 16; st++) {
        if (8 * st < half && li < G)
            qa[st] = __builtin_bit_cast(h8, *(const u32x4a*)(a.q + (int64_t)(kvh * G + li) * hd + lg * half + 8 * st));
        else
            qa[st] = h8{};
    }
    for (int i = l; i < 32 * AT_KEYS; i += 64) sP[i] = (_Float16)0.0f;

    // running softmax state of head li (meaningful in lanes li < G; both
    // lane halves keep identical copies)
    float run_m = -FLT_MAX, run_l = 0.0f;
    constexpr int NDT = AT_MAXHD / 32;
    f32x16 acc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) acc[i] = f32x16{};

    // raw rows of one tile: lane (li, lg) holds K[key li][lg half] and V[key li][lg half]
    u32x4a rk[RW], rv[RW];
    float ksn = 1.0f, vsn = 1.0f;
    auto load_tile = [&](int p0, u32x4a (&k_)[RW], u32x4a (&v_)[RW], float& ks_, float& vs_) {
        const int pos = min(p0 + li, kv1 - 1);
        const uint8_t* kr = (const uint8_t*)a.k + ((int64_t)pos * kv_dim + hoff + lg * half) * EB;
        const uint8_t* vr = (const uint8_t*)a.v + ((int64_t)pos * kv_dim + hoff + lg * half) * EB;
#pragma unroll
        for (int c = 0; c < RW; c++) {
            if (c * 16 < half * EB) {
                k_[c] = *(const u32x4a*)(kr + 16 * c);
                v_[c] = *(const u32x4a*)(vr + 16 * c);
            }
        }
        ks_ = (INT8 && a.ks) ? a.ks[(int64_t)pos * a.n_kv + kvh] : 1.0f;
        vs_ = (INT8 && a.vs) ? a.vs[(int64_t)pos * a.n_kv + kvh] : 1.0f;
    };

    if (kv0 < kv1) load_tile(kv0, rk, rv, ksn, vsn);
    for (int p0 = kv0; p0 < kv1; p0 += AT_KEYS) {
        const int n = min(AT_KEYS, kv1 - p0);
        u32x4a ck[RW], cv[RW];
#pragma unroll
        for (int c = 0; c < RW; c++) { ck[c] = rk[c]; cv[c] = rv[c]; }
        const float ksc = ksn * a.scale, vsc = vsn;   // scales of key li (this lane's load)
        if (p0 + AT_KEYS < kv1) load_tile(p0 + AT_KEYS, rk, rv, ksn, vsn);

        // V rows -> LDS (read back as columns below)
#pragma unroll
        for (int c = 0; c < RW; c++)
            if (c * 16 < half * EB) *(u32x4a*)(sV + (li * hd + lg * half) * EB + 16 * c) = cv[c];

        // 1. transposed scores: C = K.q^T, lane li = head, rows = keys
        //    8*(v/4) + 4*lg + v%4 (v = 0..15): each lane holds 16 of the tile's
        //    32 keys for its head, the other 16 are in lane li ^ 32.
        f32x16 sc = {};
#pragma unroll
        for (int st = 0; st < AT_MAXHD / 16; st++) {
            if (8 * st < half) {
                const uint8_t* kb8 = (const uint8_t*)&ck[(8 * st * EB) / 16] + (8 * st * EB) % 16;
                const h8 kb = kv8_to_h8<INT8>(kb8);
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb, qa[st], sc, 0, 0, 0);
            }
        }
        // per-key scales: lane li (lg = 0) loaded key li's; through LDS to the
        // lanes that hold that key's scores (keys 8m + 4lg + [0,4))
        if (lg == 0) { sMisc[32 + li] = ksc; sMisc[64 + li] = vsc; }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        float kscl[16], vscl[16];
#pragma unroll
        for (int m4 = 0; m4 < 4; m4++) {
            const f32x4a k4 = *(const f32x4a*)&sMisc[32 + 8 * m4 + 4 * lg];
            const f32x4a v4 = *(const f32x4a*)&sMisc[64 + 8 * m4 + 4 * lg];
#pragma unroll
            for (int r = 0; r < 4; r++) { kscl[4 * m4 + r] = k4[r]; vscl[4 * m4 + r] = v4[r]; }
        }
        // 2. online softmax for head li (lanes li < G do the useful work)
        float mx = -FLT_MAX;
#pragma unroll
        for (int vv = 0; vv < 16; vv++) {
            const int key = 8 * (vv >> 2) + 4 * lg + (vv & 3);
            sc[vv] = key < n ? sc[vv] * kscl[vv] : -INFINITY;
            mx = fmaxf(mx, sc[vv]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(run_m, mx);
        const float corr = __expf(run_m - m_new);
        float ps = 0.0f;
        uint32_t hi2[8], lo2[8];
#pragma unroll
        for (int vv = 0; vv < 16; vv += 2) {
            const float p0 = __expf(sc[vv] - m_new), p1 = __expf(sc[vv + 1] - m_new);
            ps += p0 + p1;
            const float q0 = p0 * vscl[vv], q1 = p1 * vscl[vv + 1];
            const _Float16 h0 = (_Float16)q0, h1 = (_Float16)q1;
            const _Float16 l0 = (_Float16)(q0 - (float)h0), l1 = (_Float16)(q1 - (float)h1);
            hi2[vv / 2] = h2_bits(half2_t{h0, h1});
            lo2[vv / 2] = h2_bits(half2_t{l0, l1});
        }
        ps += __shfl_xor(ps, 32, 64);
        run_l = run_l * corr + ps;
        run_m = m_new;
        if (li < G) {
            // keys 8m + 4lg + [0,4) for m = 0..3: four consecutive keys per 8-byte store
#pragma unroll
            for (int m4 = 0; m4 < 4; m4++) {
                const int key0 = 8 * m4 + 4 * lg;
                *(u32x2a*)&sP[li * AT_KEYS + key0] = u32x2a{hi2[2 * m4], hi2[2 * m4 + 1]};
                *(u32x2a*)&sP[(G + li) * AT_KEYS + key0] = u32x2a{lo2[2 * m4], lo2[2 * m4 + 1]};
            }
            if (lg == 0) sMisc[li] = corr;
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);           // lgkmcnt(0): this wave's LDS writes are visible
        __builtin_amdgcn_wave_barrier();
        // 3. acc = acc * corr + P'.V
        float cr[16];
#pragma unroll
        for (int vv = 0; vv < 16; vv++) {
            const int r = 8 * (vv >> 2) + 4 * lg + (vv & 3);
            cr[vv] = r < 2 * G ? sMisc[r < G ? r : r - G] : 1.0f;
        }
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            if (32 * dt < hd) {
#pragma unroll
                for (int vv = 0; vv < 16; vv++) acc[dt][vv] *= cr[vv];
                const int d = 32 * dt + li;
#pragma unroll
                for (int st = 0; st < AT_KEYS / 16; st++) {
                    const int k0 = 16 * st + 8 * lg;
                    const h8 pa = *(const h8*)&sP[li * AT_KEYS + k0];
                    h8 vb;
                    if (INT8) {
                        const uint8_t* col = sV + d;
                        uint32_t w0 = 0, w1 = 0;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            w0 |= (uint32_t)col[(k0 + e) * hd] << (8 * e);
                            w1 |= (uint32_t)col[(k0 + 4 + e) * hd] << (8 * e);
                        }
                        const u32x2a lo = i8x4_to_h4(w0), hi = i8x4_to_h4(w1);
                        vb = __builtin_bit_cast(h8, u32x4a{lo.x, lo.y, hi.x, hi.y});
                    } else {
                        const _Float16* col = (const _Float16*)sV + d;
#pragma unroll
                        for (int e = 0; e < 8; e++) vb[e] = col[(k0 + e) * hd];
                    }
                    acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, vb, acc[dt], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }

    // 4. unnormalised partials: m, l per head; acc = high rows + low rows
    const int pbase = kvh * G;
    float* pm = a.part;
    float* pl = a.part + (int64_t)a.n_heads * S;
    float* pacc = a.part + (int64_t)a.n_heads * S * 2;
    if (li < G && lg == 0) {
        pm[(int64_t)(pbase + li) * S + split] = run_m;
        pl[(int64_t)(pbase + li) * S + split] = run_l;
    }
    float* sO = (float*)smem;                                  // [2G][hd]
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        if (32 * dt < hd) {
#pragma unroll
            for (int vv = 0; vv < 16; vv++) {
                const int r = 8 * (vv >> 2) + 4 * lg + (vv & 3);
                if (r < 2 * G) sO[r * hd + 32 * dt + li] = acc[dt][vv];
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    for (int e = l; e < G * hd; e += 64) {
        const int h = e / hd, d = e % hd;
        pacc[((int64_t)(pbase + h) * S + split) * hd + d] = sO[h * hd + d] + sO[(G + h) * hd + d];
    }
}

// out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M), M = max_s m_s
// (flash_decode_reduce_kernel, attention.cu:944-969).  One workgroup per head;
// the split weights are computed once in LDS, then every output element
// issues its S partial loads together.
__global__ __launch_bounds__(128)
void attn_reduce_kernel(uint16_t* __restrict__ out, const float* __restrict__ part, int n_heads, int hd, int S) {
    __shared__ float sW[AT_MAXS];
    __shared__ float sInv;
    const int h = blockIdx.x, t = threadIdx.x;
    const float* pm = part + (int64_t)h * S;
    const float* pl = part + (int64_t)n_heads * S + (int64_t)h * S;
    const float* pacc = part + (int64_t)n_heads * S * 2 + (int64_t)h * S * hd;
    __shared__ float sRed[2];
    // blockDim.x == AT_MAXS == 128: thread t owns split t
    const float m = t < S ? pm[t] : -FLT_MAX;
    const float lv = t < S ? pl[t] : 0.0f;
    float mx = m;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((t & 63) == 0) sRed[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(sRed[0], sRed[1]);
    const float wgt = t < S ? expf(m - mx) : 0.0f;
    sW[t] = wgt;
    float L = lv * wgt;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
    __syncthreads();
    if ((t & 63) == 0) sRed[t >> 6] = L;
    __syncthreads();
    if (t == 0) { const float Lt = sRed[0] + sRed[1]; sInv = Lt > 0.0f ? 1.0f / Lt : 0.0f; }
    __syncthreads();
    for (int d = t; d < hd; d += blockDim.x) {
        float o = 0.0f;
        for (int s0 = 0; s0 < S; s0 += 16) {
            float pv[16];
#pragma unroll
            for (int i = 0; i < 16; i++) pv[i] = s0 + i < S ? pacc[(int64_t)(s0 + i) * hd + d] : 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) o += pv[i] * sW[min(s0 + i, AT_MAXS - 1)];
        }
        out[(int64_t)h * hd + d] = f32_to_f16_bits(o * sInv);
    }
}

hipError_t attn_launch(const AttnArgs& a, bool kv_int8, hipStream_t st) {
    dim3 grid(a.n_kv, a.n_splits);
    const size_t lds = attn_lds_bytes(a.n_heads, a.n_kv, a.head_dim);
    if (kv_int8) hipLaunchKernelGGL(attn_partial_kernel<true>, grid, dim3(64), lds, st, a);
    else         hipLaunchKernelGGL(attn_partial_kernel<false>, grid, dim3(64), lds, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attn_reduce_kernel, dim3(a.n_heads), dim3(AT_MAXS), 0, st, a.out, (const float*)a.part,
                       a.n_heads, a.head_dim, a.n_splits);
    return hipGetLastError();
}

}  // namespace jllm_hip
