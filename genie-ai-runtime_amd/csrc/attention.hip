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
// Prefill (flash_attention_prefill_batched_kernel, attention.cu:382-514)
// is the same computation per query token t with the causal bound
// seq = start_pos + t + 1: grid z runs over blocks of tq tokens, one split
// each; a wave's MFMA columns are its tq tokens x G heads (each column with
// its own causal bound, so a K/V tile read once serves all of them) and the
// wave writes the normalised outputs directly (no partials, no reduce); a
// decode call with a single split does the same for its one token.
//
// MI355X mapping: one wave64 per (KV head, split[, token]) computes ALL
// query heads of its GQA group, so each KV byte is read from HBM once.
// Keys go in 32-key tiles held in registers (the next tile's rows load
// while the current one is computed).  Q.K^T runs on the matrix cores
// transposed (C = K.q^T: keys are rows, one lane per head, so the softmax
// needs one cross-lane step); the V tile is transposed by an identity MFMA
// (int8: v_mfma_i32_32x32x32_i8 against I, exact) and P.V runs as
// v_mfma_f32_32x32x16_f16 with the fp32 probabilities (times vs) split into
// a high and a low fp16 part, so the P.V products keep ~22 bits: in decode
// the two parts are extra rows of the A operand (2 x G rows), in prefill two
// A operands accumulating into the same rows, so a prefill wave serves 32
// columns (8 tokens x 4 heads).
#include <float.h>
#include <stdlib.h>
#include <string.h>
#include "kq_common.h"
#include "attention.h"
#include "quant_chunk.h"

#ifndef ATTN_RED_XCD
#define ATTN_RED_XCD 1
#endif

namespace jllm_hip {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));
typedef float f32x4a __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int AT_KEYS = 32;          // keys per tile (one MFMA column block)
// LDS row stride of the P' tile (halves): 18 dwords, so the 8-byte writes
// and reads of lanes (row li, key group lg) spread evenly over the 32 banks
// (a 16-dword stride put every row on the same 4 banks)
constexpr int AT_PLD = AT_KEYS + 4;
constexpr int AT_MAXHD = 128;
constexpr int AT_MAXG = 16;          // max query heads per KV head
constexpr int AT_MAXS = ATTN_MAX_SPLITS;   // max splits

// 4 signed int8 (one word) -> 4 exact fp16 values (two words): with u = b ^ 0x80
// in [1, 255], the half with bits 0x64 : u is 1024 + u (byte permutes against
// a word of 0x64 bytes), minus 1152 gives b.
__device__ __forceinline__ u32x2a i8x4_to_h4(uint32_t w) {
    const half2_t bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
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

#ifdef JLLM_ATTN_TRACE
// probe builds only: per-wave timestamps (s_memrealtime, 100 MHz) of the last
// decode launch: [start, first tile done, tiles done, partials issued]
__device__ uint64_t g_attn_trace[8192 * 4];
#define AT_MARK(i) do { tr[i] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define AT_MARK(i) do { } while (0)
#endif

// JLLM_SPLITK=0 switches split-K off (one split per head), read once, as the
// reference's splitk_enabled does (attention.cu:990-996)
bool attn_splitk_enabled() {
    static const bool enabled = [] {
        const char* v = getenv("JLLM_SPLITK");
        return !v || strcmp(v, "0") != 0;
    }();
    return enabled;
}

int attn_splits(int seq_len, int n_kv) {
    // one wave per (KV head, split): at least 32 keys (one tile) per split,
    // at most 128 splits (measured on MI355X: short splits keep every SIMD
    // busy; past 128 the partials and the reduce cost more than they save)
    (void)n_kv;
    if (!attn_splitk_enabled() || seq_len <= 0) return 1;
    const int s = (seq_len + 31) / 32;
    return s < 128 ? s : 128;
}

int attn_decode_waves(int n_splits) {
    // measured on MI355X (32 / 8 heads x 128, INT8 KV, >= 256 MB of distinct
    // caches): 4 waves per workgroup from 64 key ranges on (ctx 2048 / 4096 /
    // 8192: 10.9 -> 10.5, 13.2 -> 12.1, 15.3 -> 14.6 us), since the split
    // combination then reads a quarter of the partials; below that the LDS
    // combination costs more than it saves (ctx 512, 16 ranges: 8.2 us with
    // one wave per workgroup, 9.6 / 10.1 / 11.9 us with 2 / 4 / 8), and one
    // workgroup per head (no second launch) is slower still (12.1 us): its
    // waves share a CU's SIMDs, where the per-tile arithmetic is the bound
    return n_splits >= 64 ? 4 : 1;
}

size_t attn_partials_floats(int n_heads, int n_splits, int head_dim) {
    return (size_t)n_heads * n_splits * 2 + (size_t)n_heads * n_splits * head_dim;
}

size_t attn_scratch_bytes(int n_heads, int n_splits, int head_dim) {
    return ATTN_COUNTER_BYTES + attn_partials_floats(n_heads, n_splits, head_dim) * sizeof(float);
}

// LDS of one wave (P' tile, per-key scales, then its final hi/lo rows)
__host__ __device__ size_t attn_wave_lds_bytes(int n_heads, int n_kv, int head_dim, int tq) {
    const int G = n_heads / n_kv * tq;                                // columns of a wave
    const bool ps = tq > 1;                                          // prefill: one row per column
    const size_t loop = (size_t)(ps ? 64 : 32) * AT_PLD * 2 + 96 * 4; // P' rows (fp16) + corr/ks/vs
    // final rows (fp32, >= 8); prefill: all 32 rows of the accumulator layout,
    // so the epilogue stores them without a per-row predicate
    const size_t outb = (size_t)(ps ? 32 : ((2 * G + 7) & ~7)) * head_dim * 4;
    return ((loop > outb ? loop : outb) + 15) & ~(size_t)15;
}
// a workgroup of W waves: W wave regions, then (m, l) of each wave's columns
__host__ __device__ size_t attn_lds_bytes(int n_heads, int n_kv, int head_dim, int tq, int W) {
    return (size_t)W * attn_wave_lds_bytes(n_heads, n_kv, head_dim, tq) +
           (W > 1 ? (size_t)W * 2 * 32 * 4 + (size_t)(ATTN_MAX_WAVES + 1) * 32 * 4 + (size_t)W * 32 * 4 : 0);
}

// One wave per (KV head, split[, block of tq query tokens]).  The wave's
// "columns" are its (token, head) pairs: column c = token tok0 + c / G, head
// kvh * G + c % G, GC = tq * G <= 32 of them; each has its own causal bound
// (and window), so one key tile serves tq tokens.  Lane (li = lane & 31,
// lg = lane >> 5); below, "head li" means column li.
//   Q.K^T : C = K.q^T (rows = the tile's 32 keys, cols = query heads, K = d);
//           lane group lg covers d in [lg*hd/2, (lg+1)*hd/2), 8 at a time
//   V^T   : the V rows are turned into columns on the matrix cores: with A =
//           V rows (K = d) and B = the identity, C = V lands in the MFMA
//           output layout, i.e. lane (d = li, lg) holds 16 keys of column d
//           (int8: one v_mfma_i32_32x32x32_i8 per 32 d, exact)
//   P.V   : A = P'  (decode: rows = heads, high parts then low parts;
//           prefill: rows = columns, the high and the low parts as two A
//           operands into the same accumulator; K = keys in the order the
//           transpose delivers them), B = those V columns
// The K and V rows of the next tile are loaded into registers while the
// current tile is computed.
// MT: several query tokens per wave (per-column causal bounds); the
// single-token form (decode, or tq == 1) compiles without the column masks.
// G4: at most 4 columns (decode with <= 4 q heads per KV head): the P.V rows
// 8 and up hold nothing, so their accumulators are never rescaled.
template <bool INT8, int HD, bool MT, bool G4>
__global__ __launch_bounds__(64 * ATTN_MAX_WAVES) __attribute__((amdgpu_waves_per_eu(2)))
void attn_partial_kernel(AttnArgs a) {
    constexpr int EB = INT8 ? 1 : 2;
    constexpr int hd = HD, half = HD / 2;
    constexpr int KW = (half * EB + 15) / 16;           // K: 16-byte chunks per lane (half a row)
    constexpr int NDT = HD / 32;                        // 32-wide d chunks
    constexpr int VW = NDT * EB;                        // V: 16-byte chunks per lane
    constexpr int NST = half / 8;                       // Q.K^T MFMA steps
    // prefill (MT): the high and low fp16 parts of P' are two A operands
    // accumulating into the same accumulator row, one row per column, so a
    // wave serves 32 columns; decode keeps a row for each (2 x G rows)
    constexpr bool PS = MT;
    constexpr int PROWS = PS ? 64 : 32;                 // P' tile rows in LDS
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_wg[];
    const int W = a.wsplit;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const size_t wave_lds = attn_wave_lds_bytes(a.n_heads, a.n_kv, a.head_dim, a.tq);
    uint8_t* smem = smem_wg + (size_t)wv * wave_lds;
    uint64_t tr[4] = {0, 0, 0, 0};
    AT_MARK(0);
    // prefill: the last token blocks (the most key tiles) are dispatched first
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int tok0 = MT ? ((int)gridDim.z - 1 - (int)blockIdx.z) * a.tq : blockIdx.z;
    const int aseq = (!MT && a.pos_dev) ? __builtin_amdgcn_readfirstlane(*a.pos_dev) + 1 : a.seq;
    const int G = a.n_heads / a.n_kv;
    const int ntok = MT ? min(a.tq, a.tokens - tok0) : 1;       // tokens of this wave
    const int GC = ntok * G;                                    // live columns
    const int l = (int)threadIdx.x & 63, li = l & 31, lg = l >> 5;
    // column li: its token, causal bound and window start
    const int ctok = MT ? tok0 + (li < GC ? li / G : 0) : tok0;
    const int seq_c = aseq + ctok;
    const int lo_c = a.window > 0 ? max(0, seq_c - a.window) : 0;
    // the wave's key range covers every column's
    const int seq = aseq + tok0 + ntok - 1;
    const int kv_dim = a.n_kv * a.cache_head_dim, hoff = kvh * a.cache_head_dim;
    const int lo_pos = a.window > 0 ? max(0, aseq + tok0 - a.window) : 0;
    const int span = seq - lo_pos;
    const int S = a.n_splits;
    const int per = (span + S - 1) / S;
    const int kv0 = lo_pos + split * per;
    const int kv1 = min(kv0 + per, seq);

    // raw rows of one tile: lane (li, lg) holds K[key li][lg half] and the V
    // pieces of key li its lane group feeds to the transpose: int8
    // V[32m + 16lg, +16); fp16 V[32m + 8lg, +8) and V[32m + 16 + 8lg, +8)
    u32x4a rk[KW], rv[VW];
    float ksn = 1.0f, vsn = 1.0f;
    auto load_tile = [&](int p0, u32x4a (&k_)[KW], u32x4a (&v_)[VW], float& ks_, float& vs_) {
        const int pos = min(p0 + li, kv1 - 1);
        const uint8_t* kr = (const uint8_t*)a.k + ((int64_t)pos * kv_dim + hoff + lg * half) * EB;
        const uint8_t* vr = (const uint8_t*)a.v + ((int64_t)pos * kv_dim + hoff) * EB;
#pragma unroll
        for (int c = 0; c < KW; c++) k_[c] = *(const u32x4a*)(kr + 16 * c);
#pragma unroll
        for (int m = 0; m < NDT; m++) {
            if (INT8) {
                v_[m] = *(const u32x4a*)(vr + 32 * m + 16 * lg);
            } else {
                v_[2 * m] = *(const u32x4a*)(vr + (32 * m + 8 * lg) * 2);
                v_[2 * m + 1] = *(const u32x4a*)(vr + (32 * m + 16 + 8 * lg) * 2);
            }
        }
        ks_ = (INT8 && a.ks) ? a.ks[(int64_t)pos * a.n_kv + kvh] : 1.0f;
        vs_ = (INT8 && a.vs) ? a.vs[(int64_t)pos * a.n_kv + kvh] : 1.0f;
    };

    // the first tile's loads go out before any other set-up work, so that
    // their latency overlaps it
    const int first = kv0 + wv * AT_KEYS, stride = W * AT_KEYS;
    if (first < kv1) load_tile(first, rk, rv, ksn, vsn);
    __builtin_amdgcn_sched_barrier(0);

    _Float16* sP = (_Float16*)smem;                              // [32 rows][AT_PLD: 32 keys + pad]
    float* sMisc = (float*)(smem + PROWS * AT_PLD * 2);         // corr[32] | ks[32] | vs[32]

    // q operand: lane (head li, lg), step st -> d = lg*half + 8*st + [0, 8)
    // (every lane loads a valid row -- its column's head modulo G -- so the
    // loads issue unpredicated; lanes without a column then zero theirs)
    h8 qa[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        const u32x4a qv = *(const u32x4a*)(a.q + (int64_t)ctok * a.n_heads * hd + (int64_t)(kvh * G + li % G) * hd +
                                           lg * half + 8 * st);
        qa[st] = __builtin_bit_cast(h8, li < GC ? qv : u32x4a{0u, 0u, 0u, 0u});
    }
    for (int i = l; i < PROWS * AT_PLD; i += 64) sP[i] = (_Float16)0.0f;

    // identity operands of the V transpose.  int8: lane (col li, lg) holds
    // B[16lg + i][li] = (16lg + i == li).  fp16: two K = 16 halves, lane
    // (col li, lg) holds B_hh[8lg + e][li] = (16hh + 8lg + e == li).
    i32x4 eye8;
    h8 eyeh[2];
    {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        const int pos = li - 16 * lg;
        if (pos >= 0 && pos < 16) w[pos >> 2] = 1u << (8 * (pos & 3));
        eye8 = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
#pragma unroll
            for (int e = 0; e < 8; e++) eyeh[hh][e] = (_Float16)((16 * hh + 8 * lg + e == li) ? 1.0f : 0.0f);
    }

    // running softmax state of column li (meaningful in lanes li < GC; both
    // lane halves keep identical copies)
    float run_m = -FLT_MAX, run_l = 0.0f;
    f32x16 acc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) acc[i] = f32x16{};

    // one tile from the registers (ck, cv; key scales ksc, vsc of key li)
    auto tile = [&](int p0, const u32x4a (&ck)[KW], const u32x4a (&cv)[VW], float ksc, float vsc) {
        const int n = min(AT_KEYS, kv1 - p0);
        // 1. transposed scores: C = K.q^T, lane li = head, rows = keys
        //    8*(v/4) + 4*lg + v%4 (v = 0..15): each lane holds 16 of the tile's
        //    32 keys for its head, the other 16 are in lane li ^ 32.
        f32x16 sc = {};
#pragma unroll
        for (int st = 0; st < NST; st++) {
            const uint8_t* kb8 = (const uint8_t*)&ck[(8 * st * EB) / 16] + (8 * st * EB) % 16;
            const h8 kb = kv8_to_h8<INT8>(kb8);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb, qa[st], sc, 0, 0, 0);
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
        // 2. online softmax for column li (lanes li < GC do the useful work)
        float mx = -FLT_MAX;
#pragma unroll
        for (int vv = 0; vv < 16; vv++) sc[vv] *= kscl[vv];
        // key masks only where a tile can hold dead keys (uniform branch): a
        // prefill tile that reaches past the first column's causal bound or
        // below the last column's window start, or a tile of fewer than
        // AT_KEYS keys (a live key keeps its score either way, so skipping
        // the masks of a full tile changes no bit)
        const bool full = n == AT_KEYS && (!MT || (p0 + AT_KEYS <= aseq + tok0 &&
                                                   (a.window <= 0 || p0 >= aseq + tok0 + ntok - 1 - a.window)));
        if (!full) {
#pragma unroll
            for (int vv = 0; vv < 16; vv++) {
                const int key = 8 * (vv >> 2) + 4 * lg + (vv & 3);
                const int pos = p0 + key;
                const bool live = MT ? (key < n && pos < seq_c && pos >= lo_c) : key < n;
                sc[vv] = live ? sc[vv] : -INFINITY;
            }
        }
#pragma unroll
        for (int vv = 0; vv < 16; vv++) mx = fmaxf(mx, sc[vv]);
        {
            float a0, a1;
            wave_halves(mx, a0, a1);
            mx = fmaxf(a0, a1);
        }
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
        {
            float a0, a1;
            wave_halves(ps, a0, a1);
            ps = a0 + a1;
        }
        run_l = run_l * corr + ps;
        run_m = m_new;
        // no live column's maximum moved: every rescale factor is exactly 1
        // (e^0), so the accumulators keep their values without the multiply
        const bool rescale = __builtin_amdgcn_ballot_w64(li < GC && corr != 1.0f) != 0;
        if (li < GC) {
            // keys 8m + 4lg + [0,4) for m = 0..3: four consecutive keys per 8-byte store
#pragma unroll
            for (int m4 = 0; m4 < 4; m4++) {
                const int key0 = 8 * m4 + 4 * lg;
                *(u32x2a*)&sP[li * AT_PLD + key0] = u32x2a{hi2[2 * m4], hi2[2 * m4 + 1]};
                *(u32x2a*)&sP[((PS ? 32 : GC) + li) * AT_PLD + key0] = u32x2a{lo2[2 * m4], lo2[2 * m4 + 1]};
            }
            if (lg == 0) sMisc[li] = corr;
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);           // lgkmcnt(0): this wave's LDS writes are visible
        __builtin_amdgcn_wave_barrier();
        // 3. acc = acc * corr + P'.V.  The transpose delivers keys
        //    8*(v/4) + 4lg + v%4 in element v; MFMA step st takes v = 8st..8st+7,
        //    so P' is read at keys 16st + 4lg + [0,4) and 16st + 8 + 4lg + [0,4).
        constexpr int NLIVE = G4 ? 4 : 16;              // accumulator elements that can hold a row
        float cr[16];
#pragma unroll
        for (int vv = 0; vv < NLIVE; vv++) {
            const int r = 8 * (vv >> 2) + 4 * lg + (vv & 3);
            cr[vv] = PS ? (r < GC ? sMisc[r] : 1.0f) : (r < 2 * GC ? sMisc[r < GC ? r : r - GC] : 1.0f);
        }
        if (rescale) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int vv = 0; vv < NLIVE; vv++) acc[dt][vv] *= cr[vv];
        }
        h8 pa[2], pl[2];
#pragma unroll
        for (int st = 0; st < 2; st++) {
            const u32x2a lo4 = *(const u32x2a*)&sP[li * AT_PLD + 16 * st + 4 * lg];
            const u32x2a hi4 = *(const u32x2a*)&sP[li * AT_PLD + 16 * st + 8 + 4 * lg];
            pa[st] = __builtin_bit_cast(h8, u32x4a{lo4.x, lo4.y, hi4.x, hi4.y});
            if (PS) {
                const u32x2a a4 = *(const u32x2a*)&sP[(32 + li) * AT_PLD + 16 * st + 4 * lg];
                const u32x2a b4 = *(const u32x2a*)&sP[(32 + li) * AT_PLD + 16 * st + 8 + 4 * lg];
                pl[st] = __builtin_bit_cast(h8, u32x4a{a4.x, a4.y, b4.x, b4.y});
            }
        }
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            {
                float vt[16];                            // V[key 8(v/4)+4lg+v%4][32dt + li]
                if (INT8) {
                    const i32x16 ct = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, cv[dt]), eye8,
                                                                             i32x16{}, 0, 0, 0);
#pragma unroll
                    for (int vv = 0; vv < 16; vv++) vt[vv] = (float)ct[vv];
                } else {
                    f32x16 ct = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, cv[2 * dt]), eyeh[0],
                                                                      f32x16{}, 0, 0, 0);
                    ct = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, cv[2 * dt + 1]), eyeh[1], ct, 0, 0, 0);
#pragma unroll
                    for (int vv = 0; vv < 16; vv++) vt[vv] = ct[vv];
                }

#pragma unroll
                for (int st = 0; st < 2; st++) {
                    h8 vb;
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        const auto h2 = __builtin_amdgcn_cvt_pkrtz(vt[8 * st + e], vt[8 * st + e + 1]);   // exact
                        vb[e] = h2[0];
                        vb[e + 1] = h2[1];
                    }
                    acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[st], vb, acc[dt], 0, 0, 0);
                    if (PS) acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pl[st], vb, acc[dt], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    };
    // the next tile's rows load into (rk, rv) while the current one (a copy)
    // is computed
    // wave wv of W takes tiles wv, wv + W, ... of the workgroup's key range
    // (the last tile is computed straight from the load registers: no copy,
    // and Q.K^T starts once the K rows have landed)
    int p0 = first;
    for (; p0 + stride < kv1; p0 += stride) {
        u32x4a ck[KW], cv[VW];
#pragma unroll
        for (int c = 0; c < KW; c++) ck[c] = rk[c];
#pragma unroll
        for (int c = 0; c < VW; c++) cv[c] = rv[c];
        const float ksc = ksn * a.scale, vsc = vsn;
        load_tile(p0 + stride, rk, rv, ksn, vsn);
        tile(p0, ck, cv, ksc, vsc);
        if (p0 == first) AT_MARK(1);
    }
    if (p0 < kv1) {
        tile(p0, rk, rv, ksn * a.scale, vsn);
        if (p0 == first) AT_MARK(1);
    }
    AT_MARK(2);

    // 4. S == 1: the normalised output straight from this wave; else the
    //    unnormalised partials m, l per head (acc = high rows + low rows)
    const int pbase = kvh * G;
    float* sO = (float*)smem;                                  // [2G][hd]
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    if constexpr (!MT) {
        // decode: the rows go to LDS transposed, sOT[d][R] (R = 2G rounded up
        // to 8), four consecutive rows of a column per 16-byte store, only the
        // row groups that hold a head; then lane l forms the outputs of
        // d = l, l + 64, ... for every head (high + low row) and stores them
        // coalesced along d
        const int R = (2 * G + 7) & ~7;
        float* sOT = (float*)smem;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
            for (int m4 = 0; m4 < 4; m4++) {
                if (8 * m4 >= 2 * G) break;
                *(f32x4a*)&sOT[(32 * dt + li) * R + 8 * m4 + 4 * lg] =
                    f32x4a{acc[dt][4 * m4], acc[dt][4 * m4 + 1], acc[dt][4 * m4 + 2], acc[dt][4 * m4 + 3]};
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        if (W > 1) {
            // combine the W waves' states per head, waves in order:
            // M = max_w m_w, num = sum_w acc_w e^(m_w - M), den = sum_w l_w e^(m_w - M);
            // the workgroup's output (S == 1) or its partial (M, den, num).
            // Wave weights e^(m_w - M) are formed once per (wave, head), then
            // every thread issues all its LDS reads before it adds.
            float* sML = (float*)(smem_wg + (size_t)W * wave_lds);     // [W][m[32] | l[32]], then f [W][32]
            float* sF = sML + W * 64;
            if (lg == 0) { sML[wv * 64 + li] = run_m; sML[wv * 64 + 32 + li] = run_l; }
            __syncthreads();
            const int t = (int)threadIdx.x;
            if (t < W * G) {
                const int u = t / G, h = t % G;
                float M = -FLT_MAX;
                for (int w = 0; w < W; w++) M = fmaxf(M, sML[w * 64 + h]);
                sF[u * 32 + h] = expf(sML[u * 64 + h] - M);
                if (u == 0) sF[ATTN_MAX_WAVES * 32 + h] = M;
            }
            __syncthreads();
            float* pm = a.part;
            float* pl = a.part + (int64_t)a.n_heads * S;
            float* pacc = a.part + (int64_t)a.n_heads * S * 2;
            for (int e = t; e < G * hd; e += 64 * W) {
                const int d = e / G, h = e % G;     // lanes: consecutive heads of one d, then d
                float hi[ATTN_MAX_WAVES], lo[ATTN_MAX_WAVES], f[ATTN_MAX_WAVES], lv[ATTN_MAX_WAVES];
#pragma unroll
                for (int u = 0; u < ATTN_MAX_WAVES; u++) {
                    if (u < W) {
                        const float* so = (const float*)(smem_wg + (size_t)u * wave_lds);
                        hi[u] = so[d * R + h];
                        lo[u] = so[d * R + G + h];
                        f[u] = sF[u * 32 + h];
                        lv[u] = sML[u * 64 + 32 + h];
                    }
                }
                float num = 0.0f, den = 0.0f;
#pragma unroll
                for (int u = 0; u < ATTN_MAX_WAVES; u++) {
                    if (u < W) {
                        num += (hi[u] + lo[u]) * f[u];
                        den += lv[u] * f[u];
                    }
                }
                if (S == 1) {
                    a.out[(int64_t)(pbase + h) * hd + d] = f32_to_f16_bits(den > 0.0f ? num / den : 0.0f);
                } else {
                    pacc[((int64_t)(pbase + h) * S + split) * hd + d] = num;
                    if (d == 0) {
                        pm[(int64_t)(pbase + h) * S + split] = sF[ATTN_MAX_WAVES * 32 + h];
                        pl[(int64_t)(pbase + h) * S + split] = den;
                    }
                }
            }
#ifdef JLLM_ATTN_TRACE
            AT_MARK(3);
            {
                const int gw = ((int)blockIdx.y * (int)gridDim.x + (int)blockIdx.x) * W + wv;
                if (l < 4 && gw < 8192) {
                    uint64_t tv = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) if (l == i) tv = tr[i];
                    g_attn_trace[gw * 4 + l] = tv;
                }
            }
#endif
            return;
        }
        if (S == 1) {
            const float inv_l = run_l > 0.0f ? 1.0f / run_l : 0.0f;
            for (int h = 0; h < G; h++) {
                const float il = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, inv_l), h));
                uint16_t* ot = a.out + (int64_t)(pbase + h) * hd;
                for (int d = l; d < hd; d += 64)
                    ot[d] = f32_to_f16_bits((sOT[d * R + h] + sOT[d * R + G + h]) * il);
            }
            return;
        }
        float* pm = a.part;
        float* pl = a.part + (int64_t)a.n_heads * S;
        if (li < G && lg == 0) {
            pm[(int64_t)(pbase + li) * S + split] = run_m;
            pl[(int64_t)(pbase + li) * S + split] = run_l;
        }
        float* pacc = a.part + (int64_t)a.n_heads * S * 2 + ((int64_t)pbase * S + split) * hd;
        for (int h = 0; h < G; h++) {
            for (int d = l; d < hd; d += 64) pacc[(int64_t)h * S * hd + d] = sOT[d * R + h] + sOT[d * R + G + h];
        }
#ifdef JLLM_ATTN_TRACE
        AT_MARK(3);
        const int gw = blockIdx.y * gridDim.x + blockIdx.x;
        if (l < 4 && gw < 8192) {
            uint64_t tv = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) if (l == i) tv = tr[i];
            g_attn_trace[gw * 4 + l] = tv;
        }
#endif
        return;
    }
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
        for (int vv = 0; vv < 16; vv++) {
            const int r = 8 * (vv >> 2) + 4 * lg + (vv & 3);
            if (PS || r < 2 * GC) sO[r * hd + 32 * dt + li] = acc[dt][vv];   // PS: rows >= GC are never read
        }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    if (MT && W > 1) {
        // combine the W waves' states per column, waves in order:
        // out = sum_w acc_w e^(m_w - M) / sum_w l_w e^(m_w - M), M = max_w m_w.
        // The per-column quantities (wave weights, denominator, output row)
        // are formed once per column; then each thread takes 8 consecutive d
        // of a column: 16-byte LDS reads and one 16-byte store of 8 halves
        // (the arithmetic per element as written above, in wave order, so the
        // division and every rounding are those of the per-element form).
        float* sML = (float*)(smem_wg + (size_t)W * wave_lds);     // [W][m[32] | l[32]]
        float* sF = sML + W * 64;                                  // [W][32] wave weights
        float* sDen = sF + ATTN_MAX_WAVES * 32;                    // [32] denominators
        if (lg == 0) { sML[wv * 64 + li] = run_m; sML[wv * 64 + 32 + li] = run_l; }
        __syncthreads();
        const int t = (int)threadIdx.x;
        if (t < GC) {
            float M = -FLT_MAX;
            for (int u = 0; u < W; u++) M = fmaxf(M, sML[u * 64 + t]);
            float den = 0.0f;
            for (int u = 0; u < W; u++) {
                const float f = expf(sML[u * 64 + t] - M);
                sF[u * 32 + t] = f;
                den += sML[u * 64 + 32 + t] * f;
            }
            sDen[t] = den;
        }
        __syncthreads();
        const int nd8 = hd / 8;
        const bool vec = ((uintptr_t)a.out & 15u) == 0;
        for (int e = t; e < GC * nd8; e += 64 * W) {
            const int c = e / nd8, d0 = (e - c * nd8) * 8;
            float num[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            for (int u = 0; u < W; u++) {
                const float f = sF[u * 32 + c];
                const float* so = (const float*)(smem_wg + (size_t)u * wave_lds);
                const f32x4a h0 = *(const f32x4a*)&so[c * hd + d0], h1 = *(const f32x4a*)&so[c * hd + d0 + 4];
                f32x4a l0 = f32x4a{0.0f, 0.0f, 0.0f, 0.0f}, l1 = l0;
                if (!PS) { l0 = *(const f32x4a*)&so[(GC + c) * hd + d0]; l1 = *(const f32x4a*)&so[(GC + c) * hd + d0 + 4]; }
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    num[i] += (h0[i] + l0[i]) * f;
                    num[4 + i] += (h1[i] + l1[i]) * f;
                }
            }
            const float den = sDen[c];
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                o[i] = (uint32_t)f32_to_f16_bits(den > 0.0f ? num[2 * i] / den : 0.0f) |
                       ((uint32_t)f32_to_f16_bits(den > 0.0f ? num[2 * i + 1] / den : 0.0f) << 16);
            const int ct = c / G, ch = c - ct * G;
            uint16_t* ot = a.out + (int64_t)(tok0 + ct) * a.n_heads * hd + (int64_t)(pbase + ch) * hd + d0;
            if (vec) {
                *(u32x4a*)ot = u32x4a{o[0], o[1], o[2], o[3]};
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) { ot[2 * i] = (uint16_t)(o[i] & 0xFFFFu); ot[2 * i + 1] = (uint16_t)(o[i] >> 16); }
            }
            if (a.qcodes) {
                // the 4 lanes of an aligned quad hold the 32 values of one
                // quantiser block (hd % 32 == 0, nd8 % 4 == 0)
                float v[8];
#pragma unroll
                for (int i = 0; i < 4; i++) { v[2 * i] = f16_bits_to_f32(o[i] & 0xFFFFu); v[2 * i + 1] = f16_bits_to_f32(o[i] >> 16); }
                const int kb32 = ((pbase + ch) * hd + d0) >> 5, sub = (d0 >> 3) & 3;
                if (a.q_i8) quant_chunk<true>(v, sub, kb32, tok0 + ct, a.q_npad, a.qcodes, a.qscl, true);
                else        quant_chunk<false>(v, sub, kb32, tok0 + ct, a.q_npad, a.qcodes, a.qscl, false);
            }
        }
        return;
    }
    if (S == 1) {
        const float inv_l = run_l > 0.0f ? 1.0f / run_l : 0.0f;
        for (int e = l; e < GC * hd; e += 64) {
            const int c = e / hd, d = e % hd;
            const float il = __shfl(inv_l, c, 64);
            const int ct = MT ? c / G : 0, ch = MT ? c % G : c;
            uint16_t* ot = a.out + (int64_t)(tok0 + ct) * a.n_heads * hd + (int64_t)(pbase + ch) * hd;
            ot[d] = f32_to_f16_bits((PS ? sO[c * hd + d] : sO[c * hd + d] + sO[(GC + c) * hd + d]) * il);
        }
        return;
    }
    float* pm = a.part;
    float* pl = a.part + (int64_t)a.n_heads * S;
    float* pacc = a.part + (int64_t)a.n_heads * S * 2;
    if (li < G && lg == 0) {
        pm[(int64_t)(pbase + li) * S + split] = run_m;
        pl[(int64_t)(pbase + li) * S + split] = run_l;
    }
    for (int e = l; e < G * hd; e += 64) {
        const int h = e / hd, d = e % hd;
        pacc[((int64_t)(pbase + h) * S + split) * hd + d] = sO[h * hd + d] + sO[(G + h) * hd + d];
    }
}

// out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M), M = max_s m_s
// (flash_decode_reduce_kernel, attention.cu:944-969).  One workgroup of 8
// waves per head: the split weights go to LDS, then wave w sums the splits
// s = w, w + 8, ... for two d per lane (all its partial loads in flight at
// once), and the 8 wave sums are added in a fixed order.
// The head a combination workgroup takes.  Workgroup b of a launch runs on
// XCD b % 8, and the partial kernel's workgroup (kvh, range) has linear
// index kvh + n_kv * range, so with n_kv a multiple of 8 every key range of
// KV head kvh ran on XCD kvh % 8; handing workgroup b the head (b % n_kv) *
// G + b / n_kv puts the combination on that XCD too, where the partials may
// still sit in its L2.  (Any n_kv: still a permutation of the heads.)
__device__ __forceinline__ int red_head(int n_heads, int n_kv) {
#if ATTN_RED_XCD
    const int b = blockIdx.x;
    return (b % n_kv) * (n_heads / n_kv) + b / n_kv;
#else
    (void)n_heads; (void)n_kv;
    return blockIdx.x;
#endif
}

constexpr int AT_RED_THREADS = 512;
__global__ __launch_bounds__(AT_RED_THREADS)
void attn_reduce_kernel(uint16_t* __restrict__ out, const float* __restrict__ part, int n_heads, int n_kv, int hd,
                        int S) {
    __shared__ float sW[AT_MAXS];
    __shared__ float sRed[AT_RED_THREADS / 64];
    __shared__ float sSum[AT_RED_THREADS / 64][AT_MAXHD];
    const int h = red_head(n_heads, n_kv), t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    const float* pm = part + (int64_t)h * S;
    const float* pl = part + (int64_t)n_heads * S + (int64_t)h * S;
    const float* pacc = part + (int64_t)n_heads * S * 2 + (int64_t)h * S * hd;
    // wave w: splits w, w+8, ...; lane l: d = 2l, 2l+1 -- loaded first, with
    // (m, l), so that both take one round trip to memory
    constexpr int NW = AT_RED_THREADS / 64;
    constexpr int MAXPER = AT_MAXS / NW;
    float2 pv[MAXPER];
#pragma unroll
    for (int i = 0; i < MAXPER; i++) {
        const int sp = w + NW * i;
        pv[i] = (sp < S && 2 * l < hd) ? *(const float2*)(pacc + (int64_t)sp * hd + 2 * l) : make_float2(0.0f, 0.0f);
    }
    const float m = t < S ? pm[t] : -FLT_MAX;
    const float lv = t < S ? pl[t] : 0.0f;
    float mx = m;
    mx = wave_max(mx);
    if (l == 0) sRed[w] = mx;
    __syncthreads();
    mx = sRed[0];
#pragma unroll
    for (int i = 1; i < AT_RED_THREADS / 64; i++) mx = fmaxf(mx, sRed[i]);
    const float wgt = t < S ? expf(m - mx) : 0.0f;
    if (t < AT_MAXS) sW[t] = wgt;
    float L = lv * wgt;
    L = wave_sum(L);
    __syncthreads();
    if (l == 0) sRed[w] = L;
    __syncthreads();
    float Lt = 0.0f;
#pragma unroll
    for (int i = 0; i < AT_RED_THREADS / 64; i++) Lt += sRed[i];
    const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
    float2 o = make_float2(0.0f, 0.0f);
    if (2 * l < hd) {
#pragma unroll
        for (int i = 0; i < MAXPER; i++) {
            const int sp = w + NW * i;
            const float wi = sp < S ? sW[sp] : 0.0f;
            o.x += pv[i].x * wi;
            o.y += pv[i].y * wi;
        }
        sSum[w][2 * l] = o.x;
        sSum[w][2 * l + 1] = o.y;
    }
    __syncthreads();
    if (t < hd) {
        float r = 0.0f;
#pragma unroll
        for (int i = 0; i < NW; i++) r += sSum[i][t];
        out[(int64_t)h * hd + t] = f32_to_f16_bits(r * inv);
    }
}

// The same combination with one wave per head: lane l holds splits l, l+64,
// ... (m, l) and then sums the acc of every split for d = 2l, 2l+1 in split
// order; no workgroup barriers.
__global__ __launch_bounds__(64)
void attn_reduce_wave_kernel(uint16_t* __restrict__ out, const float* __restrict__ part, int n_heads, int n_kv, int hd,
                             int S) {
    __shared__ float sW[AT_MAXS];
    const int h = red_head(n_heads, n_kv), l = threadIdx.x;
    const float* pm = part + (int64_t)h * S;
    const float* pl = part + (int64_t)n_heads * S + (int64_t)h * S;
    const float* pacc = part + (int64_t)n_heads * S * 2 + (int64_t)h * S * hd;
    // every split's accumulator (this kernel serves <= 32) is loaded with
    // (m, l): one round trip to memory for all of them
    constexpr int NB = 32;
    const bool lane_d = 2 * l < hd;
    float2 v[NB];
#pragma unroll
    for (int i = 0; i < NB; i++)
        v[i] = (i < S && lane_d) ? *(const float2*)(pacc + (int64_t)i * hd + 2 * l) : make_float2(0.0f, 0.0f);
    float mv[AT_MAXS / 64], lv[AT_MAXS / 64];
    float mx = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < AT_MAXS / 64; i++) {
        const int sp = l + 64 * i;
        mv[i] = sp < S ? pm[sp] : -FLT_MAX;
        lv[i] = sp < S ? pl[sp] : 0.0f;
        mx = fmaxf(mx, mv[i]);
    }
    mx = wave_max(mx);
    float L = 0.0f;
#pragma unroll
    for (int i = 0; i < AT_MAXS / 64; i++) {
        const float wgt = l + 64 * i < S ? expf(mv[i] - mx) : 0.0f;
        sW[l + 64 * i] = wgt;
        L += lv[i] * wgt;
    }
    L = wave_sum(L);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    if (!lane_d) return;
    float ox = 0.0f, oy = 0.0f;
    for (int s0 = 0; s0 < S; s0 += NB) {
        if (s0 > 0) {
#pragma unroll
            for (int i = 0; i < NB; i++)
                v[i] = s0 + i < S ? *(const float2*)(pacc + (int64_t)(s0 + i) * hd + 2 * l) : make_float2(0.0f, 0.0f);
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const float wi = s0 + i < S ? sW[s0 + i] : 0.0f;
            ox += v[i].x * wi;
            oy += v[i].y * wi;
        }
    }
    *(uint32_t*)(out + (int64_t)h * hd + 2 * l) =
        (uint32_t)f32_to_f16_bits(ox * inv) | ((uint32_t)f32_to_f16_bits(oy * inv) << 16);
}

#ifdef JLLM_ATTN_TRACE
extern "C" int jllm_hip_attn_trace_read(uint64_t* host) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_attn_trace), sizeof(g_attn_trace), 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif

hipError_t attn_launch(const AttnArgs& a, bool kv_int8, hipStream_t st) {
    if (a.tokens < 1 || a.tq < 1 || (a.tokens > 1 && a.n_splits != 1) || (a.n_splits > 1 && a.tq != 1) ||
        (a.n_heads / a.n_kv) * a.tq > (a.tq > 1 ? ATTN_MAX_COLUMNS : AT_MAXG))
        return hipErrorInvalidValue;
    dim3 grid(a.n_kv, a.n_splits, (a.tokens + a.tq - 1) / a.tq);
    const bool mt = a.tq > 1;
    const int W = a.wsplit;
    if (W < 1 || W > ATTN_MAX_WAVES) return hipErrorInvalidValue;
    if (a.qcodes && (!mt || W < 2 || a.head_dim % 32 || !a.qscl || a.q_npad < a.tokens)) return hipErrorInvalidValue;
    const size_t lds = attn_lds_bytes(a.n_heads, a.n_kv, a.head_dim, a.tq, W);
    const bool g4 = !mt && a.n_heads / a.n_kv <= 4;
#define ATTN_CASE(I8, HDV)                                                                                   \
    if (mt)      hipLaunchKernelGGL((attn_partial_kernel<I8, HDV, true, false>), grid, dim3(64 * W), lds, st, a); \
    else if (g4) hipLaunchKernelGGL((attn_partial_kernel<I8, HDV, false, true>), grid, dim3(64 * W), lds, st, a); \
    else         hipLaunchKernelGGL((attn_partial_kernel<I8, HDV, false, false>), grid, dim3(64 * W), lds, st, a);
    switch (a.head_dim * 2 + (kv_int8 ? 1 : 0)) {
    case 64:  ATTN_CASE(false, 32) break;
    case 65:  ATTN_CASE(true, 32) break;
    case 128: ATTN_CASE(false, 64) break;
    case 129: ATTN_CASE(true, 64) break;
    case 192: ATTN_CASE(false, 96) break;
    case 193: ATTN_CASE(true, 96) break;
    case 256: ATTN_CASE(false, 128) break;
    case 257: ATTN_CASE(true, 128) break;
    default: return hipErrorInvalidValue;
    }
#undef ATTN_CASE
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.n_splits == 1) return e;
    // one wave per head up to 32 splits (ctx 512: 10.4 -> 9.2 us for partial +
    // reduce), 8 waves per head beyond (128 splits: 13.0 us against 16.1)
    if (a.n_splits <= 32)
        hipLaunchKernelGGL(attn_reduce_wave_kernel, dim3(a.n_heads), dim3(64), 0, st, a.out, (const float*)a.part,
                           a.n_heads, a.n_kv, a.head_dim, a.n_splits);
    else
        hipLaunchKernelGGL(attn_reduce_kernel, dim3(a.n_heads), dim3(AT_RED_THREADS), 0, st, a.out,
                           (const float*)a.part, a.n_heads, a.n_kv, a.head_dim, a.n_splits);
    return hipGetLastError();
}

}  // namespace jllm_hip
