/*
 * kquant_oracle.c -- CPU restatement of genie-ai-runtime's quantized-matmul
 * hot path, used ONLY as the parity checker (tests/, __graft_entry__.smoke(),
 * bench.py's cpu_baseline leg).  It is test infrastructure: no product code
 * path may call it.
 *
 * Every function cites the reference source it restates (paths relative to
 * the genie-ai-runtime tree).  Arithmetic is plain IEEE fp32 with no
 * fast-math and no FMA contraction (built with -ffp-contract=off), in the
 * loop order of the cited reference code.
 *
 * Pinning (what checks each function independently of this file):
 *   orc_f16_to_f32 / orc_f32_to_f16 : numpy float16 conversions, all 65536
 *                                     patterns / 1e6 random floats.
 *   orc_get_scale_min_k4           : bit-level numpy unpack of all 16 six-bit
 *                                     fields (each of the 96 bits used once).
 *   orc_dequant_q4k/q5k/q6k        : numpy vectorised dequant written from the
 *                                     GGUF block spec; x = e_k column probes.
 *   orc_gemv_quant_cpu             : float64 numpy dot of the dequantised
 *                                     matrix; closed forms (d=0, qs=0; Q5_K
 *                                     with qh=0 equals Q4_K of the same
 *                                     header and qs, qh=0xFF adds 16*d*sc*x).
 *   orc_quantize_q8_1*             : closed forms (amax element -> +-127,
 *                                     zero block -> d=0), numpy restatement.
 *   orc_mmvq_* / orc_mmq_*         : int32 dots brute-forced in numpy int64,
 *                                     DIAG probe (A=k, B=1 -> 496).
 *   orc_attn_*                     : float64 numpy softmax attention,
 *                                     seq=1 / identical-key / window identities.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#include <float.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_K 256

/* Thread count of the row/token-parallel loops below (orc_mmvq, orc_mmq_*,
 * the prefill attention).  Each output element is computed by one thread in
 * the same operation order as the serial loop, so results do not depend on
 * it; it only makes the full-size decoder oracle finish in minutes. */
int orc_threads = 1;
void orc_set_threads(int n) { orc_threads = n > 0 ? n : 1; }

/* GGUF block layouts, gemv_q4.cu:141-164 */
#pragma pack(push, 1)
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } orc_block_q4k;   /* 144 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } orc_block_q6k;  /* 210 B */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } orc_block_q5k;  /* 176 B */
typedef struct { uint16_t d; uint16_t s; int8_t qs[32]; } orc_block_q8_1;                           /* 36 B  */
typedef struct { uint16_t ds4[8]; int8_t qs[128]; } orc_block_q8_1_mmq;                             /* 144 B */
#pragma pack(pop)

/* raw_fp16_to_float host branch, gemv_q4.cu:166-183 */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    float r;
    if (e == 0) r = ldexpf((float)m, -24);
    else if (e == 31) r = m ? NAN : INFINITY;
    else r = ldexpf((float)(m + 1024), (int)e - 25);
    return sign ? -r : r;
}

/* IEEE binary32 -> binary16, round-to-nearest-even (the semantics of CUDA's
 * __float2half used throughout the reference). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);          /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                            /* result is subnormal or 0 */
        if (ax < 0x33000000u) return (uint16_t)sign;                   /* < 2^-25 -> 0 */
        /* value = mant * 2^(e-150); in units of 2^-24 that is mant >> (126-e) */
        uint32_t e = ax >> 23, mant = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t sh = 126 - e;
        uint32_t res = mant >> sh, rem = mant & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (res & 1))) res++;
        return (uint16_t)(sign | res);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t mant = ax & 0x7FFFFFu;
    uint32_t res = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (res & 1))) res++;
    return (uint16_t)(sign | res);
}

/* get_scale_min_k4, gemv_q4.cu:185-195 */
void orc_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

/* Row dequant (fp32 values before any half rounding), decode.cu:133-223 and
 * the weight expressions of gemv_quant_cpu, gemv_q4.cu:2533-2625. */
void orc_dequant_q4k(float* out, const void* W, int64_t n_blocks) {
    const orc_block_q4k* B = (const orc_block_q4k*)W;
    for (int64_t b = 0; b < n_blocks; b++) {
        const orc_block_q4k* blk = &B[b];
        float dall = orc_f16_to_f32(blk->d), dmin = orc_f16_to_f32(blk->dmin);
        const uint8_t* q = blk->qs;
        float* o = out + b * QK_K;
        for (int j = 0, is = 0; j < QK_K; j += 64, is += 2, q += 32) {
            uint8_t sc1, m1, sc2, m2;
            orc_get_scale_min_k4(is, blk->scales, &sc1, &m1);
            orc_get_scale_min_k4(is + 1, blk->scales, &sc2, &m2);
            float d1 = dall * sc1, dm1 = dmin * m1, d2 = dall * sc2, dm2 = dmin * m2;
            for (int l = 0; l < 32; l++) o[j + l] = d1 * (q[l] & 0xF) - dm1;
            for (int l = 0; l < 32; l++) o[j + 32 + l] = d2 * (q[l] >> 4) - dm2;
        }
    }
}

/* Q5_K: the Q4_K scale/min packing plus a fifth code bit from qh (bit 2*il
 * for the low nibbles of qs[32*il..], bit 2*il+1 for the high nibbles),
 * dot_q5k_row, gemv_q4.cu:318-363. */
void orc_dequant_q5k(float* out, const void* W, int64_t n_blocks) {
    const orc_block_q5k* B = (const orc_block_q5k*)W;
    for (int64_t b = 0; b < n_blocks; b++) {
        const orc_block_q5k* blk = &B[b];
        const float dall = orc_f16_to_f32(blk->d), dmin = orc_f16_to_f32(blk->dmin);
        float* o = out + b * QK_K;
        uint8_t u1 = 1, u2 = 2;
        for (int il = 0; il < 4; il++, u1 <<= 2, u2 <<= 2) {
            uint8_t sc1, m1, sc2, m2;
            orc_get_scale_min_k4(2 * il, blk->scales, &sc1, &m1);
            orc_get_scale_min_k4(2 * il + 1, blk->scales, &sc2, &m2);
            const float d1 = dall * sc1, dm1 = dmin * m1, d2 = dall * sc2, dm2 = dmin * m2;
            const uint8_t* ql = blk->qs + 32 * il;
            for (int l = 0; l < 32; l++) {
                o[64 * il + l] = d1 * ((ql[l] & 0xF) + ((blk->qh[l] & u1) ? 16 : 0)) - dm1;
                o[64 * il + 32 + l] = d2 * ((ql[l] >> 4) + ((blk->qh[l] & u2) ? 16 : 0)) - dm2;
            }
        }
    }
}

void orc_dequant_q6k(float* out, const void* W, int64_t n_blocks) {
    const orc_block_q6k* B = (const orc_block_q6k*)W;
    for (int64_t b = 0; b < n_blocks; b++) {
        const orc_block_q6k* blk = &B[b];
        float d = orc_f16_to_f32(blk->d);
        const uint8_t* ql = blk->ql; const uint8_t* qh = blk->qh; const int8_t* sc = blk->scales;
        float* o = out + b * QK_K;
        for (int n = 0; n < QK_K; n += 128, ql += 64, qh += 32, sc += 8) {
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                o[n + l]      = d * (float)sc[is + 0] * (float)q1;
                o[n + l + 32] = d * (float)sc[is + 2] * (float)q2;
                o[n + l + 64] = d * (float)sc[is + 4] * (float)q3;
                o[n + l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}

/* gemv_quant_cpu, gemv_q4.cu:2519-2631 (Q4_K, Q5_K and Q6_K branches): one row at
 * a time, fp32 accumulator, fp16 activations widened per element. Returns 0
 * on success, -1 for an unsupported type (the reference prints FATAL and the
 * caller zero-fills y). row0/row1 select a row range so a threaded caller can
 * split rows exactly as an OpenMP row split would. */
static void gemv_rows(float* y, const void* W, int type, const uint16_t* x, int64_t r0, int64_t r1, int K) {
    const int nb = K / QK_K;
    for (int64_t row = r0; row < r1; row++) {
        float acc = 0.0f;
        if (type == 12) {
            const orc_block_q4k* rb = (const orc_block_q4k*)W + row * nb;
            for (int b = 0; b < nb; b++) {
                const orc_block_q4k* blk = &rb[b];
                const float dall = orc_f16_to_f32(blk->d), dmin = orc_f16_to_f32(blk->dmin);
                const uint8_t* q = blk->qs;
                int is = 0, k = b * QK_K;
                for (int j = 0; j < QK_K; j += 64) {
                    uint8_t sc1, m1, sc2, m2;
                    orc_get_scale_min_k4(is + 0, blk->scales, &sc1, &m1);
                    orc_get_scale_min_k4(is + 1, blk->scales, &sc2, &m2);
                    const float d1 = dall * sc1, dm1 = dmin * m1, d2 = dall * sc2, dm2 = dmin * m2;
                    for (int l = 0; l < 32; l++) acc += (d1 * (q[l] & 0xF) - dm1) * orc_f16_to_f32(x[k + l]);
                    for (int l = 0; l < 32; l++) acc += (d2 * (q[l] >> 4) - dm2) * orc_f16_to_f32(x[k + 32 + l]);
                    q += 32; is += 2; k += 64;
                }
            }
        } else if (type == 13) {
            const orc_block_q5k* rb = (const orc_block_q5k*)W + row * nb;
            for (int b = 0; b < nb; b++) {
                const orc_block_q5k* blk = &rb[b];
                const float dall = orc_f16_to_f32(blk->d), dmin = orc_f16_to_f32(blk->dmin);
                const uint8_t* ql = blk->qs; const uint8_t* qh = blk->qh;
                uint8_t u1 = 1, u2 = 2;
                int is = 0, k = b * QK_K;
                for (int j = 0; j < QK_K; j += 64) {
                    uint8_t sc1, m1, sc2, m2;
                    orc_get_scale_min_k4(is + 0, blk->scales, &sc1, &m1);
                    orc_get_scale_min_k4(is + 1, blk->scales, &sc2, &m2);
                    const float d1 = dall * sc1, dm1 = dmin * m1, d2 = dall * sc2, dm2 = dmin * m2;
                    for (int l = 0; l < 32; l++)
                        acc += (d1 * ((ql[l] & 0xF) + ((qh[l] & u1) ? 16 : 0)) - dm1) * orc_f16_to_f32(x[k + l]);
                    for (int l = 0; l < 32; l++)
                        acc += (d2 * ((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) - dm2) * orc_f16_to_f32(x[k + 32 + l]);
                    ql += 32; is += 2; u1 <<= 2; u2 <<= 2; k += 64;
                }
            }
        } else {
            const orc_block_q6k* rb = (const orc_block_q6k*)W + row * nb;
            for (int b = 0; b < nb; b++) {
                const orc_block_q6k* blk = &rb[b];
                const float d = orc_f16_to_f32(blk->d);
                const uint8_t* ql = blk->ql; const uint8_t* qh = blk->qh; const int8_t* sc = blk->scales;
                const int kb = b * QK_K;
                for (int n = 0; n < QK_K; n += 128) {
                    for (int l = 0; l < 32; l++) {
                        const int is = l / 16;
                        const int q1 = (int)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = (int)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        const int k = kb + n + l;
                        acc += d * (float)sc[is + 0] * (float)q1 * orc_f16_to_f32(x[k + 0]);
                        acc += d * (float)sc[is + 2] * (float)q2 * orc_f16_to_f32(x[k + 32]);
                        acc += d * (float)sc[is + 4] * (float)q3 * orc_f16_to_f32(x[k + 64]);
                        acc += d * (float)sc[is + 6] * (float)q4 * orc_f16_to_f32(x[k + 96]);
                    }
                    ql += 64; qh += 32; sc += 8;
                }
            }
        }
        y[row] = acc;
    }
}

int orc_gemv_quant_cpu(float* y, const void* W, int type, const uint16_t* x, int M, int K) {
    if (type < 12 || type > 14) return -1;
    gemv_rows(y, W, type, x, 0, M, K);
    return 0;
}

/* Same arithmetic per row, rows split over `threads` OpenMP threads (the
 * all-cores CPU baseline; per-row results are identical to the 1-core path). */
int orc_gemv_quant_cpu_mt(float* y, const void* W, int type, const uint16_t* x, int M, int K, int threads) {
    if (type < 12 || type > 14) return -1;
#ifdef _OPENMP
    #pragma omp parallel for num_threads(threads) schedule(static)
    for (int t = 0; t < threads; t++) {
        int64_t r0 = (int64_t)M * t / threads, r1 = (int64_t)M * (t + 1) / threads;
        gemv_rows(y, W, type, x, r0, r1, K);
    }
#else
    (void)threads;
    gemv_rows(y, W, type, x, 0, M, K);
#endif
    return 0;
}

/* quantize_q8_1_kernel, gemv_q4.cu:445-466 (host mirror host_q8_1,
 * test_mmq_q4k_int8.cu:374-388): d = amax/127, q = rn(v*(1/d)) clamped to
 * +-127, s = d*sum(q); d and s stored as fp16 (RNE). */
void orc_quantize_q8_1(const uint16_t* x, void* out, int K) {
    orc_block_q8_1* y = (orc_block_q8_1*)out;
    for (int b = 0; b < K / 32; b++) {
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(orc_f16_to_f32(x[b * 32 + i])));
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        int sumq = 0;
        for (int i = 0; i < 32; i++) {
            int q = (int)nearbyintf(orc_f16_to_f32(x[b * 32 + i]) * id);
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            y[b].qs[i] = (int8_t)q; sumq += q;
        }
        y[b].d = orc_f32_to_f16(d);
        y[b].s = orc_f32_to_f16(d * (float)sumq);
    }
}

/* Sum of 32 floats in the order of a 5-step xor butterfly (offsets 16,8,4,2,1),
 * the order quantize_mmq_q8_1_ds4's __shfl_xor_sync reduction produces. */
static float butterfly_sum32(const float* v) {
    float a[32];
    for (int i = 0; i < 32; i++) a[i] = v[i];
    for (int o = 16; o > 0; o >>= 1) {
        float b[32];
        for (int i = 0; i < 32; i++) b[i] = a[i] + a[i ^ o];
        memcpy(a, b, sizeof(a));
    }
    return a[0];
}

/* quantize_mmq_q8_1_ds4, mmq_q4k_llama.cu:383-404 (ds4 = 1) and
 * quantize_mmq_q8_1_d4, mmq_q6k_llama.cu:424-438 (ds4 = 0): per 32 values
 * d = amax/127, q = rn(v*(1/d)) WITHOUT clamp; DS4 stores half2(d, sum v),
 * D4 stores float d.  Output layout [K/128][Npad] blocks of 144 B; columns
 * >= N are all-zero. */
void orc_quantize_mmq(const uint16_t* x, void* out, int N, int K, int Npad, int ds4) {
    orc_block_q8_1_mmq* y = (orc_block_q8_1_mmq*)out;
    memset(out, 0, (size_t)(K / 128) * Npad * sizeof(orc_block_q8_1_mmq));
    for (int kb = 0; kb < K / 128; kb++)
        for (int col = 0; col < Npad; col++) {
            orc_block_q8_1_mmq* blk = &y[(int64_t)kb * Npad + col];
            for (int sub = 0; sub < 4; sub++) {
                float v[32], amax = 0.0f;
                for (int l = 0; l < 32; l++) {
                    v[l] = col < N ? orc_f16_to_f32(x[(int64_t)col * K + kb * 128 + sub * 32 + l]) : 0.0f;
                    amax = fmaxf(amax, fabsf(v[l]));
                }
                const float d = amax / 127.0f;
                const float dinv = d > 0.0f ? 1.0f / d : 0.0f;
                for (int l = 0; l < 32; l++) blk->qs[sub * 32 + l] = (int8_t)(int)nearbyintf(v[l] * dinv);
                if (ds4) {
                    blk->ds4[2 * sub] = orc_f32_to_f16(d);
                    blk->ds4[2 * sub + 1] = orc_f32_to_f16(butterfly_sum32(v));
                } else {
                    memcpy(&blk->ds4[2 * sub], &d, 4);
                }
            }
        }
}

/* MMVQ Q4_K x q8_1, dot_q4k_row_q8_1 (gemv_q4.cu:474-502): per 32-weight
 * sub-block an exact int32 dot, then acc += dall*sc*(d8*dot) - dmin*m*s8,
 * sub-blocks in ascending order. */
float orc_mmvq_q4k_row(const void* Wrow, const void* xq, int K) {
    const orc_block_q4k* row = (const orc_block_q4k*)Wrow;
    const orc_block_q8_1* q8 = (const orc_block_q8_1*)xq;
    float acc = 0.0f;
    for (int s = 0; s < K / 32; s++) {
        const orc_block_q4k* blk = &row[s >> 3];
        const int j = s & 7, il = j >> 1, hi = j & 1;
        uint8_t sc, m; orc_get_scale_min_k4(j, blk->scales, &sc, &m);
        int dot = 0;
        for (int e = 0; e < 32; e++) {
            const uint8_t qb = blk->qs[32 * il + e];
            dot += (hi ? (qb >> 4) : (qb & 0xF)) * (int)q8[s].qs[e];
        }
        const float dall = orc_f16_to_f32(blk->d), dmin = orc_f16_to_f32(blk->dmin);
        const float d8 = orc_f16_to_f32(q8[s].d), s8 = orc_f16_to_f32(q8[s].s);
        acc += dall * sc * (d8 * dot) - dmin * m * s8;
    }
    return acc;
}

/* Q6_K element value q6-32 at position p of a block (the unpack of
 * q6_unpack4, gemv_q4.cu:562-575, element-wise). */
static int q6_val(const orc_block_q6k* blk, int p) {
    const int n = p >= 128 ? 1 : 0, ph = p & 127, g = ph >> 5, r = ph & 31;
    const uint8_t* ql = blk->ql + 64 * n; const uint8_t* qh = blk->qh + 32 * n;
    const int lo = (g & 1) ? ql[r + 32] : ql[r];
    const int nib = (g >= 2) ? (lo >> 4) : (lo & 0xF);
    const int h = (qh[r] >> (2 * g)) & 3;
    return (nib | (h << 4)) - 32;
}

/* MMVQ Q6_K x q8_1, dot_q6k_row_q8_1 (gemv_q4.cu:581-618): per group of 4
 * weights an int32 dot, acc += d*sc*(d8*dot), groups in ascending order. */
float orc_mmvq_q6k_row(const void* Wrow, const void* xq, int K) {
    const orc_block_q6k* row = (const orc_block_q6k*)Wrow;
    const orc_block_q8_1* q8 = (const orc_block_q8_1*)xq;
    float acc = 0.0f;
    for (int sb = 0; sb < K / QK_K; sb++) {
        const orc_block_q6k* blk = &row[sb];
        const float d = orc_f16_to_f32(blk->d);
        for (int gi = 0; gi < 64; gi++) {
            const int p = 4 * gi;
            const orc_block_q8_1* qb = &q8[sb * 8 + (p >> 5)];
            int dot = 0;
            for (int e = 0; e < 4; e++) dot += q6_val(blk, p + e) * (int)qb->qs[(p & 31) + e];
            const int sc = blk->scales[p >> 4];
            const float d8 = orc_f16_to_f32(qb->d);
            acc += d * sc * (d8 * (float)dot);
        }
    }
    return acc;
}

void orc_mmvq(float* y, const void* W, int type, const void* xq, int M, int K) {
    const int nb = K / QK_K;
    #pragma omp parallel for num_threads(orc_threads) schedule(static)
    for (int r = 0; r < M; r++) {
        if (type == 12) y[r] = orc_mmvq_q4k_row((const orc_block_q4k*)W + (int64_t)r * nb, xq, K);
        else            y[r] = orc_mmvq_q6k_row((const orc_block_q6k*)W + (int64_t)r * nb, xq, K);
    }
}

/* Raw int32 sub-block dots of the int8 MMQ: Q4_K (type 12) -> one per 32-K
 * sub-block, C = sum q4*q8;  Q6_K (type 14) -> one per 16-K group,
 * C = sum (q6-32)*q8.  out layout [N][M][K/G].  q8 is the [K/128][Npad]
 * mmq layout. */
void orc_mmq_subdots(int32_t* out, const void* W, int type, const void* q8v, int M, int N, int K, int Npad) {
    const orc_block_q8_1_mmq* q8 = (const orc_block_q8_1_mmq*)q8v;
    const int nb = K / QK_K, G = type == 12 ? 32 : 16, ng = K / G;
    for (int t = 0; t < N; t++)
        for (int r = 0; r < M; r++)
            for (int g = 0; g < ng; g++) {
                const int k0 = g * G;
                const int kb = k0 / 128;
                const orc_block_q8_1_mmq* qb = &q8[(int64_t)kb * Npad + t];
                int dot = 0;
                for (int e = 0; e < G; e++) {
                    const int k = k0 + e, b = k / QK_K, p = k % QK_K;
                    int w;
                    if (type == 12) {
                        const orc_block_q4k* blk = (const orc_block_q4k*)W + (int64_t)r * nb + b;
                        const int j = p >> 5, il = j >> 1, pos = p & 31;
                        const uint8_t byte = blk->qs[32 * il + pos];
                        w = (j & 1) ? (byte >> 4) : (byte & 0xF);
                    } else {
                        w = q6_val((const orc_block_q6k*)W + (int64_t)r * nb + b, p);
                    }
                    dot += w * (int)qb->qs[k % 128];
                }
                out[((int64_t)t * M + r) * ng + g] = dot;
            }
}

/* Q4_K int8 MMQ, mul_mat_q_llama + vec_dot_q8_1_q8_1_mma (SM 8.x path)
 * mmq_q4k_llama.cu:92-453: per (token t, row r), per super-block, per
 * 32-sub-block j ascending:
 *   sum += (dmA.x*dsB.x)*C ; sum += dmA.y*dsB.y
 * with dmA = (half(d*sc), half(-dmin*m)) (half products, :159-163) and
 * dsB = (d8, sum x) from the DS4 block.  y[t][r] = sum (fp32). */
void orc_mmq_q4k(float* y, const void* W, const void* q8v, int M, int N, int K, int Npad) {
    const orc_block_q8_1_mmq* q8 = (const orc_block_q8_1_mmq*)q8v;
    const int nb = K / QK_K;
    #pragma omp parallel for collapse(2) num_threads(orc_threads) schedule(static)
    for (int t = 0; t < N; t++)
        for (int r = 0; r < M; r++) {
            float sum = 0.0f;
            for (int b = 0; b < nb; b++) {
                const orc_block_q4k* blk = (const orc_block_q4k*)W + (int64_t)r * nb + b;
                const float d = orc_f16_to_f32(blk->d), dmin = orc_f16_to_f32(blk->dmin);
                for (int j = 0; j < 8; j++) {
                    uint8_t sc, m; orc_get_scale_min_k4(j, blk->scales, &sc, &m);
                    const float ax = orc_f16_to_f32(orc_f32_to_f16(d * (float)sc));
                    const float ay = orc_f16_to_f32(orc_f32_to_f16(-dmin * (float)m));
                    const int kglob = b * QK_K + j * 32;
                    const orc_block_q8_1_mmq* qb = &q8[(int64_t)(kglob / 128) * Npad + t];
                    const int sub = (kglob % 128) / 32;
                    const float bx = orc_f16_to_f32(qb->ds4[2 * sub]), by = orc_f16_to_f32(qb->ds4[2 * sub + 1]);
                    int C = 0;
                    const int il = j >> 1;
                    for (int e = 0; e < 32; e++) {
                        const uint8_t byte = blk->qs[32 * il + e];
                        const int w = (j & 1) ? (byte >> 4) : (byte & 0xF);
                        C += w * (int)qb->qs[sub * 32 + e];
                    }
                    sum += ax * bx * (float)C;
                    sum += ay * by;
                }
            }
            y[(int64_t)t * M + r] = sum;
        }
}

/* Q6_K int8 MMQ, mul_mat_q6k_llama + vec_dot_q6_K_q8_1_mma SM 8.x path
 * (mmq_q6k_llama.cu:264-364): per super-block, per 128-half h, tmp = 0; for
 * each 32-block s: tmp += (float)(C0*sc0 + C1*sc1) * d8 (C0,C1 the two
 * 16-group int dots); then sum += tmp * d(block). */
void orc_mmq_q6k(float* y, const void* W, const void* q8v, int M, int N, int K, int Npad) {
    const orc_block_q8_1_mmq* q8 = (const orc_block_q8_1_mmq*)q8v;
    const int nb = K / QK_K;
    #pragma omp parallel for collapse(2) num_threads(orc_threads) schedule(static)
    for (int t = 0; t < N; t++)
        for (int r = 0; r < M; r++) {
            float sum = 0.0f;
            for (int b = 0; b < nb; b++) {
                const orc_block_q6k* blk = (const orc_block_q6k*)W + (int64_t)r * nb + b;
                const float dA = orc_f16_to_f32(blk->d);
                for (int h = 0; h < 2; h++) {
                    const orc_block_q8_1_mmq* qb = &q8[(int64_t)(b * 2 + h) * Npad + t];
                    float tmp = 0.0f;
                    for (int s = 0; s < 4; s++) {
                        int C[2] = {0, 0};
                        for (int g = 0; g < 2; g++)
                            for (int e = 0; e < 16; e++) {
                                const int p = h * 128 + s * 32 + g * 16 + e;
                                C[g] += q6_val(blk, p) * (int)qb->qs[s * 32 + g * 16 + e];
                            }
                        const int sc0 = blk->scales[h * 8 + 2 * s], sc1 = blk->scales[h * 8 + 2 * s + 1];
                        float dB; memcpy(&dB, &qb->ds4[2 * s], 4);
                        tmp += (float)(C[0] * sc0 + C[1] * sc1) * dB;
                    }
                    sum += tmp * dA;
                }
            }
            y[(int64_t)t * M + r] = sum;
        }
}

/* fp16_to_int8_kernel, convert.cu:26-69: per row scale = absmax/127,
 * q = rn(v * (127/absmax)) clamped to +-127 (inv = 0 when absmax = 0). */
void orc_fp16_to_int8(int8_t* dst, float* scale_out, const uint16_t* src, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        float mx = 0.0f;
        for (int c = 0; c < cols; c++) mx = fmaxf(mx, fabsf(orc_f16_to_f32(src[(int64_t)r * cols + c])));
        const float scale = mx / 127.0f;
        const float inv = scale > 0.0f ? 127.0f / mx : 0.0f;
        if (scale_out) scale_out[r] = scale;
        for (int c = 0; c < cols; c++) {
            int q = (int)nearbyintf(orc_f16_to_f32(src[(int64_t)r * cols + c]) * inv);
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            dst[(int64_t)r * cols + c] = (int8_t)q;
        }
    }
}

/* decode_attn_splits, attention.cu:1000-1005 */
int orc_decode_attn_splits(int seq_len) { return seq_len < 64 ? 1 : (seq_len < 128 ? 4 : 8); }

/* INT8-KV split-K flash decode: flash_decode_splitk_partial_kernel
 * (attention.cu:837-941) then flash_decode_reduce_kernel (:944-969);
 * n_splits = 1 is the single-block kernel (:244-380, same tile math).
 * Per (head, split): kv range [s*per, min((s+1)*per, seq)), per =
 * ceil(seq/n_splits); 64-key tiles; score = (sum_d q[d]*(k[d]*ks))*scale,
 * window-masked positions -> -inf; online softmax with running max m
 * (init -FLT_MAX), correction expf(m_old - m_new); acc[d] += sum_t p_t*(v*vs).
 * Reduce: M = max m_s, L = sum l_s*e^(m_s-M), out = half(sum acc_s*e^(m_s-M) / L).
 * k/v: int8 [pos][n_kv*cache_head_dim]; ks/vs: fp32 [pos][n_kv]. */
void orc_attn_decode_int8(uint16_t* out, const uint16_t* q, const int8_t* kc, const int8_t* vc,
                          int n_heads, int n_kv, int hd, int chd, int seq, float scale,
                          const float* ks, const float* vs, int window, int n_splits) {
    const int kv_dim = n_kv * chd;
    float* pm = (float*)malloc(sizeof(float) * n_splits);
    float* pl = (float*)malloc(sizeof(float) * n_splits);
    float* pacc = (float*)malloc(sizeof(float) * n_splits * hd);
    float* sq = (float*)malloc(sizeof(float) * hd);
    float sc[64];
    for (int h = 0; h < n_heads; h++) {
        const int kvh = h / (n_heads / n_kv), hoff = kvh * chd;
        for (int d = 0; d < hd; d++) sq[d] = orc_f16_to_f32(q[h * hd + d]);
        const int per = (seq + n_splits - 1) / n_splits;
        for (int s = 0; s < n_splits; s++) {
            const int kv0 = s * per, kv1 = kv0 + per < seq ? kv0 + per : seq;
            float* acc = pacc + (int64_t)s * hd;
            for (int d = 0; d < hd; d++) acc[d] = 0.0f;
            float m = -FLT_MAX, l = 0.0f;
            if (kv0 >= kv1) { pm[s] = -FLT_MAX; pl[s] = 0.0f; continue; }
            for (int t0 = kv0; t0 < kv1; t0 += 64) {
                const int tl = (kv1 - t0) < 64 ? (kv1 - t0) : 64;
                for (int t = 0; t < tl; t++) {
                    const int pos = t0 + t;
                    if (window > 0 && pos < seq - window) { sc[t] = -INFINITY; continue; }
                    const int8_t* kr = kc + (int64_t)pos * kv_dim + hoff;
                    const float kscale = ks ? ks[(int64_t)pos * n_kv + kvh] : 1.0f;
                    float dot = 0.0f;
                    for (int d = 0; d < hd; d++) dot += sq[d] * ((float)kr[d] * kscale);
                    sc[t] = dot * scale;
                }
                float tmax = -FLT_MAX;
                for (int t = 0; t < tl; t++) tmax = fmaxf(tmax, sc[t]);
                const float om = m;
                m = fmaxf(m, tmax);
                const float corr = expf(om - m);
                l *= corr;
                for (int d = 0; d < hd; d++) acc[d] *= corr;
                float tsum = 0.0f;
                for (int t = 0; t < tl; t++) { sc[t] = expf(sc[t] - m); tsum += sc[t]; }
                l += tsum;
                for (int d = 0; d < hd; d++) {
                    float v = 0.0f;
                    for (int t = 0; t < tl; t++) {
                        const int pos = t0 + t;
                        const float vscale = vs ? vs[(int64_t)pos * n_kv + kvh] : 1.0f;
                        v += sc[t] * ((float)vc[(int64_t)pos * kv_dim + hoff + d] * vscale);
                    }
                    acc[d] += v;
                }
            }
            pm[s] = m; pl[s] = l;
        }
        float M = -FLT_MAX, L = 0.0f;
        for (int s = 0; s < n_splits; s++) M = fmaxf(M, pm[s]);
        for (int s = 0; s < n_splits; s++) L += pl[s] * expf(pm[s] - M);
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        for (int d = 0; d < hd; d++) {
            float a = 0.0f;
            for (int s = 0; s < n_splits; s++) a += pacc[(int64_t)s * hd + d] * expf(pm[s] - M);
            out[h * hd + d] = orc_f32_to_f16(a * inv);
        }
    }
    free(pm); free(pl); free(pacc); free(sq);
}
