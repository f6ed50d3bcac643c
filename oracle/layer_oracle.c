/*
 * layer_oracle.c -- CPU restatement of the decoder-layer operations around
 * genie-ai-runtime's quantized matmuls (RMSNorm, SwiGLU, residual add, RoPE,
 * embedding-row dequant, greedy argmax, prefill attention).  TEST
 * INFRASTRUCTURE ONLY: used as the checker by tests/ and
 * __graft_entry__.smoke(); no product code path may call it.
 *
 * Plain IEEE fp32, no FMA contraction (-ffp-contract=off), in the operation
 * order of the cited reference code; fp16 results round to nearest even.
 *
 * Pinning (independent checks, tests/test_oracle_layer_pins.py):
 *   orc_rmsnorm    : tests/test_kernels.cu known answer (x + res = 2, w = 1
 *                    -> 1.0); closed forms for a constant row and a one-hot
 *                    row (catch the dim/eps placement, a dropped residual,
 *                    a wrong weight index); float64 numpy.
 *   orc_swiglu     : test_kernels.cu known answer silu(1) * 2 = 1.4621;
 *                    silu(0) = 0; float64 numpy.
 *   orc_rope       : position 0 is the identity (test_kernels.cu); pair norm
 *                    preserved; one-hot input gives (cos, sin) of
 *                    position * theta^(-2i/hd) at (i, i + hd/2) (neox) or
 *                    (2i, 2i+1) in float64; composition R(a)R(b) = R(a+b).
 *   orc_embed_row  : the dequant oracle pinned in kquant_oracle.c.
 *   orc_argmax     : numpy argmax over the finite values (first index).
 *   orc_attn_prefill: float64 numpy causal softmax attention.
 *   orc_geglu      : |gelu_tanh(g) - g*Phi(g)| <= 5e-4 against the exact
 *                    erf GELU (float64), odd part gelu(g) - gelu(-g) = g,
 *                    u = 0 -> 0.
 *   orc_vec_scale  : numpy float16 products (one rounding of the exact
 *                    product) for pairs, float32 for a trailing element.
 *   orc_logit_softcap: float64 cap * tanh(x / cap); |x| << cap -> x.
 *   orc_softmax    : float64 softmax; shift invariance; sums to 1.
 *   orc_dense      : float64 numpy dot of the widened weights (bf16 via
 *                    torch's bfloat16 conversion).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_dequant_q4k(float* out, const void* W, int64_t n_blocks);
void orc_dequant_q6k(float* out, const void* W, int64_t n_blocks);
void orc_dequant_q5k(float* out, const void* W, int64_t n_blocks);
void orc_attn_decode_int8(uint16_t* out, const uint16_t* q, const int8_t* kc, const int8_t* vc,
                          int n_heads, int n_kv, int hd, int chd, int seq, float scale,
                          const float* ks, const float* vs, int window, int n_splits);
extern int orc_threads;


/* fused_rmsnorm_residual_kernel, fused_norm.cu:33-101: v = x + residual
 * (fp32), rrms = 1/sqrt(sum v^2 / dim + eps), out = half(v * rrms * w).
 * The sum of squares runs in row order here (the kernel's is a strided
 * tree; both are fp32). */
void orc_rmsnorm(uint16_t* out, const uint16_t* x, const uint16_t* res, const void* w, int rows, int dim,
                 float eps, int w_fp32) {
    float* v = (float*)malloc(sizeof(float) * (size_t)dim);
    for (int r = 0; r < rows; r++) {
        const int64_t off = (int64_t)r * dim;
        float ss = 0.0f;
        for (int i = 0; i < dim; i++) {
            v[i] = orc_f16_to_f32(x[off + i]);
            if (res) v[i] += orc_f16_to_f32(res[off + i]);
            ss += v[i] * v[i];
        }
        const float rrms = 1.0f / sqrtf(ss / (float)dim + eps);
        for (int i = 0; i < dim; i++) {
            const float wi = w_fp32 ? ((const float*)w)[i] : orc_f16_to_f32(((const uint16_t*)w)[i]);
            out[off + i] = orc_f32_to_f16(v[i] * rrms * wi);
        }
    }
    free(v);
}

/* swiglu_kernel, convert.cu:85-106: out = half(g / (1 + expf(-g)) * u). */
void orc_swiglu(uint16_t* out, const uint16_t* gate, const uint16_t* up, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const float g = orc_f16_to_f32(gate[i]), u = orc_f16_to_f32(up[i]);
        out[i] = orc_f32_to_f16(g / (1.0f + expf(-g)) * u);
    }
}

/* vec_add_kernel, src/engine/decode.cu:60-71: out = half(a + b). */
void orc_vec_add(uint16_t* out, const uint16_t* a, const uint16_t* b, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(orc_f16_to_f32(a[i]) + orc_f16_to_f32(b[i]));
}

/* rope_kernel, rope.cu:322-367 (and the batched form :476-497, position =
 * start_pos + t): freq = 1 / powf(theta, (2i)/hd), angle = position * freq
 * in fp32, (v0, v1) -> (half(v0 c - v1 s), half(v0 s + v1 c)) for the pair
 * (i, i + hd/2) when neox, else (2i, 2i+1).  k may be NULL. */
void orc_rope(uint16_t* q, uint16_t* k, int n_heads, int n_kv, int hd, int start_pos, int N, int q_stride,
              int k_stride, float theta, int neox) {
    const int h2 = hd / 2;
    for (int t = 0; t < N; t++)
        for (int head = 0; head < n_heads + (k ? n_kv : 0); head++) {
            uint16_t* p = head < n_heads ? q + (int64_t)t * q_stride + (int64_t)head * hd
                                         : k + (int64_t)t * k_stride + (int64_t)(head - n_heads) * hd;
            for (int i = 0; i < h2; i++) {
                const float freq = 1.0f / powf(theta, (2.0f * (float)i) / (float)hd);
                const float ang = (float)(start_pos + t) * freq;
                const float c = cosf(ang), s = sinf(ang);
                const int i0 = neox ? i : 2 * i, i1 = neox ? i + h2 : 2 * i + 1;
                const float v0 = orc_f16_to_f32(p[i0]), v1 = orc_f16_to_f32(p[i1]);
                p[i0] = orc_f32_to_f16(v0 * c - v1 * s);
                p[i1] = orc_f32_to_f16(v0 * s + v1 * c);
            }
        }
}

/* The engine's attention front, src/engine/decode.cu:1441-1478 (decode) and
 * :1795-1842 (prefill), for N tokens: q_norm / k_norm RMSNorm per head
 * (when q_norm is not NULL) -> rope_inplace -> fp16_to_int8 of k and v
 * (kv_int8) or fp16 copies, into the cache rows of positions start_pos + t
 * ([pos][n_kv * chd]; scales [pos][n_kv]).  q and k are updated in place. */
void orc_fp16_to_int8(int8_t* dst, float* scale_out, const uint16_t* src, int rows, int cols);
void orc_qk_post(uint16_t* q, uint16_t* k, const uint16_t* v, const void* q_norm, const void* k_norm,
                 int norm_fp32, float eps, void* k_cache, void* v_cache, float* k_scales, float* v_scales,
                 int n_heads, int n_kv, int hd, int chd, int start_pos, int N, float theta, int neox, int kv_int8) {
    const int qd = n_heads * hd, kd = n_kv * hd;
    if (q_norm) {
        orc_rmsnorm(q, q, NULL, q_norm, N * n_heads, hd, eps, norm_fp32);
        orc_rmsnorm(k, k, NULL, k_norm, N * n_kv, hd, eps, norm_fp32);
    }
    orc_rope(q, k, n_heads, n_kv, hd, start_pos, N, qd, kd, theta, neox);
    int8_t* tmp = (int8_t*)malloc((size_t)kd);
    for (int t = 0; t < N; t++) {
        const int64_t pos = start_pos + t;
        for (int which = 0; which < 2; which++) {
            const uint16_t* src = (which ? v : k) + (int64_t)t * kd;
            void* cache = which ? v_cache : k_cache;
            if (kv_int8) {
                float* sc = which ? v_scales : k_scales;
                float scl[256];
                orc_fp16_to_int8(tmp, scl, src, n_kv, hd);
                for (int h = 0; h < n_kv; h++) {
                    memcpy((int8_t*)cache + (pos * n_kv + h) * chd, tmp + (int64_t)h * hd, (size_t)hd);
                    if (sc) sc[pos * n_kv + h] = scl[h];
                }
            } else {
                for (int h = 0; h < n_kv; h++)
                    memcpy((uint16_t*)cache + (pos * n_kv + h) * chd, src + (int64_t)h * hd, (size_t)hd * 2);
            }
        }
    }
    free(tmp);
}

/* dequant_embedding_q4k_kernel / _q6k_kernel, gemv_q4.cu:793-864, and the
 * engine's host Q5_K row dequant, decode.cu:230-266: dst = half(dequantised
 * row token of the table); same fp32 expressions as the row dequant
 * (dall*sc*q - dmin*m; d*sc*(q-32)). */
void orc_embed_row(uint16_t* dst, const void* W, int type, int token, int hidden) {
    const int nb = hidden / 256;
    float* row = (float*)malloc(sizeof(float) * (size_t)hidden);
    if (type == 12) orc_dequant_q4k(row, (const uint8_t*)W + (int64_t)token * nb * 144, nb);
    else if (type == 13) orc_dequant_q5k(row, (const uint8_t*)W + (int64_t)token * nb * 176, nb);
    else orc_dequant_q6k(row, (const uint8_t*)W + (int64_t)token * nb * 210, nb);
    for (int i = 0; i < hidden; i++) dst[i] = orc_f32_to_f16(row[i]);
    free(row);
}

/* sample_greedy, src/engine/sample.cpp:160-170: the first index holding the
 * largest finite value; 0 when none is finite. */
int orc_argmax(const float* x, int n) {
    int best = 0;
    float bv = -INFINITY;
    for (int i = 0; i < n; i++)
        if (isfinite(x[i]) && x[i] > bv) { best = i; bv = x[i]; }
    return best;
}

/* flash_attention_prefill_batched_kernel, attention.cu:382-514: query token
 * t (position start_pos + t) runs the single-block online-softmax loop over
 * keys [0, start_pos + t] in 64-key tiles -- the computation of the decode
 * kernel with seq = start_pos + t + 1 and one split (orc_attn_decode_int8,
 * n_splits = 1).  q, out: [N][n_heads * hd]. */
void orc_attn_prefill_int8(uint16_t* out, const uint16_t* q, const int8_t* kc, const int8_t* vc, int n_heads,
                           int n_kv, int hd, int chd, int N, int start_pos, float scale, const float* ks,
                           const float* vs, int window) {
    const int64_t qd = (int64_t)n_heads * hd;
    #pragma omp parallel for num_threads(orc_threads) schedule(dynamic)
    for (int t = 0; t < N; t++)
        orc_attn_decode_int8(out + t * qd, q + t * qd, kc, vc, n_heads, n_kv, hd, chd, start_pos + t + 1, scale, ks,
                             vs, window, 1);
}

/* ---- kernels outside the Llama/Qwen decode path (Gemma family, logits) ---- */

/* geglu_kernel, convert.cu:121-151: out = half(gelu_tanh(g) * u),
 * gelu_tanh(g) = 0.5*g*(1 + tanhf(0.7978845608028654*(g + 0.044715*g*g*g))). */
void orc_geglu(uint16_t* out, const uint16_t* gate, const uint16_t* up, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const float g = orc_f16_to_f32(gate[i]), u = orc_f16_to_f32(up[i]);
        const float gl = 0.5f * g * (1.0f + tanhf(0.7978845608028654f * (g + 0.044715f * g * g * g)));
        out[i] = orc_f32_to_f16(gl * u);
    }
}

/* vec_scale_kernel, convert.cu:155-170: pairs (2i, 2i+1) with 2i+1 < n are
 * multiplied in fp16 by half(s) (__hmul2: the exact product rounded once);
 * a trailing odd element in fp32 by s. */
void orc_vec_scale(uint16_t* x, int64_t n, float s) {
    const float sh = orc_f16_to_f32(orc_f32_to_f16(s));
    for (int64_t i = 0; i < n; i++) {
        const float f = (i < (n & ~(int64_t)1)) ? sh : s;
        x[i] = orc_f32_to_f16(orc_f16_to_f32(x[i]) * f);
    }
}

/* logit_softcap_kernel, convert.cu:173-181: x = cap * tanhf(x / cap). */
void orc_logit_softcap(float* x, int64_t n, float cap) {
    for (int64_t i = 0; i < n; i++) x[i] = cap * tanhf(x[i] / cap);
}

/* softmax_kernel, softmax.cu:15-81: max, e = expf(x - max) with its sum,
 * then x = e * (1/sum) (sums here in index order). */
void orc_softmax(float* x, int n) {
    float m = -FLT_MAX;
    for (int i = 0; i < n; i++) m = fmaxf(m, x[i]);
    float s = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - m); s += x[i]; }
    const float inv = 1.0f / s;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* gemv_dense_kernel / gemm_dense_batched_kernel, gemv_q4.cu:2815-2885:
 * out[t][m] = half(sum_k w(m, k) * x[t][k]), w from F32 (wtype 0), F16 (1)
 * or BF16 (30, the high half of an fp32), fp32 sum in k order. */
void orc_dense(uint16_t* out, const void* W, int wtype, const uint16_t* x, int M, int N, int K) {
    for (int t = 0; t < N; t++)
        for (int m = 0; m < M; m++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) {
                const int64_t i = (int64_t)m * K + k;
                float w;
                if (wtype == 0) w = ((const float*)W)[i];
                else if (wtype == 1) w = orc_f16_to_f32(((const uint16_t*)W)[i]);
                else { const uint32_t b = (uint32_t)((const uint16_t*)W)[i] << 16; memcpy(&w, &b, 4); }
                acc += w * orc_f16_to_f32(x[(int64_t)t * K + k]);
            }
            out[(int64_t)t * M + m] = orc_f32_to_f16(acc);
        }
}
