// decoder.hip -- the Llama/Qwen3 decoder loop that drives the quantized
// matmuls: batched prefill of a prompt and greedy decode steps, with an
// INT8 (or FP16) KV cache, all on one HIP stream.
//
// Layer order and arithmetic follow the reference engine:
//   decode step  Engine::decode_step / transformer_layer /
//                transformer_layer_attn_compute / _attn_block / _ffn_block
//                (src/engine/decode.cu:2101-2158, :1168-1246, :1437-1520)
//   prefill      Engine::generate Path B + transformer_prefill
//                (src/engine/decode.cu:2779-2807, :1760-1884) and the
//                first-token sampling from the last prefill row (:2950-2990)
//   sampling     greedy (src/engine/sample.cpp:160-170), on the GPU here
// with MI355X-specific fusions that keep the arithmetic (the fp16 roundings
// of the unfused sequence are kept; only the order of the RMSNorm sums of
// squares differs): in a decode step the attention / FFN / output RMSNorms
// run inside the staging of the GEMV that consumes them, the q/k RMSNorm + RoPE + KV quantisation of each layer is
// one launch, and the greedy argmax runs on the device so the sampled token
// id never leaves HBM -- the next step's embedding gather reads it there, and
// a whole generation needs no host synchronisation until the caller copies
// the tokens out.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <new>
#include "capi_common.h"
#include "layer_ops.h"

using jllm_hip::launch_status;
using jllm_hip::GemmOut;
using jllm_hip::gemm_batched_shared_x;
using jllm_hip::gemm_batched_res;
using jllm_hip::norm_rows;
using jllm_hip::residual_finish;
using jllm_hip::ResidualRows;
using jllm_hip::qkv_front_prefill;
using jllm_hip::QKPostArgs;
using jllm_hip::AttnQuant;

struct jllm_hip_decoder {
    jllm_hip_decoder_config cfg;
    jllm_hip_model_weights mw;
    jllm_hip_layer_weights* lw = nullptr;
    // KV cache, per layer [max_seq][n_kv * head_dim] (int8 or fp16) and
    // per-(position, kv head) fp32 scales
    uint8_t* kc = nullptr;
    uint8_t* vc = nullptr;
    float* ks = nullptr;
    float* vs = nullptr;
    size_t layer_kv_bytes = 0, layer_sc_floats = 0;
    // activations, sized for max_batch rows (prefill) and one row (decode)
    uint16_t *x, *x2, *normed, *q, *k, *v, *attn, *proj, *gate, *up, *act;
    float* logits;
    int32_t* tok;            // device token scratch [max_batch]
    void* arena = nullptr;   // one allocation for everything above
    int max_batch = 0;
};

namespace {

bool valid_type(int t) { return t >= 12 && t <= 14; }   // Q4_K, Q5_K, Q6_K

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

#define TRY(call)                                        \
    do {                                                 \
        int _st = (call);                                \
        if (_st != JLLM_OK) return _st;                  \
    } while (0)

float attn_scale(const jllm_hip_decoder_config& c) { return 1.0f / sqrtf((float)c.head_dim); }

uint8_t* layer_k(jllm_hip_decoder* d, int l) { return d->kc + (size_t)l * d->layer_kv_bytes; }
uint8_t* layer_v(jllm_hip_decoder* d, int l) { return d->vc + (size_t)l * d->layer_kv_bytes; }
float* layer_ks(jllm_hip_decoder* d, int l) { return d->ks + (size_t)l * d->layer_sc_floats; }
float* layer_vs(jllm_hip_decoder* d, int l) { return d->vs + (size_t)l * d->layer_sc_floats; }

// One decoder layer for one token at position pos; x is updated in place
// (transformer_layer, decode.cu:1168-1246).
int decode_layer(jllm_hip_decoder* d, int l, int pos, void* st) {
    const jllm_hip_decoder_config& c = d->cfg;
    const jllm_hip_layer_weights& w = d->lw[l];
    const int H = c.hidden_dim, QD = c.n_heads * c.head_dim, KVD = c.n_kv_heads * c.head_dim, I = c.intermediate_dim;
    const size_t row = (size_t)KVD * (c.kv_int8 ? 1 : 2);
    // attention RMSNorm fused into the QKV GEMV's activation staging
    TRY(jllm_hip_gemv_quant_triple_rmsnorm(d->q, w.wq, w.type_wq, QD, d->k, w.wk, w.type_wk, KVD, d->v, w.wv,
                                           w.type_wv, KVD, d->x, w.rms_attn, c.norm_fp32, c.rms_eps, H, st));
    TRY(jllm_hip_qk_norm_rope_store_kv(d->q, d->k, d->v, w.q_norm, w.k_norm, c.qk_norm_fp32, c.rms_eps,
                                       layer_k(d, l) + (size_t)pos * row, layer_v(d, l) + (size_t)pos * row,
                                       layer_ks(d, l) + (size_t)pos * c.n_kv_heads,
                                       layer_vs(d, l) + (size_t)pos * c.n_kv_heads, KVD, c.n_heads, c.n_kv_heads,
                                       c.head_dim, c.head_dim, pos, 1, c.rope_theta, c.rope_neox, c.kv_int8, st));
    TRY(jllm_hip_flash_attention_decode(d->attn, d->q, layer_k(d, l), layer_v(d, l), c.n_heads, c.n_kv_heads,
                                        c.head_dim, c.head_dim, pos + 1, attn_scale(c), c.kv_int8,
                                        c.kv_int8 ? layer_ks(d, l) : nullptr, c.kv_int8 ? layer_vs(d, l) : nullptr, 0,
                                        st));
    TRY(jllm_hip_gemv_quant_add(d->x2, w.wo, w.type_wo, d->attn, d->x, H, QD, st));
    // FFN RMSNorm fused into the gate/up GEMV's staging, SwiGLU into its epilogue
    // (when gate and up share a Q4_K / Q5_K type; otherwise pair + SwiGLU)
    if (w.type_w_gate == w.type_w_up && (w.type_w_gate == 12 || w.type_w_gate == 13)) {
        TRY(jllm_hip_gemv_quant_pair_rmsnorm_swiglu(d->act, w.w_gate, w.type_w_gate, w.w_up, w.type_w_up, I, d->x2,
                                                    w.rms_ffn, c.norm_fp32, c.rms_eps, H, st));
    } else {
        TRY(jllm_hip_gemv_quant_pair_rmsnorm(d->gate, w.w_gate, w.type_w_gate, I, d->up, w.w_up, w.type_w_up, I,
                                             d->x2, w.rms_ffn, c.norm_fp32, c.rms_eps, H, st));
        TRY(jllm_hip_fused_swiglu(d->act, d->gate, d->up, 1, I, st));
    }
    TRY(jllm_hip_gemv_quant_add(d->x, w.w_down, w.type_w_down, d->act, d->x2, H, I, st));
    return JLLM_OK;
}

// One layer over N prompt tokens at positions start..start+N-1; xb [N][H]
// updated in place (transformer_prefill, decode.cu:1760-1884).
// One decoder layer over N tokens at positions start.. (the prefill).  The
// residual adds after the O and down projections are left to the RMSNorm
// that follows them (norm_rows: split-K sum, residual add, RMSNorm and the
// activation codes in one pass).  *normed_q: on entry, whether normed and
// the quantiser scratch already hold the attention RMSNorm of x and its codes
// (the previous layer's last step); on exit, the same for layer l + 1 when
// next is set (its attention RMSNorm formed here), else x is complete.
int prefill_layer(jllm_hip_decoder* d, int l, int start, int N, void* st, bool* normed_q, bool next) {
    const jllm_hip_decoder_config& c = d->cfg;
    const jllm_hip_layer_weights& w = d->lw[l];
    const int H = c.hidden_dim, QD = c.n_heads * c.head_dim, KVD = c.n_kv_heads * c.head_dim, I = c.intermediate_dim;
    const size_t row = (size_t)KVD * (c.kv_int8 ? 1 : 2);
    const GemmOut qkv[3] = {{d->q, w.wq, w.type_wq, QD}, {d->k, w.wk, w.type_wk, KVD}, {d->v, w.wv, w.type_wv, KVD}};
    if (!*normed_q)
        TRY(norm_rows("decoder", ResidualRows{d->x, nullptr, nullptr, 0, 0}, N, H, d->normed, w.rms_attn,
                      c.norm_fp32 != 0, c.rms_eps, qkv, 3, normed_q, st));
    // Q, K, V of one quantised activation, then the attention front (q/k
    // norm, RoPE, KV store) -- in the GEMM's epilogue where the shapes allow
    QKPostArgs fa;
    fa.q = d->q; fa.k = d->k; fa.v = d->v; fa.q_norm = w.q_norm; fa.k_norm = w.k_norm;
    fa.k_dst = layer_k(d, l) + (size_t)start * row; fa.v_dst = layer_v(d, l) + (size_t)start * row;
    fa.k_scales = c.kv_int8 ? layer_ks(d, l) + (size_t)start * c.n_kv_heads : nullptr;
    fa.v_scales = c.kv_int8 ? layer_vs(d, l) + (size_t)start * c.n_kv_heads : nullptr;
    fa.kv_stride = KVD; fa.n_heads = c.n_heads; fa.n_kv = c.n_kv_heads; fa.head_dim = c.head_dim;
    fa.cache_head_dim = c.head_dim; fa.start_pos = start; fa.N = N; fa.eps = c.rms_eps;
    fa.norm_fp32 = c.qk_norm_fp32 != 0; fa.neox = c.rope_neox != 0; fa.kv_int8 = c.kv_int8 != 0;
    jllm_hip::rope_frequencies(fa.fr, c.head_dim, c.rope_theta);
    bool fused = false;
    TRY(qkv_front_prefill("decoder", qkv, d->normed, N, H, *normed_q, fa, st, &fused));
    if (!fused) {
        TRY(gemm_batched_shared_x("decoder", qkv, 3, d->normed, N, H, st, *normed_q));
        TRY(jllm_hip_qk_norm_rope_store_kv(d->q, d->k, d->v, w.q_norm, w.k_norm, c.qk_norm_fp32, c.rms_eps,
                                           fa.k_dst, fa.v_dst, layer_ks(d, l) + (size_t)start * c.n_kv_heads,
                                           layer_vs(d, l) + (size_t)start * c.n_kv_heads, KVD, c.n_heads,
                                           c.n_kv_heads, c.head_dim, c.head_dim, start, N, c.rope_theta,
                                           c.rope_neox, c.kv_int8, st));
    }
    // the attention output quantised for the O GEMM in the attention's
    // epilogue where the kernel form allows
    AttnQuant aq;
    const bool want_q = N > 1 && (w.type_wo == 12 || w.type_wo == 14);
    if (want_q) TRY(jllm_hip::q8_codes("decoder", w.type_wo, N, QD, &aq));
    bool oq = false;
    TRY(jllm_hip::prefill_attention(d->attn, d->q, layer_k(d, l), layer_v(d, l), c.n_heads, c.n_kv_heads, c.head_dim,
                                    c.head_dim, N, start, attn_scale(c), c.kv_int8,
                                    c.kv_int8 ? layer_ks(d, l) : nullptr, c.kv_int8 ? layer_vs(d, l) : nullptr, 0,
                                    want_q ? &aq : nullptr, st, &oq));
    ResidualRows r;
    TRY(gemm_batched_res("decoder", d->x2, w.wo, w.type_wo, d->attn, nullptr, nullptr, d->x, H, N, QD, st, &r,
                         oq ? &aq : nullptr));
    const GemmOut gu[2] = {{d->gate, w.w_gate, w.type_w_gate, I}, {d->up, w.w_up, w.type_w_up, I}};
    bool q2 = false;
    TRY(norm_rows("decoder", r, N, H, d->normed, w.rms_ffn, c.norm_fp32 != 0, c.rms_eps, gu, 2, &q2, st));
    // gate/up with the SwiGLU quantised for the down GEMM in the epilogue
    // where the shapes allow
    AttnQuant act;
    bool swq = false;
    TRY(jllm_hip::gate_up_swiglu_prefill("decoder", gu, d->normed, N, H, q2, w.type_w_down, &act, &swq, st));
    if (!swq) TRY(gemm_batched_shared_x("decoder", gu, 2, d->normed, N, H, st, q2));
    TRY(gemm_batched_res("decoder", d->x, w.w_down, w.type_w_down, d->gate, d->up, d->act, d->x2, H, N, I, st, &r,
                         swq ? &act : nullptr));
    *normed_q = false;
    if (!next) return residual_finish("decoder", r, N, H, st);
    const jllm_hip_layer_weights& wn = d->lw[l + 1];
    const GemmOut qkvn[3] = {{d->q, wn.wq, wn.type_wq, QD}, {d->k, wn.wk, wn.type_wk, KVD}, {d->v, wn.wv, wn.type_wv, KVD}};
    return norm_rows("decoder", r, N, H, d->normed, wn.rms_attn, c.norm_fp32 != 0, c.rms_eps, qkvn, 3, normed_q, st);
}

// output norm -> lm_head (fp32 logits) -> greedy token into *out
// (decode.cu:2147-2158 and :2956-2966; sample_greedy on the device); the
// norm is fused into the lm_head GEMV's activation staging
int head(jllm_hip_decoder* d, const uint16_t* xrow, int32_t* out, void* st) {
    const jllm_hip_decoder_config& c = d->cfg;
    TRY(jllm_hip_gemv_quant_f32_rmsnorm(d->logits, d->mw.output, d->mw.output_type, xrow, d->mw.output_norm,
                                        c.output_norm_fp32, c.rms_eps, c.vocab_size, c.hidden_dim, st));
    if (out) TRY(jllm_hip_argmax_f32(out, d->logits, c.vocab_size, st));
    return JLLM_OK;
}

}  // namespace

namespace jllm_hip {
bool decoder_config_ok(const jllm_hip_decoder_config& c) {
    const char* why = nullptr;
    if (c.n_layers <= 0 || c.hidden_dim <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 ||
        c.intermediate_dim <= 0 || c.vocab_size <= 0 || c.max_seq <= 0)
        why = "every dimension must be positive";
    else if (c.hidden_dim % 256 || (c.n_heads * c.head_dim) % 256 || c.intermediate_dim % 256)
        why = "hidden_dim, n_heads * head_dim and intermediate_dim must be multiples of 256 (K-quant rows)";
    else if (c.hidden_dim > 4096)
        why = "hidden_dim must be <= 4096 (the decode GEMVs normalise the whole activation in each workgroup)";
    else if (c.intermediate_dim > 28672 || c.n_heads * c.head_dim > 28672)
        why = "intermediate_dim and n_heads * head_dim must be <= 28672 (GEMV activation staging)";
    else if (c.head_dim % 32 || c.head_dim > 128)
        why = "head_dim must be a multiple of 32 and <= 128 (attention tiles)";
    else if (c.n_heads % c.n_kv_heads || c.n_heads / c.n_kv_heads > 16)
        why = "n_heads must be a multiple of n_kv_heads with at most 16 query heads per KV head";
    if (why) {
        fprintf(stderr, "[decoder] unsupported configuration (layers %d, hidden %d, heads %d/%d, head_dim %d, "
                        "ffn %d, vocab %d, max_seq %d): %s\n", c.n_layers, c.hidden_dim, c.n_heads, c.n_kv_heads,
                c.head_dim, c.intermediate_dim, c.vocab_size, c.max_seq, why);
        return false;
    }
    return true;
}
}  // namespace jllm_hip

extern "C" {


jllm_hip_decoder* jllm_hip_decoder_create(const jllm_hip_decoder_config* cfg, const jllm_hip_model_weights* mw,
                                          const jllm_hip_layer_weights* layers, int max_batch) {
    if (!cfg || !mw || !layers) return nullptr;
    const jllm_hip_decoder_config& c = *cfg;
    if (!jllm_hip::decoder_config_ok(c) || max_batch <= 0) {
        if (max_batch <= 0) fprintf(stderr, "[decoder] max_batch=%d must be positive\n", max_batch);
        return nullptr;
    }
    if (!valid_type(mw->embd_type) || !valid_type(mw->output_type) || !mw->tok_embd || !mw->output ||
        !mw->output_norm) {
        fprintf(stderr, "[decoder] embedding / output weights missing or not Q4_K/Q5_K/Q6_K\n");
        return nullptr;
    }
    for (int l = 0; l < c.n_layers; l++) {
        const jllm_hip_layer_weights& w = layers[l];
        if (!valid_type(w.type_wq) || !valid_type(w.type_wk) || !valid_type(w.type_wv) || !valid_type(w.type_wo) ||
            !valid_type(w.type_w_gate) || !valid_type(w.type_w_up) || !valid_type(w.type_w_down) || !w.rms_attn ||
            !w.rms_ffn) {
            fprintf(stderr, "[decoder] layer %d: weights missing or not Q4_K/Q5_K/Q6_K\n", l);
            return nullptr;
        }
    }
    jllm_hip_decoder* d = new (std::nothrow) jllm_hip_decoder();
    if (!d) return nullptr;
    d->cfg = c;
    d->mw = *mw;
    d->lw = new (std::nothrow) jllm_hip_layer_weights[c.n_layers];
    if (!d->lw) { delete d; return nullptr; }
    memcpy(d->lw, layers, sizeof(jllm_hip_layer_weights) * (size_t)c.n_layers);
    d->max_batch = max_batch < c.max_seq ? max_batch : c.max_seq;

    const size_t KVD = (size_t)c.n_kv_heads * c.head_dim, QD = (size_t)c.n_heads * c.head_dim;
    const size_t B = (size_t)d->max_batch, H = c.hidden_dim, I = c.intermediate_dim;
    d->layer_kv_bytes = align256((size_t)c.max_seq * KVD * (c.kv_int8 ? 1 : 2));
    d->layer_sc_floats = align256((size_t)c.max_seq * c.n_kv_heads * 4) / 4;
    size_t sizes[] = {
        d->layer_kv_bytes * c.n_layers, d->layer_kv_bytes * c.n_layers,              // kc, vc
        d->layer_sc_floats * 4 * c.n_layers, d->layer_sc_floats * 4 * c.n_layers,    // ks, vs
        B * H * 2, B * H * 2, B * H * 2,                                             // x, x2, normed
        B * QD * 2, B * KVD * 2, B * KVD * 2, B * QD * 2, B * H * 2,                 // q, k, v, attn, proj
        B * I * 2, B * I * 2, B * I * 2,                                             // gate, up, act
        (size_t)c.vocab_size * 4, B * 4};                                            // logits, tok
    const int NB = sizeof(sizes) / sizeof(sizes[0]);
    size_t total = 0;
    for (int i = 0; i < NB; i++) total += align256(sizes[i]);
    if (hipMalloc(&d->arena, total) != hipSuccess) {
        fprintf(stderr, "[decoder] hipMalloc of %zu bytes failed\n", total);
        delete[] d->lw;
        delete d;
        return nullptr;
    }
    // zero once (no stream capture is active at creation)
    (void)hipMemset(d->arena, 0, total);
    uint8_t* p = (uint8_t*)d->arena;
    void* slot[17];
    for (int i = 0; i < NB; i++) { slot[i] = p; p += align256(sizes[i]); }
    d->kc = (uint8_t*)slot[0]; d->vc = (uint8_t*)slot[1]; d->ks = (float*)slot[2]; d->vs = (float*)slot[3];
    d->x = (uint16_t*)slot[4]; d->x2 = (uint16_t*)slot[5]; d->normed = (uint16_t*)slot[6];
    d->q = (uint16_t*)slot[7]; d->k = (uint16_t*)slot[8]; d->v = (uint16_t*)slot[9];
    d->attn = (uint16_t*)slot[10]; d->proj = (uint16_t*)slot[11];
    d->gate = (uint16_t*)slot[12]; d->up = (uint16_t*)slot[13]; d->act = (uint16_t*)slot[14];
    d->logits = (float*)slot[15]; d->tok = (int32_t*)slot[16];
    return d;
}

void jllm_hip_decoder_destroy(jllm_hip_decoder* d) {
    if (!d) return;
    if (d->arena) (void)hipFree(d->arena);
    delete[] d->lw;
    delete d;
}

int jllm_hip_decoder_prefill(jllm_hip_decoder* d, const int32_t* tokens, int N, int start_pos, int32_t* next_token,
                             void* stream) {
    if (!d || !tokens || N <= 0 || start_pos < 0 || start_pos + N > d->cfg.max_seq) return JLLM_ERR_INVALID;
    const jllm_hip_decoder_config& c = d->cfg;
    // chunks of at most max_batch tokens; each chunk attends to all earlier KV
    for (int c0 = 0; c0 < N; c0 += d->max_batch) {
        const int n = N - c0 < d->max_batch ? N - c0 : d->max_batch;
        TRY(jllm_hip_dequant_embedding_rows(d->x, d->mw.tok_embd, d->mw.embd_type, tokens + c0, n, c.hidden_dim,
                                            c.vocab_size, stream));
        bool normed_q = false;
        for (int l = 0; l < c.n_layers; l++)
            TRY(prefill_layer(d, l, start_pos + c0, n, stream, &normed_q, l + 1 < c.n_layers));
        if (c0 + n == N) TRY(head(d, d->x + (size_t)(n - 1) * c.hidden_dim, next_token, stream));
    }
    return JLLM_OK;
}

int jllm_hip_decoder_step(jllm_hip_decoder* d, const int32_t* token, int pos, int32_t* next_token, void* stream) {
    if (!d || !token || pos < 0 || pos >= d->cfg.max_seq) return JLLM_ERR_INVALID;
    const jllm_hip_decoder_config& c = d->cfg;
    TRY(jllm_hip_dequant_embedding_rows(d->x, d->mw.tok_embd, d->mw.embd_type, token, 1, c.hidden_dim, c.vocab_size,
                                        stream));
    for (int l = 0; l < c.n_layers; l++) TRY(decode_layer(d, l, pos, stream));
    return head(d, d->x, next_token, stream);
}

int jllm_hip_decoder_generate(jllm_hip_decoder* d, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out,
                              void* stream) {
    if (!d || !prompt || !out || n_prompt <= 0 || n_gen <= 0 || n_prompt + n_gen - 1 > d->cfg.max_seq)
        return JLLM_ERR_INVALID;
    TRY(jllm_hip_decoder_prefill(d, prompt, n_prompt, 0, out, stream));
    for (int i = 1; i < n_gen; i++) TRY(jllm_hip_decoder_step(d, out + i - 1, n_prompt + i - 1, out + i, stream));
    return JLLM_OK;
}

int jllm_hip_decoder_layer(jllm_hip_decoder* d, int layer, uint16_t* x, int N, int start_pos, void* stream) {
    if (!d || !x || layer < 0 || layer >= d->cfg.n_layers || N <= 0 || N > d->max_batch || start_pos < 0 ||
        start_pos + N > d->cfg.max_seq)
        return JLLM_ERR_INVALID;
    const size_t bytes = (size_t)N * d->cfg.hidden_dim * 2;
    hipStream_t st = (hipStream_t)stream;
    TRY(launch_status(hipMemcpyAsync(d->x, x, bytes, hipMemcpyDeviceToDevice, st), "decoder"));
    bool normed_q = false;
    TRY(N == 1 ? decode_layer(d, layer, start_pos, stream)
               : prefill_layer(d, layer, start_pos, N, stream, &normed_q, false));
    return launch_status(hipMemcpyAsync(x, d->x, bytes, hipMemcpyDeviceToDevice, st), "decoder");
}

int jllm_hip_decoder_copy_kv(jllm_hip_decoder* d, int layer, int n_pos, void* k, void* v, float* k_scales,
                             float* v_scales, void* stream) {
    if (!d || layer < 0 || layer >= d->cfg.n_layers || n_pos < 0 || n_pos > d->cfg.max_seq) return JLLM_ERR_INVALID;
    const jllm_hip_decoder_config& c = d->cfg;
    const size_t rows = (size_t)n_pos * c.n_kv_heads * c.head_dim * (c.kv_int8 ? 1 : 2);
    const size_t sc = (size_t)n_pos * c.n_kv_heads * 4;
    hipStream_t st = (hipStream_t)stream;
    if (k) TRY(launch_status(hipMemcpyAsync(k, layer_k(d, layer), rows, hipMemcpyDeviceToDevice, st), "decoder"));
    if (v) TRY(launch_status(hipMemcpyAsync(v, layer_v(d, layer), rows, hipMemcpyDeviceToDevice, st), "decoder"));
    if (c.kv_int8 && k_scales)
        TRY(launch_status(hipMemcpyAsync(k_scales, layer_ks(d, layer), sc, hipMemcpyDeviceToDevice, st), "decoder"));
    if (c.kv_int8 && v_scales)
        TRY(launch_status(hipMemcpyAsync(v_scales, layer_vs(d, layer), sc, hipMemcpyDeviceToDevice, st), "decoder"));
    return JLLM_OK;
}

int jllm_hip_decoder_copy_act(jllm_hip_decoder* d, int which, int rows, uint16_t* dst, void* stream) {
    if (!d || !dst || rows <= 0 || rows > d->max_batch) return JLLM_ERR_INVALID;
    const jllm_hip_decoder_config& c = d->cfg;
    const size_t QD = (size_t)c.n_heads * c.head_dim;
    const uint16_t* src = which == 0 ? d->q : which == 1 ? d->attn : which == 2 ? d->x2 : nullptr;
    if (!src) return JLLM_ERR_INVALID;
    const size_t bytes = (size_t)rows * (which == 2 ? (size_t)c.hidden_dim : QD) * 2;
    return launch_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "decoder");
}

int jllm_hip_decoder_copy_logits(const jllm_hip_decoder* d, float* dst, void* stream) {
    if (!d || !dst) return JLLM_ERR_INVALID;
    return launch_status(hipMemcpyAsync(dst, d->logits, (size_t)d->cfg.vocab_size * 4, hipMemcpyDeviceToDevice,
                                        (hipStream_t)stream), "decoder");
}

}  // extern "C"
