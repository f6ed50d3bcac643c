/*
 * jllm_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul hot path.
 *
 * Plain C: pointers, sizes and an int status.  fp16 buffers are passed as
 * uint16_t* holding IEEE binary16 bit patterns; `stream` is a hipStream_t
 * (NULL = the default stream).  Every entry point is asynchronous on the
 * given stream and returns JLLM_OK once its kernels are enqueued.
 *
 * Each declaration names the genie-ai-runtime interface it replaces
 * (include/jllm_kernels.h unless stated otherwise).  Unlike the reference,
 * nothing here falls back to a host computation: an unsupported type or a
 * pointer the GPU cannot read is reported as an error (and logged to stderr)
 * instead of being computed on the CPU.
 *
 * Requirements shared by the GEMV/GEMM entry points: ggml_type is 12 (Q4_K)
 * or 14 (Q6_K); K is a positive multiple of 256; W and x are 16-byte
 * aligned device (or registered mapped) pointers; K <= 28672.
 */
#ifndef JLLM_HIP_H
#define JLLM_HIP_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    JLLM_OK = 0,
    JLLM_ERR_INVALID = -1,      /* bad size, null or misaligned pointer */
    JLLM_ERR_UNSUPPORTED = -2,  /* ggml type not supported by the call  */
    JLLM_ERR_LAUNCH = -3,       /* the HIP runtime rejected a launch    */
    JLLM_ERR_NOMEM = -4,        /* scratch allocation failed            */
    JLLM_ERR_POINTER = -5       /* weight pointer not visible to the GPU */
};

const char* jllm_hip_status_string(int status);

/* Mapped-weight registry.  Replaces register_mapped_weight_region,
 * clear_mapped_weight_region, resolve_mapped_weight_device_ptr
 * (jllm_kernels.h:40-43, defined in src/engine/model.cpp:39-66) for callers
 * without the engine.  Resolution (here and for every weight argument)
 * looks in this registry first, then in the engine's own registry when the
 * engine's jllm::resolve_mapped_weight_device_ptr is linked into the process
 * (a weak reference: the library does not define the jllm:: registry). */
int         jllm_hip_register_mapped_weight_region(const void* host_base, const void* device_base, int64_t bytes);
void        jllm_hip_clear_mapped_weight_region(const void* host_base);
const void* jllm_hip_resolve_mapped_weight_device_ptr(const void* host_ptr);

/* y[M] (fp16) = W[M x K] . x[K]; ggml_type 12 (Q4_K), 13 (Q5_K) or 14
 * (Q6_K).  Q4_K and Q6_K use the int8 MMVQ path (activation quantised to
 * q8_1), Q5_K the float-dequant path.  Replaces gemv_quant, jllm_kernels.h:64
 * (dispatch gemv_q4.cu:1245-1306). */
int jllm_hip_gemv_quant(uint16_t* y, const void* W, int ggml_type, const uint16_t* x,
                        int M, int K, void* stream);

/* y = half(half(W . x) + residual); float-dequant arithmetic.
 * Replaces gemv_quant_add, jllm_kernels.h:78 (gemv_q4.cu:1562-1616). */
int jllm_hip_gemv_quant_add(uint16_t* y, const void* W, int ggml_type, const uint16_t* x,
                            const uint16_t* residual, int M, int K, void* stream);

/* Two / three outputs sharing one activation.  MMVQ when both are Q4_K
 * (pair) or the types are (Q4_K, Q4_K, Q4_K|Q6_K), (Q6_K, Q6_K, Q6_K) or
 * (Q6_K, Q4_K, Q4_K) (triple, the reference's instantiations); float
 * dequant otherwise (any Q5_K).  Replaces gemv_quant_pair :92 and
 * gemv_quant_triple :106 (gemv_q4.cu:1375-1560). */
int jllm_hip_gemv_quant_pair(uint16_t* y0, const void* W0, int ggml_type0, int M0,
                             uint16_t* y1, const void* W1, int ggml_type1, int M1,
                             const uint16_t* x, int K, void* stream);
int jllm_hip_gemv_quant_triple(uint16_t* y0, const void* W0, int ggml_type0, int M0,
                               uint16_t* y1, const void* W1, int ggml_type1, int M1,
                               uint16_t* y2, const void* W2, int ggml_type2, int M2,
                               const uint16_t* x, int K, void* stream);

/* fp32 output.  Q4_K: MMVQ; Q5_K / Q6_K: float dequant.  Replaces gemv_quant_f32,
 * jllm_kernels.h:148 (gemv_q4.cu:1323-1369). */
int jllm_hip_gemv_quant_f32(float* y, const void* W, int ggml_type, const uint16_t* x,
                            int M, int K, void* stream);

/* fp32 output, float-dequant arithmetic for both types: the GPU form of the
 * host scalar path gemv_quant_cpu (gemv_q4.cu:2519-2631).  No reference
 * counterpart on the GPU; for callers that want the dequant arithmetic. */
int jllm_hip_gemv_quant_dequant_f32(float* y, const void* W, int ggml_type, const uint16_t* x,
                                    int M, int K, void* stream);

/* RMSNorm fused into the GEMV's activation staging (no reference
 * counterpart: each replaces two launches of the engine's decode step).
 * x <- half(x / sqrt(mean(x^2) + eps) * norm_weight) -- the values of
 * jllm_hip_fused_rmsnorm_residual without residual, up to the order of the
 * sum of squares -- then the GEMV runs as its unfused entry point:
 *   _triple_rmsnorm / _pair_rmsnorm: gemv_quant_triple / _pair
 *     (decode.cu:1208-1224 and :1234-1238);
 *   _f32_rmsnorm: the output norm + lm_head (decode.cu:2147-2158).
 * norm_weight: fp32 (weight_fp32 != 0) or fp16, 16-byte aligned; K <= 4096
 * (hidden sizes; every workgroup sums the squares of the whole vector). */
int jllm_hip_gemv_quant_triple_rmsnorm(uint16_t* y0, const void* W0, int ggml_type0, int M0,
                                       uint16_t* y1, const void* W1, int ggml_type1, int M1,
                                       uint16_t* y2, const void* W2, int ggml_type2, int M2,
                                       const uint16_t* x, const void* norm_weight, int weight_fp32, float eps,
                                       int K, void* stream);
int jllm_hip_gemv_quant_pair_rmsnorm(uint16_t* y0, const void* W0, int ggml_type0, int M0,
                                     uint16_t* y1, const void* W1, int ggml_type1, int M1,
                                     const uint16_t* x, const void* norm_weight, int weight_fp32, float eps,
                                     int K, void* stream);
int jllm_hip_gemv_quant_f32_rmsnorm(float* y, const void* W, int ggml_type, const uint16_t* x,
                                    const void* norm_weight, int weight_fp32, float eps, int M, int K, void* stream);

/* The decode FFN's gate/up pair with the SwiGLU fused into its epilogue (no
 * reference counterpart: replaces gemv_quant_pair + swiglu, decode.cu:1234-
 * 1242).  act[r] = half(silu(g) * u) with g = half(W_gate[r] . x), u =
 * half(W_up[r] . x): the values of jllm_hip_gemv_quant_pair followed by
 * jllm_hip_fused_swiglu.  W_gate and W_up: one type, Q4_K or Q5_K (else
 * JLLM_ERR_UNSUPPORTED), M rows each; the _rmsnorm form normalises x first
 * as jllm_hip_gemv_quant_pair_rmsnorm does. */
int jllm_hip_gemv_quant_pair_swiglu(uint16_t* act, const void* W_gate, int type_gate, const void* W_up, int type_up,
                                    int M, const uint16_t* x, int K, void* stream);
int jllm_hip_gemv_quant_pair_rmsnorm_swiglu(uint16_t* act, const void* W_gate, int type_gate, const void* W_up,
                                            int type_up, int M, const uint16_t* x, const void* norm_weight,
                                            int weight_fp32, float eps, int K, void* stream);

/* q8_1 quantiser in the reference block layout {u16 d, u16 s, i8 qs[32]}
 * (36 B per 32 values).  Replaces quantize_q8_1, gemv_q4.cu:468. */
int jllm_hip_quantize_q8_1(const uint16_t* x, void* y, int K, void* stream);

/* Batched GEMM y[N x M] (fp16, token-major) = x[N x K] . W^T.  N == 1 routes
 * to jllm_hip_gemv_quant; otherwise, for Q4_K / Q6_K, the activation is
 * quantised to q8_1 (the reference's DS4 values for Q4_K, D4 for Q6_K) and
 * multiplied on the matrix cores with every 32-weight sub-block (Q4_K) /
 * 16-weight group (Q6_K) dot formed exactly, then scaled as the reference
 * does; Q5_K multiplies the fp16 activation itself (the reference's float
 * Q5_K path, gemv_q4.cu:1703-1762) with exact products and fp32 sums.
 * When the tile grid does not cover the GPU, K is split over workgroups and
 * the fp32 partials are added in a fixed order (a function of M, ceil(N/64)
 * and K).  Uses library-owned scratch buffers (q8 codes, split-K partials;
 * grown on demand, never freed); calls on one device must be serialised
 * (one stream), as in the reference.
 * Replaces gemm_quant_batched, jllm_kernels.h:135 (gemv_q4.cu:2478-2517),
 * and the internal gemm_q4k_mmq_llama / gemm_q6k_mmq_llama
 * (mmq_q4k_llama.cu:479, mmq_q6k_llama.cu:497). */
int jllm_hip_gemm_quant_batched(uint16_t* y, const void* W, int ggml_type, const uint16_t* x,
                                int M, int N, int K, void* stream);

/* Same computation with fp32 output (no fp16 rounding of y).  No reference
 * counterpart (the reference writes fp16); for callers that keep fp32. */
int jllm_hip_gemm_quant_batched_f32(float* y, const void* W, int ggml_type, const uint16_t* x,
                                    int M, int N, int K, void* stream);

/* Several products of ONE activation: y[i] [N x M[i]] (fp16) = x . W[i]^T for
 * i < n (n <= 3, shared K), the activation quantised once per kind.  When
 * every W[i] is Q4_K and their row tiles together cover the GPU, all of them
 * run as one launch without split-K (each output computed exactly as its own
 * launch without split-K would); otherwise one product at a time as
 * jllm_hip_gemm_quant_batched.  No reference counterpart: the engine issues
 * Q/K/V and gate/up as separate gemm_quant_batched calls (decode.cu:1797-1880);
 * this is the decoder's prefill path. */
int jllm_hip_gemm_quant_batched_multi(uint16_t* const* y, const void* const* W, const int* ggml_type, const int* M,
                                      int n, const uint16_t* x, int N, int K, void* stream);

/* The MMQ activation quantiser on its own: x [N x K] fp16 -> q8 [K/128][Npad]
 * blocks of 144 B.  ds4 != 0: DS4 layout {half2 (d, sum x)[4], i8 qs[128]}
 * (quantize_mmq_q8_1_ds4, mmq_q4k_llama.cu:383); ds4 == 0: D4 layout
 * {float d[4], i8 qs[128]} (quantize_mmq_q8_1_d4, mmq_q6k_llama.cu:424).
 * Npad is a multiple of 64 and >= N; columns >= N are written as zeros. */
int jllm_hip_quantize_mmq_q8_1(const uint16_t* x, void* q8, int N, int K, int Npad, int ds4, void* stream);

/* The production MMQ kernels' activation quantiser (same codes and scales
 * as jllm_hip_quantize_mmq_q8_1, in the kernels' layout): codes fp16
 * [K/256][Npad][256] (integers -127..127), scale words [K/32][Npad] (ds4:
 * half d | half sum << 16; else float d).  K a multiple of 256, Npad a
 * multiple of 64, x and codes 16-byte aligned.  No reference counterpart;
 * exposed so the layout can be checked against the reference quantiser. */
int jllm_hip_quantize_mmq_f16(const uint16_t* x, uint16_t* codes, uint32_t* scales, int N, int K, int Npad, int ds4,
                              void* stream);

/* The same quantiser writing int8 codes [K/256][Npad][256] (the Q4_K MMQ
 * kernel's layout; same codes and scale words).  No reference counterpart;
 * exposed so the layout can be checked against the reference quantiser. */
int jllm_hip_quantize_mmq_i8(const uint16_t* x, int8_t* codes, uint32_t* scales, int N, int K, int Npad, int ds4,
                             void* stream);

/* Test hook: the exact sub-block dots the production MMQ kernels form,
 * out [N][M][K/G] int32 (G = 32 for Q4_K sub-blocks, 16 for Q6_K groups),
 * for activations x [N x K] quantised by the production quantiser.  No
 * reference counterpart (the reference keeps these in registers); exists so
 * the dots can be checked bit-exactly against the reference's int32 dots. */
int jllm_hip_mmq_subdots(int32_t* out, const void* W, int ggml_type, const uint16_t* x,
                         int M, int N, int K, void* stream);

/* Single-query (decode) attention over an INT8 (kv_int8 != 0) or FP16 KV
 * cache, split-K: the keys are cut into slices processed in parallel, each
 * with an online softmax, then combined.  Layouts: q and out fp16
 * [n_heads x head_dim]; k/v [seq][n_kv_heads * cache_head_dim] (int8 or
 * fp16); k_scales/v_scales fp32 [seq][n_kv_heads] (INT8 only; NULL = 1.0).
 * window > 0 attends to the last `window` keys only.  head_dim is a multiple
 * of 32 and <= 128; n_heads/n_kv_heads <= 16.  Uses the library's partials
 * buffer (see jllm_hip_get_splitk_partials).
 * Replaces flash_attention_decode, jllm_kernels.h:323 (attention.cu:1036-1075,
 * kernels :837-969). */
int jllm_hip_flash_attention_decode(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                    int n_heads, int n_kv_heads, int head_dim, int cache_head_dim, int seq_len,
                                    float scale, int kv_int8, const float* k_scales, const float* v_scales,
                                    int window, void* stream);

/* Same with an explicit split count (1..256) instead of the policy of
 * jllm_hip_decode_attn_splits.  Replaces the n_splits argument of
 * flash_attention_decode_dyn, jllm_kernels.h:380 (attention.cu:1007-1034). */
int jllm_hip_flash_attention_decode_splits(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                           int n_heads, int n_kv_heads, int head_dim, int cache_head_dim,
                                           int seq_len, float scale, int kv_int8, const float* k_scales,
                                           const float* v_scales, int window, int n_splits, void* stream);

/* Decode attention whose key count is read on the device: seq = *d_pos + 1
 * at kernel execution time, so one captured HIP graph serves every decode
 * position; n_splits (1..256) is fixed by the caller, as in the reference
 * (size the partials buffer with jllm_hip_get_splitk_partials(n_heads,
 * n_splits, head_dim) before capture).  Splits that receive no keys
 * contribute nothing.  INT8 caches take their K and V scales separately
 * (the reference's single kv_scales argument passed one buffer as both,
 * attention.cu:1021-1024; that path is unreachable there because graph mode
 * is off for INT8 KV).  Replaces flash_attention_decode_dyn,
 * jllm_kernels.h:380 (attention.cu:1007-1034). */
int jllm_hip_flash_attention_decode_dyn(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                        int n_heads, int n_kv_heads, int head_dim, int cache_head_dim,
                                        const int32_t* d_pos, float scale, int kv_int8, const float* k_scales,
                                        const float* v_scales, int window, int n_splits, void* stream);

/* Allocation-free decode attention.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The same kernels
 * and split policy as jllm_hip_flash_attention_decode, but the split-K
 * partials live in a fixed 4 MiB array per device (allocated with the
 * library's code object, held until the process ends) instead of the
 * grown-on-demand buffer; this call makes no hipMalloc / hipFree.
 * The partials written -- n_heads * P * (2 + head_dim) * 4 bytes, where P =
 * ceil(splits / W) and W (4 from 64 splits on, else 1) is the number of
 * key ranges one workgroup combines -- must fit in 4 MiB (32 heads of 128
 * at the 128-split maximum: 0.53 MiB; 256 heads: 4.26 MB, refused), else
 * JLLM_ERR_INVALID.  Every
 * call on a device shares that device's array: calls that overlap on one
 * GPU (several streams) race. */
int jllm_hip_flash_attention_decode_noalloc(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                            int n_heads, int n_kv_heads, int head_dim, int cache_head_dim,
                                            int seq_len, float scale, int kv_int8, const float* k_scales,
                                            const float* v_scales, int window, void* stream);

/* Split-count policy and partials buffer.  Replace decode_attn_splits and
 * get_splitk_partials, jllm_kernels.h:402-403 (attention.cu:975-1005).  The
 * MI355X policy is ceil(seq/32) splits capped at 128 (one wave per KV head
 * and split, so 8 KV heads put 1024 waves on 256 CUs), not the reference's
 * 1/4/8; JLLM_SPLITK=0 in the environment (read once) gives 1 split for
 * every length, as in the reference.  With one split the output is written directly (no reduce).  The buffer (floats: m[H*S] | l[H*S] |
 * acc[H*S*head_dim]) is allocated on first use and never freed; call
 * jllm_hip_get_splitk_partials before graph capture.  NULL on failure. */
int    jllm_hip_decode_attn_splits(int seq_len);
float* jllm_hip_get_splitk_partials(int n_heads, int n_splits, int head_dim);

/* Per-row fp16 -> int8 quantiser for the KV cache: scale_out[r] =
 * absmax/127, q = rn(v * 127/absmax) clamped to +-127.  Replaces
 * fp16_to_int8, jllm_kernels.h:413 (convert.cu:26-75). */
int jllm_hip_fp16_to_int8(int8_t* dst, float* scale_out, const uint16_t* src, int rows, int cols, void* stream);

/* Causal attention of N query tokens against the cache (prefill): token t
 * (absolute position start_pos + t) attends to keys [0, start_pos + t] (the
 * last `window` of them when window > 0).  q and out are [N][n_heads x
 * head_dim]; cache layout and limits as jllm_hip_flash_attention_decode.
 * One wave per (KV head, token), no partials buffer.
 * Replaces flash_attention_prefill_batched, jllm_kernels.h:354
 * (attention.cu:382-514, launcher :617-682). */
int jllm_hip_flash_attention_prefill_batched(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                             int n_heads, int n_kv_heads, int head_dim, int cache_head_dim, int N,
                                             int start_pos, float scale, int kv_int8, const float* k_scales,
                                             const float* v_scales, int window, void* stream);

/* ---- decoder-layer kernels around the matmuls ---- */

/* out[rows x hidden_dim] = half((x + residual) / sqrt(mean((x+residual)^2)
 * + eps) * weight).  residual may be NULL; out may equal x.  weight is fp32
 * (weight_fp32 != 0) or fp16.  hidden_dim even; x, out, residual 4-byte
 * aligned.  Replaces fused_rmsnorm_residual, jllm_kernels.h:174
 * (fused_norm.cu:33-115). */
int jllm_hip_fused_rmsnorm_residual(uint16_t* out, const uint16_t* x, const uint16_t* residual, const void* weight,
                                    int rows, int hidden_dim, float eps, int weight_fp32, void* stream);

/* out = half(silu(gate) * up), silu(g) = g / (1 + e^-g), over rows x
 * intermediate_dim.  Replaces fused_swiglu, jllm_kernels.h:191
 * (convert.cu:85-112). */
int jllm_hip_fused_swiglu(uint16_t* out, const uint16_t* gate, const uint16_t* up, int rows, int intermediate_dim,
                          void* stream);

/* out = half(a + b) over n elements (the prefill residual adds).  Replaces
 * the engine-internal vec_add, src/engine/decode.cu:60-78. */
int jllm_hip_vec_add(uint16_t* out, const uint16_t* a, const uint16_t* b, int64_t n, void* stream);

/* Rotary position embedding in place: pair i of each head is (i, i + hd/2)
 * when neox != 0, else (2i, 2i+1); angle = position * 1/theta^(2i/hd)
 * (fp32).  k may be NULL (rotate q only).  head_dim even, <= 128.
 * Replace rope_inplace :241 and rope_inplace_batched :274 (rope.cu:322-367,
 * :427-446, :476-497; strides are per-token row strides in halves).
 * rope_precompute_table / rope_clear_tables (:238-239, rope.cu:82-137) are
 * accepted for interface parity and keep nothing: cos/sin are evaluated per
 * element from host-computed frequencies, with the same fp32 angle. */
int  jllm_hip_rope_inplace(uint16_t* q, uint16_t* k, int n_heads, int n_kv_heads, int head_dim, int position,
                           float theta_base, int neox, void* stream);
int  jllm_hip_rope_inplace_batched(uint16_t* q, uint16_t* k, int n_heads, int n_kv_heads, int head_dim,
                                   int start_pos, int N, int q_stride, int k_stride, float theta_base, int neox,
                                   void* stream);
/* RoPE of one token whose position is read on the device (*d_pos at kernel
 * execution time); k may be NULL with n_kv_heads 0 (rotate q only).
 * Replaces rope_inplace_dyn, jllm_kernels.h:306 (rope.cu:719-735). */
int  jllm_hip_rope_inplace_dyn(uint16_t* q, uint16_t* k, int n_heads, int n_kv_heads, int head_dim,
                               const int32_t* d_pos, float theta_base, int neox, void* stream);
/* RoPE of q and k plus fp16 copies of the rotated k and of v into the cache
 * (no q/k norm, no int8).
 *   _dyn: one token at position *d_pos (device); k and v go to
 *     k/v_cache_layer_base + pos * n_kv_heads * cache_head_dim, head h at
 *     h * cache_head_dim.  Replaces rope_inplace_store_kv_fp16_dyn,
 *     jllm_kernels.h:287 (rope.cu:737-763, kernel :581-640).
 *   _batched: N tokens at positions start_pos + t; q/k/v rows at t * q_stride
 *     / t * kv_stride halves; the cache row of token t at t * kv_slot halves
 *     from k/v_cache_base, head h at h * head_dim.  Replaces
 *     rope_inplace_store_kv_fp16_batched, jllm_kernels.h:278 (rope.cu:551-574,
 *     kernel :498-529). */
int  jllm_hip_rope_inplace_store_kv_fp16_dyn(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_cache_layer_base,
                                             uint16_t* v_cache_layer_base, int n_heads, int n_kv_heads, int head_dim,
                                             int cache_head_dim, const int32_t* d_pos, float theta_base, int neox,
                                             void* stream);
int  jllm_hip_rope_inplace_store_kv_fp16_batched(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_cache_base,
                                                 uint16_t* v_cache_base, int kv_slot, int n_heads, int n_kv_heads,
                                                 int head_dim, int start_pos, int N, int q_stride, int kv_stride,
                                                 float theta_base, int neox, void* stream);
int  jllm_hip_rope_precompute_table(int max_seq, int head_dim, float theta_base);
void jllm_hip_rope_clear_tables(void);

/* The attention front of N tokens in one launch: q_norm/k_norm RMSNorm over
 * each head (both given, or both NULL to skip the norms, as the engine
 * applies them only when a layer has both; one without the other is
 * JLLM_ERR_INVALID), RoPE of q and k (both in place),
 * then k and v written to the cache rows of positions start_pos + t: int8
 * with a per-(position, kv head) scale absmax/127 (kv_int8 != 0) or fp16.
 * q [N][n_heads*hd], k and v [N][n_kv_heads*hd].  k_dst/v_dst address the
 * cache row of position start_pos: token t goes to t * kv_stride elements
 * further, head h at h * cache_head_dim; its scales to k_scales/v_scales
 * [t * n_kv_heads + h] (may be NULL).  The intermediate fp16 roundings of
 * the unfused sequence are kept.  Replaces the sequence
 * fused_rmsnorm_residual(q), fused_rmsnorm_residual(k), rope_inplace,
 * fp16_to_int8(k), fp16_to_int8(v) of the engine (src/engine/decode.cu
 * :1441-1478 decode, :1806-1842 prefill) and rope_inplace_store_kv_fp16,
 * jllm_kernels.h:255 (rope.cu:369-410). */
int jllm_hip_qk_norm_rope_store_kv(uint16_t* q, uint16_t* k, const uint16_t* v, const void* q_norm,
                                   const void* k_norm, int norm_fp32, float eps, void* k_dst, void* v_dst,
                                   float* k_scales, float* v_scales, int64_t kv_stride, int n_heads, int n_kv_heads,
                                   int head_dim, int cache_head_dim, int start_pos, int N, float theta_base, int neox,
                                   int kv_int8, void* stream);

/* dst[hidden_dim] (fp16, 16-byte aligned) = dequantised row token_id of a
 * Q4_K / Q6_K embedding table (other types: JLLM_ERR_UNSUPPORTED, as the
 * reference returns false).  Returns a status instead of the reference's
 * bool.  Replaces dequant_embedding_row, jllm_kernels.h:160
 * (gemv_q4.cu:793-864, :2803-2828). */
int jllm_hip_dequant_embedding_row(uint16_t* dst, const void* W, int ggml_type, int token_id, int hidden_dim,
                                   void* stream);

/* The same for N tokens whose ids are in DEVICE memory (tokens[N]); an id
 * outside [0, vocab) gives a zero row; Q5_K tables too (the values of the
 * engine's host Q5_K row dequant, decode.cu:230-266).  No single reference
 * counterpart: the engine loops dequant_embedding per prompt token
 * (decode.cu:2796-2801);
 * reading ids on the device lets a greedy decode loop run without a host
 * round trip. */
int jllm_hip_dequant_embedding_rows(uint16_t* dst, const void* W, int ggml_type, const int32_t* tokens, int N,
                                    int hidden_dim, int vocab, void* stream);

/* out[0] (device int32) = the lowest index of the largest finite logit (0
 * when none is finite).  The GPU form of the host greedy sampler
 * sample_greedy, src/engine/sample.cpp:160-170.  Two launches sharing a
 * small library-owned device array of per-chunk candidates: calls on one
 * device must be serialised (one stream). */
int jllm_hip_argmax_f32(int32_t* out, const float* logits, int n, void* stream);

/* ---- kernels outside the Llama/Qwen decode path (Gemma family, logits) ---- */

/* out = half(gelu_tanh(gate) * up) over rows x intermediate_dim,
 * gelu_tanh(g) = 0.5 g (1 + tanh(0.7978845608 (g + 0.044715 g^3))).
 * Replaces fused_geglu, jllm_kernels.h:203 (convert.cu:121-151). */
int jllm_hip_fused_geglu(uint16_t* out, const uint16_t* gate, const uint16_t* up, int rows, int intermediate_dim,
                         void* stream);
/* x *= s in place: element pairs (0,1), (2,3), ... are multiplied in fp16 by
 * half(s); a trailing odd element in fp32 by s, then rounded.  Replaces
 * vec_scale, jllm_kernels.h:207 (convert.cu:155-170). */
int jllm_hip_vec_scale(uint16_t* x, int64_t n, float s, void* stream);
/* x = cap * tanh(x / cap) in place on fp32 logits (cap > 0).  Replaces
 * logit_softcap, jllm_kernels.h:210 (convert.cu:173-181). */
int jllm_hip_logit_softcap(float* x, int64_t n, float cap, void* stream);
/* x = exp(x - max) / sum in place on fp32 logits (one workgroup).  Replaces
 * softmax_inplace, jllm_kernels.h:407 (softmax.cu:15-81). */
int jllm_hip_softmax_inplace(float* x, int n, void* stream);
/* Dense projections, W row-major [M][K] of F32 (wtype 0), F16 (1) or BF16
 * (30): out[t][m] = half(sum_k W[m][k] x[t][k]), fp32 accumulation; x fp16
 * [N][K].  Other types: JLLM_ERR_UNSUPPORTED.  Replace gemv_dense and
 * gemm_dense_batched, jllm_kernels.h:214-226 (gemv_q4.cu:2815-2885). */
int jllm_hip_gemv_dense(uint16_t* out, const void* W, int wtype, const uint16_t* x, int M, int K, void* stream);
int jllm_hip_gemm_dense_batched(uint16_t* out, const void* W, int wtype, const uint16_t* x, int M, int N, int K,
                                void* stream);

/* ---- decoder loop (the engine-side caller of the kernels above) ---- */

/* Model shape (ModelConfig, include/jllm_engine.h:59; Llama/Qwen3 family: RMSNorm,
 * GQA attention with optional per-head q/k RMSNorm, RoPE, SwiGLU FFN).
 * hidden_dim, n_heads*head_dim and intermediate_dim are multiples of 256. */
typedef struct {
    int   n_layers, hidden_dim, n_heads, n_kv_heads, head_dim, intermediate_dim, vocab_size;
    int   max_seq;            /* KV-cache positions                              */
    float rms_eps, rope_theta;
    int   rope_neox;          /* 1: pairs (i, i + hd/2) (Qwen3)                  */
    int   kv_int8;            /* 1: INT8 KV cache with per-(pos, head) scales   */
    int   norm_fp32;          /* rms_attn / rms_ffn weights fp32 (1) or fp16 (0) */
    int   qk_norm_fp32;       /* q_norm / k_norm weights fp32 (1) or fp16 (0)    */
    int   output_norm_fp32;   /* output_norm weight fp32 (1) or fp16 (0)         */
} jllm_hip_decoder_config;

/* Device pointers of one layer (LayerWeights, include/jllm_engine.h:165); matrix
 * types are 12 (Q4_K) or 14 (Q6_K); q_norm/k_norm may be NULL. */
typedef struct {
    const void *rms_attn, *rms_ffn, *q_norm, *k_norm;
    const void *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down;
    int type_wq, type_wk, type_wv, type_wo, type_w_gate, type_w_up, type_w_down;
} jllm_hip_layer_weights;

typedef struct {
    const void* tok_embd;  int embd_type;      /* [vocab][hidden] Q4_K/Q5_K/Q6_K (may alias output) */
    const void* output_norm;                   /* [hidden]                                      */
    const void* output;    int output_type;    /* lm_head [vocab][hidden]                       */
} jllm_hip_model_weights;

typedef struct jllm_hip_decoder jllm_hip_decoder;

/* Allocates the KV cache (n_layers x max_seq) and the activation buffers
 * for prefill chunks of up to max_batch tokens, in one device allocation
 * freed by jllm_hip_decoder_destroy.  The weights stay owned by the caller.
 * NULL on an invalid configuration or allocation failure. */
jllm_hip_decoder* jllm_hip_decoder_create(const jllm_hip_decoder_config* cfg, const jllm_hip_model_weights* mw,
                                          const jllm_hip_layer_weights* layers, int max_batch);
void jllm_hip_decoder_destroy(jllm_hip_decoder* d);

/* Prefill N prompt tokens (DEVICE int32 ids) at positions start_pos..,
 * layer-major in chunks of max_batch tokens, then the greedy next token into
 * *next_token (DEVICE).  Engine::generate Path B + transformer_prefill +
 * first-token sampling (src/engine/decode.cu:2779-2807, :1760-1884,
 * :2950-2990). */
int jllm_hip_decoder_prefill(jllm_hip_decoder* d, const int32_t* tokens, int N, int start_pos, int32_t* next_token,
                             void* stream);

/* One greedy decode step: embed *token (DEVICE) at position pos, all layers,
 * output norm, lm_head, argmax into *next_token (DEVICE).
 * Engine::decode_step (src/engine/decode.cu:2101-2236, greedy sampling). */
int jllm_hip_decoder_step(jllm_hip_decoder* d, const int32_t* token, int pos, int32_t* next_token, void* stream);

/* prefill(prompt) then n_gen - 1 decode steps; out[n_gen] (DEVICE) receives
 * the generated ids.  Asynchronous: no host synchronisation inside. */
int jllm_hip_decoder_generate(jllm_hip_decoder* d, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out,
                              void* stream);

/* Test hook (no reference counterpart): runs decoder layer `layer` alone
 * on the caller's hidden rows x[N][hidden_dim] (fp16, DEVICE), in place, at
 * positions start_pos..start_pos+N-1 -- the decode step's layer
 * (transformer_layer, decode.cu:1168-1246) for N == 1, the prefill layer
 * (transformer_prefill, decode.cu:1760-1884) for 1 < N <= max_batch --
 * writing that layer's KV-cache rows, so that a test can feed each layer an
 * input of its choice and compare the layer's output. */
int jllm_hip_decoder_layer(jllm_hip_decoder* d, int layer, uint16_t* x, int N, int start_pos, void* stream);

/* Test hook (no reference counterpart): enqueue copies of positions
 * 0..n_pos-1 of layer `layer`'s KV cache into caller buffers (DEVICE) --
 * K and V [n_pos][n_kv_heads * head_dim] (int8, or fp16) and, for an INT8
 * cache, the fp32 scales [n_pos][n_kv_heads].  Any destination may be NULL. */
int jllm_hip_decoder_copy_kv(jllm_hip_decoder* d, int layer, int n_pos, void* k, void* v, float* k_scales,
                             float* v_scales, void* stream);

/* Test hook (no reference counterpart): enqueue a copy of the first `rows`
 * rows of an intermediate of the last layer run (fp16, into dst, DEVICE):
 * which 0 = q after q-RMSNorm and RoPE [rows][n_heads * head_dim], 1 = the
 * attention output [rows][n_heads * head_dim], 2 = the hidden state after
 * the attention block's residual add [rows][hidden_dim]. */
int jllm_hip_decoder_copy_act(jllm_hip_decoder* d, int which, int rows, uint16_t* dst, void* stream);

/* Enqueue a copy of the fp32 logits [vocab] of the last prefill/step into
 * dst (device memory). */
int jllm_hip_decoder_copy_logits(const jllm_hip_decoder* d, float* dst, void* stream);

/* ---- GGUF models ---- */

/* Reader: maps a GGUF v2/v3 file read-only and parses its metadata and
 * tensor table (every field bounds-checked; NULL and a message on stderr
 * for a malformed file).  Replaces the reference loader's GGUF parsing,
 * src/engine/model.cpp:150-345 (config) and :445-657 (tensor infos, mmap).
 * Tensor data pointers are host pointers into the mapping, valid until
 * jllm_hip_gguf_close. */
typedef struct jllm_hip_gguf jllm_hip_gguf;
jllm_hip_gguf* jllm_hip_gguf_open(const char* path);
void           jllm_hip_gguf_close(jllm_hip_gguf* g);
int64_t        jllm_hip_gguf_n_tensors(const jllm_hip_gguf* g);
int64_t        jllm_hip_gguf_find_tensor(const jllm_hip_gguf* g, const char* name);
int            jllm_hip_gguf_tensor(const jllm_hip_gguf* g, int64_t i, const char** name, int* ggml_type,
                                    int* n_dims, int64_t* dims /* [4], dims[0] fastest */,
                                    const void** data, int64_t* bytes);
int            jllm_hip_gguf_get_u64(const jllm_hip_gguf* g, const char* key, uint64_t* out);
int            jllm_hip_gguf_get_f64(const jllm_hip_gguf* g, const char* key, double* out);
const char*    jllm_hip_gguf_get_str(const jllm_hip_gguf* g, const char* key);

/* The decoder shape from the metadata (`<arch>.block_count`,
 * `.embedding_length`, `.attention.head_count(_kv)`, `.attention.key_length`,
 * `.feed_forward_length`, `.rope.freq_base`,
 * `.attention.layer_norm_rms_epsilon`, vocab from token_embd.weight when
 * `.vocab_size` is absent, neox RoPE for the Qwen/Gemma/Phi families; norm
 * weight types from the blk.0 / output_norm tensors), as load_gguf_config
 * does (model.cpp:150-345).  max_seq = `.context_length`; kv_int8 = 1. */
int jllm_hip_gguf_config(const jllm_hip_gguf* g, jllm_hip_decoder_config* cfg);

/* Uploads the decoder's tensors (token_embd, output_norm, output -- tied to
 * token_embd when absent --, and per layer attn_q/k/v/output, ffn_gate/up/
 * down, attn_norm, ffn_norm, attn_q_norm/k_norm) into one device allocation
 * and fills the weight structs for jllm_hip_decoder_create, by the names of
 * load_and_map_weights (model.cpp:657-810). */
typedef struct jllm_hip_gguf_model jllm_hip_gguf_model;
jllm_hip_gguf_model*          jllm_hip_gguf_model_load(const jllm_hip_gguf* g, const jllm_hip_decoder_config* cfg);
const jllm_hip_model_weights* jllm_hip_gguf_model_weights(const jllm_hip_gguf_model* m);
const jllm_hip_layer_weights* jllm_hip_gguf_layer_weights(const jllm_hip_gguf_model* m);
void                          jllm_hip_gguf_model_free(jllm_hip_gguf_model* m);

/* Writer (GGUF v3, alignment 32): scalar u32 / f32 / string metadata and
 * tensors (copied at add time).  No reference counterpart in the runtime
 * (the reference reads files made by llama.cpp tools); used to store models
 * such as the benchmark's random Q4_K_M decoder. */
typedef struct jllm_hip_gguf_writer jllm_hip_gguf_writer;
jllm_hip_gguf_writer* jllm_hip_gguf_writer_create(void);
void jllm_hip_gguf_writer_free(jllm_hip_gguf_writer* w);
int  jllm_hip_gguf_writer_set_u32(jllm_hip_gguf_writer* w, const char* key, uint32_t value);
int  jllm_hip_gguf_writer_set_f32(jllm_hip_gguf_writer* w, const char* key, float value);
int  jllm_hip_gguf_writer_set_str(jllm_hip_gguf_writer* w, const char* key, const char* value);
int  jllm_hip_gguf_writer_add_tensor(jllm_hip_gguf_writer* w, const char* name, int ggml_type, int n_dims,
                                     const int64_t* dims, const void* data, int64_t bytes);
int  jllm_hip_gguf_writer_write(const jllm_hip_gguf_writer* w, const char* path);

#ifdef __cplusplus
}
#endif
#endif /* JLLM_HIP_H */
