// mmq.h -- internal interface of the gfx950 prefill GEMM (MMQ).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace jllm_hip {

constexpr int MMQ_TILE_N = 64;    // tokens per workgroup tile (Npad granularity of the kernel layout)
constexpr int MMQ_REF_NPAD = 64;  // Npad granularity of the reference-layout quantiser entry point

// activation quantiser in the reference block layout: x [N x K] fp16 ->
// [K/128][Npad] blocks of 144 B (ds4 = 1: half2 (d, sum x) per 32; ds4 = 0:
// float d per 32)
hipError_t quantize_mmq_launch(const uint16_t* x, void* q8, int N, int K, int Npad, bool ds4, hipStream_t st);

// the same values in the kernels' layout: codes [K/256][Npad][256] as fp16
// values (i8 = false; the Q6_K kernel) or int8 bytes (i8 = true; the Q4_K
// kernel), scale words [K/32][Npad] (DS4: half d | half sum << 16; D4:
// float d) (up != null: the values are half(silu(x) * up), the SwiGLU of
// gate x and up)
hipError_t quantize_mmq_f16_launch(const uint16_t* x, void* codes, uint32_t* scl, int N, int K, int Npad,
                                   bool ds4, hipStream_t st, const uint16_t* up = nullptr, bool i8 = false);
inline size_t mmq_codes_bytes(int K, int Npad) { return (size_t)K * Npad * 2; }     // fp16 layout
inline size_t mmq_codes8_bytes(int K, int Npad) { return (size_t)K * Npad; }        // int8 layout
inline size_t mmq_scales_bytes(int K, int Npad) { return (size_t)(K / 32) * Npad * 4; }

// RMSNorm + activation quantisation of residual-stream rows y [N][H] in one
// pass (one workgroup per row of Npad), the residual add that forms y
// optionally in front: mode 0: y as given; 1: y = half(y + res); 2: y =
// half(half(sum of the S fp32 partials ws[s][N][H]) + res).  normed =
// half(y * rrms * w) (not written when normed is null); the codes and scale
// words of each kind whose codes pointer is non-null (c8/s8: int8 codes, DS4
// words -- the Q4_K kernel's;
// c16/s16: fp16 codes, D4 words -- the Q6_K kernel's).  Every output has the
// bits of the separate residual add, rmsnorm_launch and quantiser.
struct NormQuantArgs {
    uint16_t* y;
    const uint16_t* res;
    const float* ws;
    int S, mode;
    uint16_t* normed;
    const void* w;
    float eps;
    void* c8;
    uint32_t* s8;
    void* c16;
    uint32_t* s16;
    int N, H, Npad;
};
// whether norm_quant_launch takes these arguments (16-byte aligned rows, H a
// multiple of 32 and <= 4096, w aligned like rmsnorm_launch's 16-byte path)
bool norm_quant_supported(const NormQuantArgs& a, bool w_fp32);
hipError_t norm_quant_launch(const NormQuantArgs& a, bool w_fp32, hipStream_t st);

// out_kind: 0 = fp16 y[N x M], 1 = fp32 y[N x M], 2 = raw int32 sub-block
// dots [N][M][K/G] (G = 32 for Q4_K, 16 for Q6_K).  splits > 1 (fp32 only):
// K is cut into `splits` ranges of whole super-blocks and range s writes
// its partial sums to y + s*N*M (reduce with splitk_reduce_launch).
// codes: int8 layout for Q4_K, fp16 layout for Q6_K
hipError_t mmq_launch(void* y, const uint8_t* W, int type, const void* codes, const uint32_t* scl, int M, int N,
                      int K, int Npad, int out_kind, int splits, hipStream_t st);

// Weight matrices of one multi-matrix launch (row tiles of segment s:
// [rt0[s], rt0[s+1]) of the grid's row-tile index; unused segments M = 0).
struct MmqSegs {
    const uint8_t* W[3];
    void* y[3];
    int M[3];
    int rt0[4];
};

// tile count from which a multi-matrix launch needs no split-K (the
// threshold of mmq_splits)
constexpr int MMQ_MULTI_MIN_TILES = 384;

// Q4_K only, fp16 y, no split: the nseg (<= 3) products W[s] . x -> y[s]
// of one quantised activation, one launch over all their row tiles.
hipError_t mmq_q4k_multi_launch(const uint8_t* const* W, void* const* y, const int* M, int nseg, const uint8_t* codes,
                                const uint32_t* scl, int N, int K, int Npad, hipStream_t st);

// The decoder's prefill Q/K/V (all Q4_K, no split) with the attention front
// (qk_post_kernel's step: q/k RMSNorm, RoPE, the KV-cache store) run in the
// tiles' epilogue: head_dim 128 (one workgroup tile = one head), y[0..2] =
// fa.q / fa.k / fa.v with packed rows, M = heads x 128; fa's other fields as
// qk_post_launch takes them (start_pos: position of token 0, k_dst / v_dst /
// scales addressing token 0's row).  Every output has the bits of the plain
// launch followed by qk_post_launch.
struct QKPostArgs;
hipError_t mmq_q4k_qkv_front_launch(const uint8_t* const* W, uint16_t* const* y, const int* M, const uint8_t* codes,
                                    const uint32_t* scl, int N, int K, int Npad, const QKPostArgs& fa,
                                    hipStream_t st);

// The decoder's prefill gate/up (both Q4_K, M rows each, M % 64 == 0, no
// split) with the SwiGLU half(silu(gate) * up) of the fp16 products
// quantised in the epilogue as the down GEMM's activation: act codes and
// scale words for K = M (int8 + DS4 when act_i8, else fp16 + D4), Npad
// token rows -- the bits quantize_mmq_f16_launch(gate, .., up) writes from
// the plain launch's gate and up.
hipError_t mmq_q4k_swiglu_launch(const uint8_t* gate, const uint8_t* up, int M, const uint8_t* codes,
                                 const uint32_t* scl, int N, int K, int Npad, void* act_codes, uint32_t* act_scl,
                                 bool act_i8, hipStream_t st);

// Split count for an N x M x K GEMM of weight type `type`: ranges of whole
// super-blocks chosen by a measured cost model (at most 16 ranges for Q4_K /
// Q5_K, 19 for Q6_K); a function of M, N, K and the type only.
int mmq_splits(int M, int N, int K, int type);

// y = sum of the `splits` fp32 partials ws[s][n], added in order s = 0, 1, ...
// (fp16 out with res: y = half(half(sum) + res))
hipError_t splitk_reduce_launch(void* y, const float* ws, int64_t n, int splits, int out_kind, hipStream_t st,
                                const uint16_t* res = nullptr);

// Q5_K batched GEMM (fp16 activation, no quantisation): out_kind 0 = fp16
// y[N x M], 1 = fp32 y[N x M]
hipError_t gemm_q5k_launch(void* y, const uint8_t* W, const uint16_t* x, int M, int N, int K, int out_kind,
                           int splits, hipStream_t st);

}  // namespace jllm_hip
