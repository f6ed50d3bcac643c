// capi_mmq.hip -- C ABI for the batched (prefill) GEMM: activation
// quantiser, int8 MFMA MMQ, and the routing of gemm_quant_batched
// (gemv_q4.cu:2478-2517): Q4_K / Q6_K through the MMQ, Q5_K through its
// fp16 GEMM (the reference runs Q5_K in float, gemv_q4.cu:2436-2440).
#include "capi_common.h"
#include "mmq.h"

using namespace jllm_hip;

namespace {
DeviceScratch g_q8;     // quantised activations (fp16 codes + scale words), grown on demand, never freed
DeviceScratch g_ws;     // split-K fp32 partials [splits][N][M], grown on demand, never freed

int npad_of(int N) { return ((N + MMQ_TILE_N - 1) / MMQ_TILE_N) * MMQ_TILE_N; }

int check_gemm(const char* tag, const void* y, int type, const uint16_t* x, int M, int N, int K, bool q5 = false) {
    if (type != 12 && type != 14 && !(q5 && type == 13)) {
        fprintf(stderr, "[%s] FATAL: unsupported GPU GGML type %d\n", tag, type);
        return JLLM_ERR_UNSUPPORTED;
    }
    if (M < 0 || N < 0 || K <= 0 || K % 256 != 0) {
        fprintf(stderr, "[%s] bad shape M=%d N=%d K=%d (K must be a positive multiple of 256)\n", tag, M, N, K);
        return JLLM_ERR_INVALID;
    }
    if ((M > 0 && N > 0) && (!y || !x || !aligned16(x))) {
        fprintf(stderr, "[%s] output and 16-byte aligned activation pointers are required\n", tag);
        return JLLM_ERR_INVALID;
    }
    return JLLM_OK;
}

int run_mmq(const char* tag, void* y, const void* W, int type, const uint16_t* x, int M, int N, int K,
            int out_kind, void* stream) {
    const void* Wd = resolve_weight(W);
    if (!Wd) {
        fprintf(stderr, "[%s] weight pointer %p is not device-visible (no host fallback)\n", tag, W);
        return JLLM_ERR_POINTER;
    }
    if (!aligned16(Wd)) return JLLM_ERR_INVALID;
    hipStream_t st = (hipStream_t)stream;
    // split-K when the tile grid alone does not cover the chip: partials to
    // the workspace, then one ordered reduction into y
    const int splits = out_kind == 2 ? 1 : mmq_splits(M, N, K);
    void* dst = y;
    if (splits > 1) {
        dst = g_ws.get((size_t)splits * N * M * sizeof(float));
        if (!dst) {
            fprintf(stderr, "[%s] split-K workspace allocation failed\n", tag);
            return JLLM_ERR_NOMEM;
        }
    }
    const int kind = splits > 1 ? 1 : out_kind;
    hipError_t e;
    if (type == 13) {
        e = gemm_q5k_launch(dst, (const uint8_t*)Wd, x, M, N, K, kind, splits, st);
    } else {
        const int Npad = npad_of(N);
        const size_t cb = mmq_codes_bytes(K, Npad);
        uint8_t* q8 = (uint8_t*)g_q8.get(cb + mmq_scales_bytes(K, Npad));
        if (!q8) {
            fprintf(stderr, "[%s] q8 scratch allocation failed\n", tag);
            return JLLM_ERR_NOMEM;
        }
        uint16_t* codes = (uint16_t*)q8;
        uint32_t* scl = (uint32_t*)(q8 + cb);
        e = quantize_mmq_f16_launch(x, codes, scl, N, K, Npad, type == 12, st);
        if (e == hipSuccess) e = mmq_launch(dst, (const uint8_t*)Wd, type, codes, scl, M, N, K, Npad, kind, splits, st);
    }
    if (e == hipSuccess && splits > 1) e = splitk_reduce_launch(y, (const float*)dst, (int64_t)N * M, splits, out_kind, st);
    return launch_status(e, tag);
}
}  // namespace

extern "C" {

int jllm_hip_gemm_quant_batched(uint16_t* y, const void* W, int type, const uint16_t* x,
                                int M, int N, int K, void* stream) {
    int st = check_gemm("GEMM", y, type, x, M, N, K, true); if (st) return st;
    if (M == 0 || N == 0) return JLLM_OK;
    if (N == 1) return jllm_hip_gemv_quant(y, W, type, x, M, K, stream);
    return run_mmq("GEMM", y, W, type, x, M, N, K, 0, stream);
}

int jllm_hip_gemm_quant_batched_f32(float* y, const void* W, int type, const uint16_t* x,
                                    int M, int N, int K, void* stream) {
    int st = check_gemm("GEMM", y, type, x, M, N, K, true); if (st) return st;
    if (M == 0 || N == 0) return JLLM_OK;
    return run_mmq("GEMM", y, W, type, x, M, N, K, 1, stream);
}

int jllm_hip_quantize_mmq_q8_1(const uint16_t* x, void* q8, int N, int K, int Npad, int ds4, void* stream) {
    if (!x || !q8 || N < 0 || K <= 0 || K % 128 != 0 || Npad < N || Npad % MMQ_REF_NPAD != 0) return JLLM_ERR_INVALID;
    if (Npad == 0) return JLLM_OK;
    return launch_status(quantize_mmq_launch(x, q8, N, K, Npad, ds4 != 0, (hipStream_t)stream), "GEMM");
}

int jllm_hip_mmq_subdots(int32_t* out, const void* W, int type, const uint16_t* x, int M, int N, int K,
                         void* stream) {
    int st = check_gemm("GEMM", out, type, x, M, N, K); if (st) return st;
    if (M == 0 || N == 0) return JLLM_OK;
    return run_mmq("GEMM", out, W, type, x, M, N, K, 2, stream);
}

}  // extern "C"
