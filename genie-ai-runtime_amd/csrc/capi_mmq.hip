// capi_mmq.hip -- C ABI for the batched (prefill) GEMM: activation
// quantiser, int8 MFMA MMQ, and the routing of gemm_quant_batched
// (gemv_q4.cu:2478-2517): Q4_K / Q6_K through the MMQ, Q5_K through its
// fp16 GEMM (the reference runs Q5_K in float, gemv_q4.cu:2436-2440).
#include "capi_common.h"
#include "mmq.h"
#include "layer_ops.h"

using namespace jllm_hip;

namespace {
DeviceScratch g_q8;     // quantised activations (int8 and fp16 codes + scale words), grown on demand, never freed
DeviceScratch g_ws;     // split-K fp32 partials [splits][N][M], grown on demand, never freed
DeviceScratch g_q8b;    // a GEMM epilogue's output codes for the next GEMM (read while g_q8 is), never freed

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
    // the kernels address the weight matrix and the quantised activation
    // with 32-bit buffer offsets: refuse shapes whose byte counts would not
    // fit rather than read a truncated range
    const int64_t lim = ((int64_t)1 << 31) - 1;
    const int64_t wbytes = (int64_t)M * (K / 256) * 210, abytes = (int64_t)K * ((N + 63) / 64 * 64) * 2;
    if (wbytes > lim || abytes > lim) {
        fprintf(stderr, "[%s] shape M=%d N=%d K=%d exceeds the 2 GiB weight / activation ranges of the kernels\n",
                tag, M, N, K);
        return JLLM_ERR_INVALID;
    }
    return JLLM_OK;
}

// The product of an already quantised activation (q8 = codes + scale words
// of the right kind, or null for Q5_K) into y.
int mmq_after_quant(const char* tag, void* y, const void* Wd, int type, const uint16_t* x, const void* codes,
                    const uint32_t* scl, int M, int N, int K, int out_kind, hipStream_t st,
                    const uint16_t* res = nullptr, ResidualRows* defer = nullptr) {
    // split-K when the tile grid alone does not cover the chip: partials to
    // the workspace, then one ordered reduction into y
    const int splits = out_kind == 2 ? 1 : mmq_splits(M, N, K, type);
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
    if (type == 13) e = gemm_q5k_launch(dst, (const uint8_t*)Wd, x, M, N, K, kind, splits, st);
    else e = mmq_launch(dst, (const uint8_t*)Wd, type, codes, scl, M, N, K, npad_of(N), kind, splits, st);
    if (e == hipSuccess && defer && res) {
        // the residual add (and the split sum) left to the caller's next step
        *defer = ResidualRows{(uint16_t*)y, res, splits > 1 ? (const float*)dst : nullptr, splits, splits > 1 ? 2 : 1};
        return launch_status(e, tag);
    }
    if (e == hipSuccess && splits > 1) e = splitk_reduce_launch(y, (const float*)dst, (int64_t)N * M, splits, out_kind, st, res);
    else if (e == hipSuccess && res) e = vec_add_launch((uint16_t*)y, (const uint16_t*)y, res, (int64_t)N * M, st);
    return launch_status(e, tag);
}

const void* device_weight(const char* tag, const void* W) {
    const void* Wd = resolve_weight(W);
    if (!Wd) fprintf(stderr, "[%s] weight pointer %p is not device-visible (no host fallback)\n", tag, W);
    return Wd;
}

// q8 scratch for the two quantiser kinds, kind 0 = DS4 (Q4_K kernel: int8
// codes), kind 1 = D4 (Q6_K kernel: fp16 codes): the codes, then the scale
// words of each kind
int q8_scratch(const char* tag, int N, int K, void* (&codes)[2], uint32_t* (&scl)[2]) {
    const int Npad = npad_of(N);
    const size_t c8 = mmq_codes8_bytes(K, Npad), c16 = mmq_codes_bytes(K, Npad), sb = mmq_scales_bytes(K, Npad);
    uint8_t* q8 = (uint8_t*)g_q8.get(c8 + c16 + 2 * sb);
    if (!q8) {
        fprintf(stderr, "[%s] q8 scratch allocation failed\n", tag);
        return JLLM_ERR_NOMEM;
    }
    codes[0] = q8;
    codes[1] = q8 + c8;
    scl[0] = (uint32_t*)(q8 + c8 + c16);
    scl[1] = (uint32_t*)(q8 + c8 + c16 + sb);
    return JLLM_OK;
}

// the activation quantised for weight type `type` (12: kind 0, 14: kind 1)
hipError_t quantize_for(int type, const uint16_t* x, void* const (&codes)[2], uint32_t* const (&scl)[2], int N, int K,
                        hipStream_t st, const uint16_t* up = nullptr) {
    const int k = type == 12 ? 0 : 1;
    return quantize_mmq_f16_launch(x, codes[k], scl[k], N, K, npad_of(N), k == 0, st, up, k == 0);
}

int run_mmq(const char* tag, void* y, const void* W, int type, const uint16_t* x, int M, int N, int K,
            int out_kind, void* stream) {
    const void* Wd = device_weight(tag, W);
    if (!Wd) return JLLM_ERR_POINTER;
    if (!aligned16(Wd)) return JLLM_ERR_INVALID;
    hipStream_t st = (hipStream_t)stream;
    void* codes[2] = {nullptr, nullptr};
    uint32_t* scl[2] = {nullptr, nullptr};
    const int k = type == 12 ? 0 : 1;
    if (type != 13) {
        int r = q8_scratch(tag, N, K, codes, scl); if (r) return r;
        const hipError_t e = quantize_for(type, x, codes, scl, N, K, st);
        if (e != hipSuccess) return launch_status(e, tag);
    }
    return mmq_after_quant(tag, y, Wd, type, x, codes[k], scl[k], M, N, K, out_kind, st);
}
}  // namespace

namespace jllm_hip {
int gemm_batched_res(const char* tag, uint16_t* y, const void* W, int type, const uint16_t* x, const uint16_t* up,
                     uint16_t* act_tmp, const uint16_t* res, int M, int N, int K, void* stream,
                     ResidualRows* defer, const AttnQuant* pre) {
    if (defer) *defer = ResidualRows{y, res, nullptr, 0, 0};
    int st = check_gemm(tag, y, type, x, M, N, K, true); if (st) return st;
    if (M == 0 || N == 0) return JLLM_OK;
    if (!res || (up && (!act_tmp || !aligned16(up)))) return JLLM_ERR_INVALID;
    hipStream_t hs = (hipStream_t)stream;
    if (N == 1 || type == 13) {
        // no fused form: the SwiGLU into act_tmp, the product, the residual add
        if (up) {
            const hipError_t e = swiglu_launch(act_tmp, x, up, (int64_t)N * K, hs);
            if (e != hipSuccess) return launch_status(e, tag);
            x = act_tmp;
        }
        if (N == 1) {
            st = jllm_hip_gemv_quant_add(y, W, type, x, res, M, K, stream);
            return st;
        }
    }
    const void* Wd = device_weight(tag, W);
    if (!Wd) return JLLM_ERR_POINTER;
    if (!aligned16(Wd)) return JLLM_ERR_INVALID;
    void* codes[2] = {nullptr, nullptr};
    uint32_t* scl[2] = {nullptr, nullptr};
    const int k = type == 12 ? 0 : 1;
    if (type != 13 && pre) {
        if (pre->i8 != (type == 12) || pre->npad != npad_of(N)) return JLLM_ERR_INVALID;
        codes[k] = pre->codes;
        scl[k] = pre->scl;
    } else if (type != 13) {
        st = q8_scratch(tag, N, K, codes, scl); if (st) return st;
        const hipError_t e = quantize_for(type, x, codes, scl, N, K, hs, up);
        if (e != hipSuccess) return launch_status(e, tag);
    }
    return mmq_after_quant(tag, y, Wd, type, x, codes[k], scl[k], M, N, K, 0, hs, res, defer);
}

int gate_up_swiglu_prefill(const char* tag, const GemmOut* gu, const uint16_t* x, int N, int K, bool quantized,
                           int down_type, AttnQuant* act, bool* done, void* stream) {
    *done = false;
    const int M = gu[0].M;
    if (N <= 1 || gu[0].type != 12 || gu[1].type != 12 || gu[1].M != M || M <= 0 || M % 256 ||
        (down_type != 12 && down_type != 14))
        return JLLM_OK;
    const int Npad = npad_of(N);
    if ((int64_t)(M / 64) * (Npad / MMQ_TILE_N) < MMQ_MULTI_MIN_TILES) return JLLM_OK;
    const uint8_t* Wd[2];
    for (int i = 0; i < 2; i++) {
        int st = check_gemm(tag, gu[i].y, gu[i].type, x, M, N, K, true); if (st) return st;
        const void* w = device_weight(tag, gu[i].W);
        if (!w) return JLLM_ERR_POINTER;
        if (!aligned16(w)) return JLLM_ERR_INVALID;
        Wd[i] = (const uint8_t*)w;
    }
    hipStream_t hs = (hipStream_t)stream;
    void* codes[2] = {nullptr, nullptr};
    uint32_t* scl[2] = {nullptr, nullptr};
    int st = q8_scratch(tag, N, K, codes, scl); if (st) return st;
    if (!quantized) {
        const hipError_t e = quantize_for(12, x, codes, scl, N, K, hs);
        if (e != hipSuccess) return launch_status(e, tag);
    }
    // the down GEMM's codes (K = M) in their own scratch: g_q8 is being read
    const bool i8 = down_type == 12;
    const size_t cb = i8 ? mmq_codes8_bytes(M, Npad) : mmq_codes_bytes(M, Npad);
    uint8_t* o = (uint8_t*)g_q8b.get(cb + mmq_scales_bytes(M, Npad));
    if (!o) {
        fprintf(stderr, "[%s] activation scratch allocation failed\n", tag);
        return JLLM_ERR_NOMEM;
    }
    *act = AttnQuant{o, (uint32_t*)(o + cb), Npad, i8};
    st = launch_status(mmq_q4k_swiglu_launch(Wd[0], Wd[1], M, (const uint8_t*)codes[0], scl[0], N, K, Npad, o,
                                             (uint32_t*)(o + cb), i8, hs), tag);
    if (st == JLLM_OK) *done = true;
    return st;
}

int q8_codes(const char* tag, int type, int N, int K, AttnQuant* q) {
    if ((type != 12 && type != 14) || N <= 1 || K <= 0 || K % 256) return JLLM_ERR_INVALID;
    void* codes[2] = {nullptr, nullptr};
    uint32_t* scl[2] = {nullptr, nullptr};
    int st = q8_scratch(tag, N, K, codes, scl); if (st) return st;
    const int k = type == 12 ? 0 : 1;
    *q = AttnQuant{codes[k], scl[k], npad_of(N), k == 0};
    return JLLM_OK;
}

int residual_finish(const char* tag, const ResidualRows& r, int N, int M, void* stream) {
    const int64_t n = (int64_t)N * M;
    hipStream_t hs = (hipStream_t)stream;
    if (r.mode == 2) return launch_status(splitk_reduce_launch(r.y, r.ws, n, r.S, 0, hs, r.res), tag);
    if (r.mode == 1) return launch_status(vec_add_launch(r.y, r.y, r.res, n, hs), tag);
    return JLLM_OK;
}

int norm_rows(const char* tag, const ResidualRows& r, int N, int H, uint16_t* normed, const void* w, bool w_fp32,
              float eps, const GemmOut* outs, int n, bool* quantized, void* stream) {
    *quantized = false;
    if (N <= 0) return JLLM_OK;
    bool need[2] = {false, false};                   // DS4 (Q4_K), D4 (Q6_K)
    bool need_f16 = false;                           // an output reads the fp16 rows (Q5_K)
    for (int i = 0; i < n; i++) {
        if (outs[i].M == 0) continue;
        if (outs[i].type == 12) need[0] = true;
        else if (outs[i].type == 14) need[1] = true;
        else need_f16 = true;
    }
    NormQuantArgs a;
    a.y = r.y; a.res = r.res; a.ws = r.ws; a.S = r.S; a.mode = r.mode;
    a.normed = normed; a.w = w; a.eps = eps;
    a.c8 = nullptr; a.s8 = nullptr; a.c16 = nullptr; a.s16 = nullptr;
    a.N = N; a.H = H; a.Npad = N > 1 ? npad_of(N) : N;
    if (N > 1 && H % 256 == 0 && norm_quant_supported(a, w_fp32)) {
        void* codes[2] = {nullptr, nullptr};
        uint32_t* scl[2] = {nullptr, nullptr};
        if (need[0] || need[1]) {
            int st = q8_scratch(tag, N, H, codes, scl); if (st) return st;
        }
        if (need[0]) { a.c8 = codes[0]; a.s8 = scl[0]; }
        if (need[1]) { a.c16 = codes[1]; a.s16 = scl[1]; }
        if (!need_f16) a.normed = nullptr;          // every consumer reads the codes: no fp16 rows
        const int st = launch_status(norm_quant_launch(a, w_fp32, (hipStream_t)stream), tag);
        if (st == JLLM_OK) *quantized = true;
        return st;
    }
    int st = residual_finish(tag, r, N, H, stream); if (st) return st;
    return jllm_hip_fused_rmsnorm_residual(normed, r.y, nullptr, w, N, H, eps, w_fp32 ? 1 : 0, stream);
}

int qkv_front_prefill(const char* tag, const GemmOut* qkv, const uint16_t* x, int N, int K, bool quantized,
                      const QKPostArgs& fa, void* stream, bool* done) {
    *done = false;
    if (N <= 1 || fa.head_dim != 128 || fa.N != N || (fa.q_norm == nullptr) != (fa.k_norm == nullptr)) return JLLM_OK;
    const uint8_t* Wm[3];
    uint16_t* ym[3];
    int Mm[3];
    int64_t rtiles = 0;
    for (int i = 0; i < 3; i++) {
        if (qkv[i].type != 12 || qkv[i].M <= 0 || qkv[i].M % 128) return JLLM_OK;
        int st = check_gemm(tag, qkv[i].y, qkv[i].type, x, qkv[i].M, N, K, true); if (st) return st;
        const void* Wd = device_weight(tag, qkv[i].W);
        if (!Wd) return JLLM_ERR_POINTER;
        if (!aligned16(Wd)) return JLLM_ERR_INVALID;
        Wm[i] = (const uint8_t*)Wd; ym[i] = qkv[i].y; Mm[i] = qkv[i].M;
        rtiles += qkv[i].M / 128;
    }
    if (rtiles * (npad_of(N) / MMQ_TILE_N) < MMQ_MULTI_MIN_TILES) return JLLM_OK;
    hipStream_t hs = (hipStream_t)stream;
    void* codes[2] = {nullptr, nullptr};
    uint32_t* scl[2] = {nullptr, nullptr};
    int st = q8_scratch(tag, N, K, codes, scl); if (st) return st;
    if (!quantized) {
        const hipError_t e = quantize_for(12, x, codes, scl, N, K, hs);
        if (e != hipSuccess) return launch_status(e, tag);
    }
    st = launch_status(mmq_q4k_qkv_front_launch(Wm, ym, Mm, (const uint8_t*)codes[0], scl[0], N, K, npad_of(N), fa,
                                                hs), tag);
    if (st == JLLM_OK) *done = true;
    return st;
}

int gemm_batched_shared_x(const char* tag, const GemmOut* outs, int n, const uint16_t* x, int N, int K, void* stream,
                          bool quantized) {
    for (int i = 0; i < n; i++) {
        int st = check_gemm(tag, outs[i].y, outs[i].type, x, outs[i].M, N, K, true); if (st) return st;
    }
    if (N == 0) return JLLM_OK;
    if (N == 1) {
        for (int i = 0; i < n; i++) {
            int st = jllm_hip_gemv_quant(outs[i].y, outs[i].W, outs[i].type, x, outs[i].M, K, stream); if (st) return st;
        }
        return JLLM_OK;
    }
    hipStream_t hs = (hipStream_t)stream;
    void* codes[2] = {nullptr, nullptr};
    uint32_t* scl[2] = {nullptr, nullptr};
    bool need[2] = {false, false};                   // DS4 (Q4_K), D4 (Q6_K)
    for (int i = 0; i < n; i++) {
        if (outs[i].M == 0) continue;
        if (outs[i].type == 12) need[0] = true;
        if (outs[i].type == 14) need[1] = true;
    }
    if (need[0] || need[1]) {
        int st = q8_scratch(tag, N, K, codes, scl); if (st) return st;
        for (int k = 0; k < 2 && !quantized; k++) {
            if (!need[k]) continue;
            const hipError_t e = quantize_for(k == 0 ? 12 : 14, x, codes, scl, N, K, hs);
            if (e != hipSuccess) return launch_status(e, tag);
        }
    }
    // all-Q4_K products whose row tiles together cover the chip without
    // split-K (e.g. Q/K/V, or gate/up, of a 512-token chunk): one launch --
    // each tile is computed exactly as in its own launch without split-K
    {
        const uint8_t* Wm[3];
        void* ym[3];
        int Mm[3], nm = 0;
        int64_t rtiles = 0;
        bool all4 = n <= 3;
        for (int i = 0; i < n && all4; i++) {
            if (outs[i].M == 0) continue;
            if (outs[i].type != 12) { all4 = false; break; }
            const void* Wd = device_weight(tag, outs[i].W);
            if (!Wd) return JLLM_ERR_POINTER;
            if (!aligned16(Wd)) return JLLM_ERR_INVALID;
            Wm[nm] = (const uint8_t*)Wd; ym[nm] = outs[i].y; Mm[nm] = outs[i].M; nm++;
            rtiles += (outs[i].M + 127) / 128;
        }
        if (all4 && nm >= 2 && rtiles * (npad_of(N) / MMQ_TILE_N) >= MMQ_MULTI_MIN_TILES)
            return launch_status(mmq_q4k_multi_launch(Wm, ym, Mm, nm, (const uint8_t*)codes[0], scl[0], N, K,
                                                      npad_of(N), hs), tag);
    }
    for (int i = 0; i < n; i++) {
        if (outs[i].M == 0) continue;
        const void* Wd = device_weight(tag, outs[i].W);
        if (!Wd) return JLLM_ERR_POINTER;
        if (!aligned16(Wd)) return JLLM_ERR_INVALID;
        const int k = outs[i].type == 12 ? 0 : 1;
        int st = mmq_after_quant(tag, outs[i].y, Wd, outs[i].type, x, codes[k], scl[k], outs[i].M, N, K, 0, hs);
        if (st) return st;
    }
    return JLLM_OK;
}
}  // namespace jllm_hip

extern "C" {

int jllm_hip_gemm_quant_batched(uint16_t* y, const void* W, int type, const uint16_t* x,
                                int M, int N, int K, void* stream) {
    int st = check_gemm("GEMM", y, type, x, M, N, K, true); if (st) return st;
    if (M == 0 || N == 0) return JLLM_OK;
    if (N == 1) return jllm_hip_gemv_quant(y, W, type, x, M, K, stream);
    return run_mmq("GEMM", y, W, type, x, M, N, K, 0, stream);
}

int jllm_hip_gemm_quant_batched_multi(uint16_t* const* y, const void* const* W, const int* ggml_type, const int* M,
                                      int n, const uint16_t* x, int N, int K, void* stream) {
    if (!y || !W || !ggml_type || !M || n < 1 || n > 3) return JLLM_ERR_INVALID;
    GemmOut outs[3];
    for (int i = 0; i < n; i++) outs[i] = GemmOut{y[i], W[i], ggml_type[i], M[i]};
    return gemm_batched_shared_x("GEMM", outs, n, x, N, K, stream);
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

int jllm_hip_quantize_mmq_f16(const uint16_t* x, uint16_t* codes, uint32_t* scales, int N, int K, int Npad, int ds4,
                              void* stream) {
    if (!x || !codes || !scales || N < 0 || K <= 0 || K % 256 != 0 || Npad < N || Npad % MMQ_TILE_N != 0 ||
        !aligned16(x) || !aligned16(codes))
        return JLLM_ERR_INVALID;
    if (Npad == 0) return JLLM_OK;
    return launch_status(quantize_mmq_f16_launch(x, codes, scales, N, K, Npad, ds4 != 0, (hipStream_t)stream), "GEMM");
}

int jllm_hip_quantize_mmq_i8(const uint16_t* x, int8_t* codes, uint32_t* scales, int N, int K, int Npad, int ds4,
                             void* stream) {
    if (!x || !codes || !scales || N < 0 || K <= 0 || K % 256 != 0 || Npad < N || Npad % MMQ_TILE_N != 0 ||
        !aligned16(x) || !aligned16(codes))
        return JLLM_ERR_INVALID;
    if (Npad == 0) return JLLM_OK;
    return launch_status(quantize_mmq_f16_launch(x, codes, scales, N, K, Npad, ds4 != 0, (hipStream_t)stream,
                                                 nullptr, true), "GEMM");
}

int jllm_hip_mmq_subdots(int32_t* out, const void* W, int type, const uint16_t* x, int M, int N, int K,
                         void* stream) {
    int st = check_gemm("GEMM", out, type, x, M, N, K); if (st) return st;
    if (M == 0 || N == 0) return JLLM_OK;
    return run_mmq("GEMM", out, W, type, x, M, N, K, 2, stream);
}

}  // extern "C"
