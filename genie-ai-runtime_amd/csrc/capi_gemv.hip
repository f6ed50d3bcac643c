// capi_gemv.hip -- C ABI for the GEMV family, the mapped-weight registry
// and status strings.  Routing follows the reference dispatcher defaults
// (gemv_q4.cu:1245-1616, 2633-2775).
#include <mutex>
#include <vector>
#include "capi_common.h"
#include "gemv.h"

using namespace jllm_hip;

// The engine's registry lookup (defined in its src/engine/model.cpp when the
// engine is linked in; a null address otherwise).
namespace jllm {
const void* resolve_mapped_weight_device_ptr(const void* host_ptr) __attribute__((weak));
}

namespace {
struct MappedRegion { const char* host; const char* dev; int64_t bytes; };
std::mutex g_reg_mu;
std::vector<MappedRegion> g_regions;
}

namespace jllm_hip {
const void* resolve_weight(const void* W) {
    if (!W) return nullptr;
    if (const void* m = jllm_hip_resolve_mapped_weight_device_ptr(W)) return m;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, W) != hipSuccess) { (void)hipGetLastError(); return nullptr; }
    if (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged) return W;
    return nullptr;
}
}

extern "C" {

const char* jllm_hip_status_string(int s) {
    switch (s) {
        case JLLM_OK: return "ok";
        case JLLM_ERR_INVALID: return "invalid argument";
        case JLLM_ERR_UNSUPPORTED: return "unsupported ggml type";
        case JLLM_ERR_LAUNCH: return "kernel launch failed";
        case JLLM_ERR_NOMEM: return "scratch allocation failed";
        case JLLM_ERR_POINTER: return "weight pointer not visible to the GPU";
        default: return "unknown status";
    }
}

int jllm_hip_register_mapped_weight_region(const void* host_base, const void* device_base, int64_t bytes) {
    if (!host_base || !device_base || bytes <= 0) return JLLM_ERR_INVALID;
    std::lock_guard<std::mutex> lk(g_reg_mu);
    for (auto& r : g_regions)
        if (r.host == (const char*)host_base) { r.dev = (const char*)device_base; r.bytes = bytes; return JLLM_OK; }
    g_regions.push_back({(const char*)host_base, (const char*)device_base, bytes});
    return JLLM_OK;
}

void jllm_hip_clear_mapped_weight_region(const void* host_base) {
    std::lock_guard<std::mutex> lk(g_reg_mu);
    for (size_t i = 0; i < g_regions.size(); i++)
        if (g_regions[i].host == (const char*)host_base) { g_regions.erase(g_regions.begin() + i); return; }
}

const void* jllm_hip_resolve_mapped_weight_device_ptr(const void* host_ptr) {
    const char* p = (const char*)host_ptr;
    {
        std::lock_guard<std::mutex> lk(g_reg_mu);
        for (const auto& r : g_regions)
            if (p >= r.host && p < r.host + r.bytes) return r.dev + (p - r.host);
    }
    // then the engine's own registry (src/engine/model.cpp:39-66) when it is linked in
    if (&jllm::resolve_mapped_weight_device_ptr) return jllm::resolve_mapped_weight_device_ptr(host_ptr);
    return nullptr;
}

}  // extern "C"

namespace {

constexpr int MAX_K = 28672;
constexpr int QK_K_HOST = 256;

int check_common(const char* tag, int K, const uint16_t* x) {
    if (K <= 0 || K % QK_K_HOST != 0 || K > MAX_K) {
        fprintf(stderr, "[%s] K=%d must be a positive multiple of 256 and <= %d\n", tag, K, MAX_K);
        return JLLM_ERR_INVALID;
    }
    if (!x || !aligned16(x)) {
        fprintf(stderr, "[%s] activation pointer must be non-null and 16-byte aligned\n", tag);
        return JLLM_ERR_INVALID;
    }
    return JLLM_OK;
}

int make_seg(const char* tag, GemvSeg& s, void* y, const void* W, int type, int M, const uint16_t* res) {
    if (type != 12 && type != 13 && type != 14) {
        fprintf(stderr, "[%s] FATAL: unsupported GPU GGML type %d (M=%d)\n", tag, type, M);
        return JLLM_ERR_UNSUPPORTED;
    }
    if (M < 0 || (M > 0 && !y)) return JLLM_ERR_INVALID;
    const void* Wd = M > 0 ? resolve_weight(W) : W;
    if (M > 0 && !Wd) {
        fprintf(stderr, "[%s] weight pointer %p is not device-visible (no host fallback)\n", tag, W);
        return JLLM_ERR_POINTER;
    }
    if (M > 0 && !aligned16(Wd)) {
        fprintf(stderr, "[%s] weight pointer must be 16-byte aligned\n", tag);
        return JLLM_ERR_INVALID;
    }
    s.y = y; s.W = (const uint8_t*)Wd; s.res = res; s.M = M; s.type = type;
    return JLLM_OK;
}

// RMSNorm prologue: the whole activation is staged in the first pass
int set_rms(const char* tag, GemvArgs& a, const void* nw, int fp32, float eps) {
    if (a.K > 4096) {
        fprintf(stderr, "[%s] fused RMSNorm needs K <= 4096 (K=%d)\n", tag, a.K);
        return JLLM_ERR_INVALID;
    }
    if (!nw || !aligned16(nw)) {
        fprintf(stderr, "[%s] RMSNorm weight pointer must be non-null and 16-byte aligned\n", tag);
        return JLLM_ERR_INVALID;
    }
    a.pre.kind = PRE_RMS; a.pre.nw = nw; a.pre.nw_fp32 = fp32 != 0; a.pre.eps = eps;
    return JLLM_OK;
}

// MMVQ (q8_1 activation) or float dequant, by the reference dispatchers'
// routes: single rows by type (gemv_q4.cu:1263-1290: Q4_K and Q6_K MMVQ,
// Q5_K float), pairs only for Q4_K+Q4_K (:1391), triples for the four
// instantiated combinations of Q4_K/Q6_K (:1475-1490); anything else float.
bool mmvq_single(int t) { return t != 13; }
bool mmvq_pair(int t0, int t1) { return t0 == 12 && t1 == 12; }
bool mmvq_triple(int t0, int t1, int t2) {
    return (t0 == 12 && t1 == 12 && (t2 == 12 || t2 == 14)) || (t0 == 14 && t1 == 14 && t2 == 14) ||
           (t0 == 14 && t1 == 12 && t2 == 12);
}

int run(const char* tag, GemvArgs& a, bool mmvq, int out, void* stream) {
    return launch_status(gemv_launch(a, mmvq, out, (hipStream_t)stream), tag);
}

}  // namespace

extern "C" {

int jllm_hip_gemv_quant(uint16_t* y, const void* W, int type, const uint16_t* x, int M, int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    GemvArgs a{}; a.nseg = 1; a.K = K; a.x = x;
    if ((st = make_seg("GEMV", a.seg[0], y, W, type, M, nullptr))) return st;
    return run("GEMV", a, mmvq_single(type), OUT_HALF, stream);
}

int jllm_hip_gemv_quant_f32(float* y, const void* W, int type, const uint16_t* x, int M, int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    GemvArgs a{}; a.nseg = 1; a.K = K; a.x = x;
    if ((st = make_seg("GEMV", a.seg[0], y, W, type, M, nullptr))) return st;
    return run("GEMV", a, type == 12, OUT_F32, stream);
}

int jllm_hip_gemv_quant_dequant_f32(float* y, const void* W, int type, const uint16_t* x, int M, int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    GemvArgs a{}; a.nseg = 1; a.K = K; a.x = x;
    if ((st = make_seg("GEMV", a.seg[0], y, W, type, M, nullptr))) return st;
    return run("GEMV", a, false, OUT_F32, stream);
}

int jllm_hip_gemv_quant_add(uint16_t* y, const void* W, int type, const uint16_t* x, const uint16_t* residual,
                            int M, int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    if (M > 0 && !residual) return JLLM_ERR_INVALID;
    GemvArgs a{}; a.nseg = 1; a.K = K; a.x = x;
    if ((st = make_seg("GEMV", a.seg[0], y, W, type, M, residual))) return st;
    return run("GEMV", a, false, OUT_ADD, stream);
}

int jllm_hip_gemv_quant_pair(uint16_t* y0, const void* W0, int t0, int M0,
                             uint16_t* y1, const void* W1, int t1, int M1,
                             const uint16_t* x, int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    GemvArgs a{}; a.nseg = 2; a.K = K; a.x = x;
    if ((st = make_seg("GEMV", a.seg[0], y0, W0, t0, M0, nullptr))) return st;
    if ((st = make_seg("GEMV", a.seg[1], y1, W1, t1, M1, nullptr))) return st;
    return run("GEMV", a, mmvq_pair(t0, t1), OUT_HALF, stream);
}

int jllm_hip_gemv_quant_triple(uint16_t* y0, const void* W0, int t0, int M0,
                               uint16_t* y1, const void* W1, int t1, int M1,
                               uint16_t* y2, const void* W2, int t2, int M2,
                               const uint16_t* x, int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    GemvArgs a{}; a.nseg = 3; a.K = K; a.x = x;
    if ((st = make_seg("GEMV", a.seg[0], y0, W0, t0, M0, nullptr))) return st;
    if ((st = make_seg("GEMV", a.seg[1], y1, W1, t1, M1, nullptr))) return st;
    if ((st = make_seg("GEMV", a.seg[2], y2, W2, t2, M2, nullptr))) return st;
    return run("GEMV", a, mmvq_triple(t0, t1, t2), OUT_HALF, stream);
}

int jllm_hip_gemv_quant_triple_rmsnorm(uint16_t* y0, const void* W0, int t0, int M0,
                                       uint16_t* y1, const void* W1, int t1, int M1,
                                       uint16_t* y2, const void* W2, int t2, int M2,
                                       const uint16_t* x, const void* norm_weight, int weight_fp32, float eps,
                                       int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    GemvArgs a{}; a.nseg = 3; a.K = K; a.x = x;
    if ((st = set_rms("GEMV", a, norm_weight, weight_fp32, eps))) return st;
    if ((st = make_seg("GEMV", a.seg[0], y0, W0, t0, M0, nullptr))) return st;
    if ((st = make_seg("GEMV", a.seg[1], y1, W1, t1, M1, nullptr))) return st;
    if ((st = make_seg("GEMV", a.seg[2], y2, W2, t2, M2, nullptr))) return st;
    return run("GEMV", a, mmvq_triple(t0, t1, t2), OUT_HALF, stream);
}

int jllm_hip_gemv_quant_pair_rmsnorm(uint16_t* y0, const void* W0, int t0, int M0,
                                     uint16_t* y1, const void* W1, int t1, int M1,
                                     const uint16_t* x, const void* norm_weight, int weight_fp32, float eps,
                                     int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    GemvArgs a{}; a.nseg = 2; a.K = K; a.x = x;
    if ((st = set_rms("GEMV", a, norm_weight, weight_fp32, eps))) return st;
    if ((st = make_seg("GEMV", a.seg[0], y0, W0, t0, M0, nullptr))) return st;
    if ((st = make_seg("GEMV", a.seg[1], y1, W1, t1, M1, nullptr))) return st;
    return run("GEMV", a, mmvq_pair(t0, t1), OUT_HALF, stream);
}

int jllm_hip_gemv_quant_f32_rmsnorm(float* y, const void* W, int type, const uint16_t* x, const void* norm_weight,
                                    int weight_fp32, float eps, int M, int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    GemvArgs a{}; a.nseg = 1; a.K = K; a.x = x;
    if ((st = set_rms("GEMV", a, norm_weight, weight_fp32, eps))) return st;
    if ((st = make_seg("GEMV", a.seg[0], y, W, type, M, nullptr))) return st;
    return run("GEMV", a, type == 12, OUT_F32, stream);
}

// gate/up pair with the SwiGLU in the epilogue: act = half(silu(half(W_gate x)) * half(W_up x))
static int pair_swiglu(uint16_t* act, const void* Wg, int tg, const void* Wu, int tu, int M, const uint16_t* x,
                       const void* norm_weight, int weight_fp32, float eps, bool rms, int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    if (tg != tu || (tg != 12 && tg != 13)) {
        fprintf(stderr, "[GEMV] fused SwiGLU pair needs gate and up of one type, Q4_K or Q5_K (got %d, %d)\n", tg, tu);
        return JLLM_ERR_UNSUPPORTED;
    }
    GemvArgs a{}; a.nseg = 2; a.K = K; a.x = x;
    if (rms && (st = set_rms("GEMV", a, norm_weight, weight_fp32, eps))) return st;
    if ((st = make_seg("GEMV", a.seg[0], act, Wg, tg, M, nullptr))) return st;
    if ((st = make_seg("GEMV", a.seg[1], act, Wu, tu, M, nullptr))) return st;
    return run("GEMV", a, mmvq_pair(tg, tu), OUT_SWIGLU, stream);
}

int jllm_hip_gemv_quant_pair_swiglu(uint16_t* act, const void* W_gate, int type_gate, const void* W_up, int type_up,
                                    int M, const uint16_t* x, int K, void* stream) {
    return pair_swiglu(act, W_gate, type_gate, W_up, type_up, M, x, nullptr, 0, 0.0f, false, K, stream);
}

int jllm_hip_gemv_quant_pair_rmsnorm_swiglu(uint16_t* act, const void* W_gate, int type_gate, const void* W_up,
                                            int type_up, int M, const uint16_t* x, const void* norm_weight,
                                            int weight_fp32, float eps, int K, void* stream) {
    return pair_swiglu(act, W_gate, type_gate, W_up, type_up, M, x, norm_weight, weight_fp32, eps, true, K, stream);
}

int jllm_hip_quantize_q8_1(const uint16_t* x, void* y, int K, void* stream) {
    int st = check_common("GEMV", K, x); if (st) return st;
    if (!y || ((uintptr_t)y & 3u)) return JLLM_ERR_INVALID;
    return launch_status(quantize_q8_1_aos_launch(x, y, K, (hipStream_t)stream), "GEMV");
}

}  // extern "C"
