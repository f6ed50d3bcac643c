// capi_attn.hip -- C ABI for decode attention, the split-K partials buffer
// and the KV quantiser (attention.cu:975-1075, convert.cu:71-75).
#include "capi_common.h"
#include "attention.h"
#include "convert.h"
#include <mutex>

using namespace jllm_hip;

// Split-K partials of the allocation-free decode entry point: a fixed
// per-device array, held by each GPU the library runs on until the process
// ends.  Host code never uses its name as an address (that is a host-side
// stand-in): the device address comes from hipGetSymbolAddress, once per
// device, and only that address is passed to kernels.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)4 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {
DeviceScratch g_part;    // split-K partials + counters, grown on demand (zeroed), never freed

constexpr int NOALLOC_MAX_DEV = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[NOALLOC_MAX_DEV] = {};

// the device address of `scratch` on the current device (looked up on the
// first call per device); nullptr on failure
void* noalloc_scratch() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEV) return nullptr;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "[attention] hipGetSymbolAddress(scratch) failed on device %d: %s\n", dev,
                    hipGetErrorString(e));
            (void)hipGetLastError();
            return nullptr;
        }
        g_noalloc_ptr[dev] = p;
    }
    return g_noalloc_ptr[dev];
}

int attn_check(const void* out, const void* q, const void* k, const void* v, int n_heads, int n_kv, int hd,
               int chd, int seq, int kv_int8, int window) {
    if (!out || !q || (seq > 0 && (!k || !v))) return JLLM_ERR_INVALID;
    if (n_kv <= 0 || n_kv > ATTN_MAX_KV || n_heads <= 0 || n_heads % n_kv != 0 || n_heads / n_kv > 16) {
        fprintf(stderr, "[attention] n_heads=%d n_kv_heads=%d: need n_heads %% n_kv == 0 and <= 16 q heads per kv head\n", n_heads, n_kv);
        return JLLM_ERR_INVALID;
    }
    if (hd <= 0 || hd % 32 != 0 || hd > 128 || chd < hd || seq < 0 || window < 0) {
        fprintf(stderr, "[attention] head_dim=%d cache_head_dim=%d: need head_dim %% 32 == 0, <= 128, cache_head_dim >= head_dim\n", hd, chd);
        return JLLM_ERR_INVALID;
    }
    const int eb = kv_int8 ? 1 : 2;
    if ((chd * eb) % 16 != 0 || !aligned16(k) || !aligned16(v) || !aligned16(q)) {
        fprintf(stderr, "[attention] KV rows and q must be 16-byte aligned\n");
        return JLLM_ERR_INVALID;
    }
    return JLLM_OK;
}

// part: the caller's partials buffer (allocation-free entry), else the
// library's grown-on-demand one
int attn_run(uint16_t* out, const uint16_t* q, const void* k, const void* v, int n_heads, int n_kv, int hd, int chd,
             int seq, float scale, int kv_int8, const float* ks, const float* vs, int window, int n_splits,
             void* stream, const int32_t* pos_dev = nullptr, float* part = nullptr) {
    int st = attn_check(out, q, k, v, n_heads, n_kv, hd, chd, pos_dev ? 1 : seq, kv_int8, window);
    if (st) return st;
    if (n_splits < 1) n_splits = 1;
    if (n_splits > ATTN_MAX_SPLITS) n_splits = ATTN_MAX_SPLITS;
    int* counters = nullptr;
    if (!part) {
        uint8_t* sc = (uint8_t*)g_part.get(attn_scratch_bytes(n_heads, n_splits, hd));
        if (!sc) return JLLM_ERR_NOMEM;
        counters = (int*)sc;
        part = (float*)(sc + ATTN_COUNTER_BYTES);
    }
    AttnArgs a;
    a.out = out; a.q = q; a.k = k; a.v = v; a.ks = ks; a.vs = vs;
    a.counters = counters;
    a.part = part;
    a.n_heads = n_heads; a.n_kv = n_kv; a.head_dim = hd; a.cache_head_dim = chd;
    // the n_splits key ranges run as workgroups of W waves whose states are
    // combined in LDS: n_splits / W partials (one launch when that is 1)
    const int W = attn_decode_waves(n_splits);
    const int groups = (n_splits + W - 1) / W;
    a.seq = seq; a.window = window; a.n_splits = groups; a.scale = scale; a.tokens = 1; a.tq = 1; a.wsplit = W;
    a.pos_dev = pos_dev;
    return launch_status(attn_launch(a, kv_int8 != 0, (hipStream_t)stream), "attention");
}
}  // namespace

extern "C" {

int jllm_hip_decode_attn_splits(int seq_len) { return attn_splits(seq_len, 8); }

float* jllm_hip_get_splitk_partials(int n_heads, int n_splits, int head_dim) {
    if (n_heads <= 0 || n_splits <= 0 || head_dim <= 0) return nullptr;
    // the largest the decode kernels use: 256 KV heads x 16, 256 splits, head_dim 128
    if (n_heads > ATTN_MAX_KV * 16 || n_splits > ATTN_MAX_SPLITS || head_dim > 128) {
        fprintf(stderr, "[attention] get_splitk_partials(%d, %d, %d): beyond the kernels' limits\n", n_heads,
                n_splits, head_dim);
        return nullptr;
    }
    uint8_t* scratch = (uint8_t*)g_part.get(attn_scratch_bytes(n_heads, n_splits, head_dim));
    return scratch ? (float*)(scratch + ATTN_COUNTER_BYTES) : nullptr;
}

int jllm_hip_flash_attention_decode(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                    int n_heads, int n_kv_heads, int head_dim, int cache_head_dim, int seq_len,
                                    float scale, int kv_int8, const float* k_scales, const float* v_scales,
                                    int window, void* stream) {
    return attn_run(out, q, k, v, n_heads, n_kv_heads, head_dim, cache_head_dim, seq_len, scale, kv_int8,
                    k_scales, v_scales, window, attn_splits(seq_len, n_kv_heads), stream);
}

int jllm_hip_flash_attention_decode_splits(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                           int n_heads, int n_kv_heads, int head_dim, int cache_head_dim,
                                           int seq_len, float scale, int kv_int8, const float* k_scales,
                                           const float* v_scales, int window, int n_splits, void* stream) {
    return attn_run(out, q, k, v, n_heads, n_kv_heads, head_dim, cache_head_dim, seq_len, scale, kv_int8,
                    k_scales, v_scales, window, n_splits, stream);
}

int jllm_hip_flash_attention_decode_dyn(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                        int n_heads, int n_kv_heads, int head_dim, int cache_head_dim,
                                        const int32_t* d_pos, float scale, int kv_int8, const float* k_scales,
                                        const float* v_scales, int window, int n_splits, void* stream) {
    if (!d_pos) return JLLM_ERR_INVALID;
    return attn_run(out, q, k, v, n_heads, n_kv_heads, head_dim, cache_head_dim, 0, scale, kv_int8, k_scales,
                    v_scales, window, n_splits, stream, d_pos);
}

int jllm_hip_flash_attention_decode_noalloc(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                            int n_heads, int n_kv_heads, int head_dim, int cache_head_dim,
                                            int seq_len, float scale, int kv_int8, const float* k_scales,
                                            const float* v_scales, int window, void* stream) {
    const int n_splits = attn_splits(seq_len, n_kv_heads);
    // the partials attn_run writes: one per workgroup of W key ranges
    const int W = attn_decode_waves(n_splits), groups = (n_splits + W - 1) / W;
    if (n_heads > 0 && head_dim > 0 && groups > 1 &&
        attn_partials_floats(n_heads, groups, head_dim) * sizeof(float) > NOALLOC_SCRATCH_BYTES) {
        fprintf(stderr, "[attention] decode_noalloc: %d heads x %d partials x (2 + %d) floats exceed the %zu-byte "
                        "static partials buffer\n", n_heads, groups, head_dim, NOALLOC_SCRATCH_BYTES);
        return JLLM_ERR_INVALID;
    }
    // argument errors first, so that no device state is touched for them
    int st = attn_check(out, q, k, v, n_heads, n_kv_heads, head_dim, cache_head_dim, seq_len, kv_int8, window);
    if (st) return st;
    float* part = (float*)noalloc_scratch();
    if (!part) return JLLM_ERR_LAUNCH;
    return attn_run(out, q, k, v, n_heads, n_kv_heads, head_dim, cache_head_dim, seq_len, scale, kv_int8, k_scales,
                    v_scales, window, n_splits, stream, nullptr, part);
}

int jllm_hip_flash_attention_prefill_batched(uint16_t* out, const uint16_t* q, const void* k, const void* v,
                                             int n_heads, int n_kv_heads, int head_dim, int cache_head_dim, int N,
                                             int start_pos, float scale, int kv_int8, const float* k_scales,
                                             const float* v_scales, int window, void* stream) {
    return jllm_hip::prefill_attention(out, q, k, v, n_heads, n_kv_heads, head_dim, cache_head_dim, N, start_pos, scale,
                                       kv_int8, k_scales, v_scales, window, nullptr, stream, nullptr);
}
}  // extern "C"

namespace jllm_hip {
int prefill_attention(uint16_t* out, const uint16_t* q, const void* k, const void* v, int n_heads, int n_kv_heads,
                      int head_dim, int cache_head_dim, int N, int start_pos, float scale, int kv_int8,
                      const float* k_scales, const float* v_scales, int window, const AttnQuant* quant, void* stream,
                      bool* quantized) {
    if (quantized) *quantized = false;
    if (N < 0 || start_pos < 0 || N > 65535) return JLLM_ERR_INVALID;
    if (N == 0) return JLLM_OK;
    int st = attn_check(out, q, k, v, n_heads, n_kv_heads, head_dim, cache_head_dim, start_pos + 1, kv_int8, window);
    if (st) return st;
    AttnArgs a;
    a.out = out; a.q = q; a.k = k; a.v = v; a.ks = k_scales; a.vs = v_scales;
    a.counters = nullptr; a.part = nullptr;
    a.n_heads = n_heads; a.n_kv = n_kv_heads; a.head_dim = head_dim; a.cache_head_dim = cache_head_dim;
    a.seq = start_pos + 1; a.window = window; a.n_splits = 1; a.scale = scale; a.tokens = N;
    // several query tokens per wave: each KV tile serves tq tokens x G heads
    a.tq = ATTN_MAX_COLUMNS / (n_heads / n_kv_heads);
    if (a.tq < 1) a.tq = 1;
    a.wsplit = ATTN_PREFILL_WAVES;     // (used when tq > 1)
    const bool q8 = quant && quantized && a.tq > 1 && a.wsplit > 1 && head_dim % 32 == 0;
    if (q8) { a.qcodes = quant->codes; a.qscl = quant->scl; a.q_npad = quant->npad; a.q_i8 = quant->i8 ? 1 : 0; }
    const int st2 = launch_status(attn_launch(a, kv_int8 != 0, (hipStream_t)stream), "attention prefill");
    if (st2 == JLLM_OK && q8) *quantized = true;
    return st2;
}
}  // namespace jllm_hip

extern "C" {

int jllm_hip_fp16_to_int8(int8_t* dst, float* scale_out, const uint16_t* src, int rows, int cols, void* stream) {
    if (rows < 0 || cols <= 0 || (rows > 0 && (!dst || !src))) return JLLM_ERR_INVALID;
    if (rows == 0) return JLLM_OK;
    return launch_status(fp16_to_int8_launch(dst, scale_out, src, rows, cols, (hipStream_t)stream), "convert");
}

}  // extern "C"
