// attention.h -- internal interface of the gfx950 split-K decode attention.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jllm_hip {

struct AttnArgs {
    uint16_t* out;            // fp16 [n_heads x head_dim]
    const uint16_t* q;        // fp16 [n_heads x head_dim]
    const void* k;            // int8 or fp16 [seq][n_kv * cache_head_dim]
    const void* v;
    const float* ks;          // fp32 [pos][n_kv] (int8 only; may be null -> 1)
    const float* vs;
    float* part;              // partials: m [H*S] | l [H*S] | acc [H*S*hd]
    int* counters;            // [n_kv] split-completion counters, zero between calls
    int n_heads, n_kv, head_dim, cache_head_dim, seq, window, n_splits;
    // decode only (tokens == 1): when not null, the key count is read on the
    // device as *pos_dev + 1 and `seq` is ignored (a captured graph replays
    // for every position; the split count stays the host's n_splits)
    const int* pos_dev = nullptr;
    float scale;
    // query tokens (grid z): token t attends to keys [0, seq + t) and reads
    // q / writes out at t * n_heads * head_dim.  tokens > 1 needs n_splits 1.
    int tokens;
    // query tokens per wave (prefill): the wave's columns are tq tokens x
    // the G heads of its KV head, tq * G <= ATTN_MAX_COLUMNS; 1 for decode.
    int tq;
    // waves per workgroup (<= ATTN_MAX_WAVES): the workgroup's key tiles are
    // dealt to its waves round-robin by absolute tile position, and their
    // softmax states are combined in LDS in wave order (decode: into the
    // output, or into the workgroup's partial when n_splits > 1).
    int wsplit;
    // prefill with several waves per workgroup: when qcodes is set the
    // output rows are also quantised for the next GEMM, as the MMQ
    // activation quantiser would from the fp16 output: int8 codes and DS4
    // words (q_i8) or fp16 codes and D4 words, q_npad token rows
    void* qcodes = nullptr;
    uint32_t* qscl = nullptr;
    int q_npad = 0, q_i8 = 1;
};
constexpr int ATTN_MAX_WAVES = 8;
// measured (512-token prefill, one layer): 1 wave 41.4 us, 2 waves 37.5 us, 4 waves 38.6 us; with the
// token blocks dispatched last-first: 2 waves 36.1 us, 4 waves 36.8 us, 8 waves 52.7 us
// (with the combination's per-column weights formed once: 1 / 2 / 3 / 4 waves 39.0 / 29.0 / 31.3 / 29.7 us;
// with 32 columns per wave (P' high / low as two A operands): 1 / 2 / 3 / 4 / 6 / 8 waves
// 38.7 / 23.4 / 20.8 / 19.0 / 25.7 / 24.8 us)
constexpr int ATTN_PREFILL_WAVES = 4;

constexpr int ATTN_MAX_SPLITS = 256;
constexpr int ATTN_MAX_COLUMNS = 32;   // (token, head) columns per prefill wave
int attn_splits(int seq_len, int n_kv);
// waves per decode workgroup for n_splits key ranges
int attn_decode_waves(int n_splits);
size_t attn_partials_floats(int n_heads, int n_splits, int head_dim);
// Scratch layout: ATTN_COUNTER_BYTES of per-KV-head counters (fixed offset,
// zero before the first call, reset by every call) followed by the partials.
constexpr int ATTN_MAX_KV = 256;
constexpr size_t ATTN_COUNTER_BYTES = ATTN_MAX_KV * sizeof(int);
size_t attn_scratch_bytes(int n_heads, int n_splits, int head_dim);
hipError_t attn_launch(const AttnArgs& a, bool kv_int8, hipStream_t st);

}  // namespace jllm_hip
