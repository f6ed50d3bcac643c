// gemv.h -- internal interface of the gfx950 GEMV kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace jllm_hip {

// OUT_SWIGLU: a gate/up pair (segments 0 and 1, same M and type) whose rows
// r are computed by the same wave; y of segment 0 receives
// half(silu(half(gate_r)) * half(up_r)), segment 1's y is not written.
enum OutKind { OUT_HALF = 0, OUT_F32 = 1, OUT_ADD = 2, OUT_SWIGLU = 3 };

// Activation prologue applied while the activation is staged: none or
// RMSNorm of x (x <- half(x / sqrt(mean(x^2) + eps) * w)), with the values
// of the separate RMSNorm kernel (up to the order of the sum of squares).
enum PreKind { PRE_NONE = 0, PRE_RMS = 1 };
struct GemvPre {
    int kind;
    const void* nw;         // RMSNorm weight [K], fp32 or fp16
    int nw_fp32;
    float eps;
};

// One output segment of a fused GEMV launch: rows [0, M) of W (type 12 or
// 14), result to y (fp16 or fp32), optional fp16 residual for OUT_ADD.
struct GemvSeg {
    void* y;
    const uint8_t* W;
    const uint16_t* res;
    int M;
    int type;
};

struct GemvArgs {
    GemvSeg seg[3];
    int nseg;
    int K;
    const uint16_t* x;     // fp16 activation [K]
    GemvPre pre;
};

// Arguments of the streaming kernel (filled by gemv_launch).  Segments
// are ordered first class first; their rows form one sequence, split into
// contiguous row ranges per workgroup.
struct StreamArgs {
    GemvSeg seg[3];
    int K;
    int nb;                 // K / 256
    int xlds_bytes;         // LDS bytes of the staged activation
    const uint16_t* x;
    int row_off[4];         // first row of each segment in the row sequence
    int row_split;          // rows of the first-class (Q4_K / Q5_K) segments
    int wg_split;           // workgroups serving the first-class rows
    int rows_q[2], rows_r[2];       // rows per workgroup (quotient, remainder) per class
    int slots_per_wg;       // LDS block slots per workgroup (max rows per workgroup * nb, x2 for OUT_SWIGLU)
    int swiglu;             // OUT_SWIGLU launch: row sequence = the M (gate, up) row pairs
    int ilv;                // 1: a workgroup's rounds are dealt to its waves round-robin
    GemvPre pre;
};

size_t gemv_lds_bytes(bool mmvq, int K);
hipError_t gemv_launch(const GemvArgs& a, bool mmvq, int out_kind, hipStream_t st);
hipError_t quantize_q8_1_aos_launch(const uint16_t* x, void* y, int K, hipStream_t st);

}  // namespace jllm_hip
