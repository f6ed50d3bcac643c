// gemv.h -- internal interface of the gfx950 GEMV kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace jllm_hip {

enum OutKind { OUT_HALF = 0, OUT_F32 = 1, OUT_ADD = 2 };

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
    int lpr;               // lanes per row (filled by gemv_launch)
    int gend[3];           // cumulative row-group ends per segment (filled by gemv_launch)
    int per_q;             // blocks per quad and row (filled by gemv_launch)
    int g_split;           // row groups of Q4_K segments (filled by gemv_launch)
    int wg_split;          // workgroups serving Q4_K (filled by gemv_launch)
};

size_t gemv_lds_bytes(bool mmvq, int K);
hipError_t gemv_launch(const GemvArgs& a, bool mmvq, int out_kind, int lpr_override, hipStream_t st);
hipError_t quantize_q8_1_aos_launch(const uint16_t* x, void* y, int K, hipStream_t st);

}  // namespace jllm_hip
