// anyorder_launch.hip -- microbenchmark: do kernels launched on one stream
// with hipExtAnyOrderLaunch overlap on gfx950, and what does a chain of
// dependent streaming phases gain when each kernel issues its first weight
// round and then waits (bounded) on the previous kernel's completion?
//
// The 144 phases of grid_barrier.hip, one kernel each (512 workgroups of 4
// waves).  Each kernel counts its finished workgroups on 16 device-scope
// sub-counters (one per workgroup group b % 16: a single counter serialises
// 512 atomics, ~9 us per kernel); a dependent kernel polls the previous
// kernel's 16 sub-counters (2^20 tries at most, then an error counter) and
// cross-checks a word the previous kernel stored device-coherent.
//   variant 0  plain launches, no waits
//   variant 1  plain launches + waits
//   variant 2  hipExtAnyOrderLaunch + waits
//   variant 3  hipExtAnyOrderLaunch + waits + the first round issued before the wait
//   variant 4  variant 1 through hipLaunchKernelGGL
// eagerly (graph 0) and captured into a HIP graph (graph 1), seven sequences
// back to back, the last five timed.  The first phase of every sequence is
// a plain launch, and a plain-launch reset of the counters follows the last.
//
// Build: hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang
//        -packed-fp32-ops -o anyorder_launch anyorder_launch.hip
// Run:   ./anyorder_launch [workgroups = 512]
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr unsigned SPIN_LIMIT = 1u << 20;
constexpr int LPR = 4;

__device__ __forceinline__ unsigned ld_dev(const unsigned* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_dev(unsigned* p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

struct K {
    const uint8_t* buf; unsigned long long bytes;
    const unsigned* wait_cnt; unsigned wait_target;   // previous kernel's completion counter
    unsigned* done_cnt;                               // this kernel's
    const unsigned* prev_out; unsigned* out;          // cross-check words [G]
    unsigned phase; unsigned* err; unsigned* sink; int prefetch;
};

__device__ __forceinline__ void issue(const uint8_t* base, unsigned long long off, u32x4 (&v)[LPR], int lane) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)(base + off), (short)0, 4096, 0x00020000);
#pragma unroll
    for (int i = 0; i < LPR; i++) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane + 64 * i) * 16, 0, 2);
}

__global__ __launch_bounds__(256) void dep_kernel(K k) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const unsigned long long gw = blockIdx.x * 4 + wv, nw = gridDim.x * 4, rounds = k.bytes / 4096;
    u32x4 v0[LPR], v1[LPR];
    unsigned acc = 0;
    unsigned long long r = gw;
    if (k.prefetch && r < rounds) issue(k.buf, r * 4096, v0, lane);
    if (k.wait_cnt) {
        // 16 sub-counters, one per group of workgroups (b % 16), on separate lines
        if (threadIdx.x < 16) {
            const unsigned need = (k.wait_target - threadIdx.x + 15) / 16;
            unsigned it = 0;
            while (ld_dev(k.wait_cnt + threadIdx.x * 64) < need) {
                __builtin_amdgcn_s_sleep(1);
                if (++it >= SPIN_LIMIT) { atomicAdd(k.err, 1u); break; }
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            const int o = (blockIdx.x + 37) % gridDim.x;
            if (ld_dev(k.prev_out + o) != k.phase - 1) atomicAdd(k.err + 1, 1u);
        }
    }
    if (!k.prefetch && r < rounds) issue(k.buf, r * 4096, v0, lane);
    for (; r < rounds; r += nw) {
        if (r + nw < rounds) issue(k.buf, (r + nw) * 4096, v1, lane);
#pragma unroll
        for (int i = 0; i < LPR; i++) acc ^= v0[i].x ^ v0[i].y ^ v0[i].z ^ v0[i].w;
#pragma unroll
        for (int i = 0; i < LPR; i++) v0[i] = v1[i];
    }
    if (acc == 0x12345678u) k.sink[0] = acc;
    if (threadIdx.x == 0) st_dev(k.out + blockIdx.x, k.phase);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(k.done_cnt + (blockIdx.x % 16) * 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void zero_kernel(unsigned* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

int main(int argc, char** argv) {
    const int G = argc > 1 ? atoi(argv[1]) : 512;
    const unsigned long long lay[4] = {8847360ull, 5898240ull, 28016640ull, 20428800ull};
    const int NL = 36, NP = NL * 4;
    std::vector<uint8_t*> bufs(NP);
    std::vector<unsigned long long> nb(NP);
    double total = 0;
    for (int p = 0; p < NP; p++) {
        nb[p] = lay[p % 4] / 4096 * 4096; total += nb[p];
        CHECK(hipMalloc(&bufs[p], nb[p])); CHECK(hipMemset(bufs[p], p, nb[p]));
    }
    unsigned *cnt, *outs, *err, *sink;
    CHECK(hipMalloc(&cnt, (NP + 1) * 4096)); CHECK(hipMalloc(&outs, (NP + 1) * 4096 * 4)); CHECK(hipMalloc(&err, 64));
    CHECK(hipMalloc(&sink, 64));
    hipStream_t st; CHECK(hipStreamCreate(&st));
    hipEvent_t e0, e1; CHECK(hipEventCreate(&e0)); CHECK(hipEventCreate(&e1));
    auto enqueue = [&](int variant) {

        const int anyorder = variant >= 2, waits = variant >= 1, prefetch = variant == 3;
        for (int p = 0; p < NP; p++) {
            K k{bufs[p], nb[p], (waits && p > 0) ? cnt + (p - 1) * 1024 : nullptr, (unsigned)G, cnt + p * 1024,
                outs + (size_t)(p > 0 ? p - 1 : NP) * 4096, outs + (size_t)p * 4096, (unsigned)p, err, sink, prefetch};
            if (p == NP - 1) {
                // the last phase, then (after it: a barrier launch) the counters' reset
                hipExtLaunchKernelGGL(dep_kernel, dim3(G), dim3(256), 0, st, nullptr, nullptr, anyorder ? hipExtAnyOrderLaunch : 0, k);
                hipLaunchKernelGGL(zero_kernel, dim3(64), dim3(256), 0, st, cnt, (NP + 1) * 1024);
                continue;
            }
            if (variant == 4 || p == 0) hipLaunchKernelGGL(dep_kernel, dim3(G), dim3(256), 0, st, k);
            else hipExtLaunchKernelGGL(dep_kernel, dim3(G), dim3(256), 0, st, nullptr, nullptr, anyorder ? hipExtAnyOrderLaunch : 0, k);
        }
    };
    for (int graph = 0; graph < 2; graph++)
    for (int variant = 0; variant < 5; variant++) {
        float best = 1e30f;
        hipGraphExec_t ge = nullptr;
        if (graph) {
            hipGraph_t gr;
            CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
            enqueue(variant);
            CHECK(hipStreamEndCapture(st, &gr)); CHECK(hipGraphInstantiate(&ge, gr, nullptr, nullptr, 0));
        }
        CHECK(hipMemsetAsync(err, 0, 64, st));
        CHECK(hipMemsetAsync(outs, 0xff, (NP + 1) * 4096 * 4, st));
        for (int rep = 0; rep < 7; rep++) {
            if (rep == 2) CHECK(hipEventRecord(e0, st));
            if (graph) CHECK(hipGraphLaunch(ge, st)); else enqueue(variant);
        }
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(e1, st)); CHECK(hipEventSynchronize(e1));
        float ms; CHECK(hipEventElapsedTime(&ms, e0, e1));
        best = ms / 5;
        unsigned h[2]; CHECK(hipMemcpy(h, err, 8, hipMemcpyDeviceToHost));
        if (h[0] || h[1]) { printf("graph %d variant %d: timeouts %u mismatches %u\n", graph, variant, h[0], h[1]); fflush(stdout); if (h[0]) return 2; }
        printf("graph %d variant %d: %.3f ms per 144 phases = %.2f us/phase, %.0f GB/s\n",
               graph, variant, best, best * 1e3 / NP, total / (best * 1e-3) / 1e9);
        fflush(stdout);
    }
    return 0;
}
