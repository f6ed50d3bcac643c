// grid_barrier.hip -- microbenchmark: can a persistent kernel with
// grid-wide barriers beat kernel launch boundaries for a chain of dependent
// streaming phases shaped like a decode layer's GEMVs?
//
// 144 phases (36 layers x QKV 8.8 MB, O 5.9 MB, gate/up 28.0 MB, down
// 20.4 MB of distinct buffers) are streamed by 512 workgroups of 4 waves
// (4 KiB rounds of 16-byte nontemporal buffer loads, two rounds in flight
// per wave), either as one launch per phase captured in a HIP graph, or as
// ONE cooperative launch with a grid barrier after each phase:
//   mode 0  one arrival counter (device-scope atomic add, then a poll)
//   mode 1  eight group counters (workgroup b % 8), the last arrival of a
//           group adds to a top counter, everyone polls the top counter
//   mode 2  arrival flags (device-coherent stores), one gatherer per group
//           raises a group flag, everyone polls the eight group flags
// each with and without the next phase's first round issued before the
// barrier.  Every phase's output word is stored device-coherent and read
// back by another workgroup after the barrier (a mismatch counter checks
// the barrier), and every poll gives up after 2^20 tries (an error counter;
// the kernel still ends normally).  Also: the barriers alone (empty phases).
//
// Build: hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang
//        -packed-fp32-ops -o grid_barrier grid_barrier.hip
// Run:   ./grid_barrier [workgroups = 512]
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <cstring>

#define CHECK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr unsigned SPIN_LIMIT = 1u << 20;
constexpr int NG = 8;   // barrier groups

struct Phase { const uint8_t* buf; unsigned long long bytes; };
struct Args {
    const Phase* ph; int nph;
    unsigned* cnt;      // [NG * 32] group counters, then [32 * 32] top
    unsigned* flags;    // [G] arrival flags (stride 1)
    unsigned* gflags;   // [NG] group flags
    unsigned* out;      // [2][G] values for the cross-check
    unsigned* err;      // [0] spin timeouts, [1] cross-check mismatches
    unsigned* sink;
    int mode;           // 0 single counter, 1 group counters, 2 flags
    int prefetch;       // issue the next phase's first round before the barrier
};

__device__ __forceinline__ unsigned ld_dev(const unsigned* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_dev(unsigned* p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

__device__ bool spin_until_ge(const unsigned* p, unsigned target, unsigned* err) {
    for (unsigned it = 0; it < SPIN_LIMIT; it++) {
        if (ld_dev(p) >= target) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    atomicAdd(err, 1u);
    return false;
}

// all threads: barrier number `epoch` (1, 2, ...)
__device__ void grid_barrier(const Args& a, unsigned epoch) {
    const int G = gridDim.x, b = blockIdx.x, t = threadIdx.x;
    __builtin_amdgcn_s_waitcnt(0x0F70);     // vmcnt(0): this thread's stores are acknowledged
    __syncthreads();
    if (a.mode == 0) {
        if (t == 0) {
            __hip_atomic_fetch_add(a.cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            spin_until_ge(a.cnt, epoch * G, a.err);
        }
    } else if (a.mode == 1) {
        if (t == 0) {
            const int g = b % NG;
            const unsigned gsize = (G - g + NG - 1) / NG;
            const unsigned old = __hip_atomic_fetch_add(a.cnt + g * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            unsigned* top = a.cnt + NG * 32;
            if (old + 1 == epoch * gsize) __hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            spin_until_ge(top, epoch * NG, a.err);
        }
    } else {
        // flags: every workgroup stores its epoch; the first workgroup of each
        // group (b < NG) gathers its members' flags and raises the group flag
        if (t == 0) st_dev(a.flags + b, epoch);
        if (b < NG && t < 64) {
            bool ok = false;
            for (unsigned it = 0; it < SPIN_LIMIT && !ok; it++) {
                bool mine = true;
                for (int m = b + NG * t; m < G; m += NG * 64) mine = mine && ld_dev(a.flags + m) >= epoch;
                ok = __builtin_amdgcn_ballot_w64(!mine) == 0;
                if (!ok) __builtin_amdgcn_s_sleep(1);
            }
            if (!ok && t == 0) atomicAdd(a.err, 1u);
            __builtin_amdgcn_s_waitcnt(0x0F70);
            if (t == 0) st_dev(a.gflags + b, epoch);
        }
        if (t < 64) {
            bool ok = false;
            for (unsigned it = 0; it < SPIN_LIMIT && !ok; it++) {
                const bool mine = t >= NG || ld_dev(a.gflags + t) >= epoch;
                ok = __builtin_amdgcn_ballot_w64(!mine) == 0;
                if (!ok) __builtin_amdgcn_s_sleep(1);
            }
            if (!ok && t == 0) atomicAdd(a.err, 1u);
        }
    }
    __syncthreads();
}

constexpr int LPR = 4;   // 16-byte loads per lane per round (4 KiB per wave)

__device__ __forceinline__ void issue(const Phase& p, unsigned long long off, u32x4 (&v)[LPR], int lane) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)(p.buf + off), (short)0, 4096, 0x00020000);
#pragma unroll
    for (int i = 0; i < LPR; i++) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane + 64 * i) * 16, 0, 2);
}

// this wave's rounds of phase p: 4 KiB rounds dealt to the grid's waves
__device__ unsigned stream_phase(const Phase& p, int gw, int nw, int lane, u32x4 (&pre)[LPR], bool have_pre) {
    unsigned acc = 0;
    const unsigned long long rounds = p.bytes / 4096;
    u32x4 v0[LPR], v1[LPR];
    unsigned long long r = gw;
    if (have_pre) {
#pragma unroll
        for (int i = 0; i < LPR; i++) v0[i] = pre[i];
    } else if (r < rounds) issue(p, r * 4096, v0, lane);
    for (; r < rounds; r += nw) {
        if (r + nw < rounds) issue(p, (r + nw) * 4096, v1, lane);
#pragma unroll
        for (int i = 0; i < LPR; i++) acc ^= v0[i].x ^ v0[i].y ^ v0[i].z ^ v0[i].w;
#pragma unroll
        for (int i = 0; i < LPR; i++) v0[i] = v1[i];
    }
    return acc;
}

__global__ __launch_bounds__(256) void persist_kernel(Args a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int gw = blockIdx.x * 4 + wv, nw = gridDim.x * 4;
    unsigned acc = 0;
    u32x4 pre[LPR];
    bool have = false;
    for (int p = 0; p < a.nph; p++) {
        acc ^= stream_phase(a.ph[p], gw, nw, lane, pre, have);
        have = false;
        // output of this phase, device-coherent store
        if (threadIdx.x == 0) st_dev(a.out + (p & 1) * gridDim.x + blockIdx.x, (unsigned)(p * 7919 + blockIdx.x));
        if (a.prefetch && p + 1 < a.nph && (unsigned long long)gw < a.ph[p + 1].bytes / 4096) {
            issue(a.ph[p + 1], (unsigned long long)gw * 4096, pre, lane);
            have = true;
        }
        if (ld_dev(a.err) != 0) break;
        grid_barrier(a, (unsigned)(p + 1));
        // cross-check: another workgroup's output of this phase is visible
        if (threadIdx.x == 0) {
            const int o = (blockIdx.x + 37) % gridDim.x;
            if (ld_dev(a.out + (p & 1) * gridDim.x + o) != (unsigned)(p * 7919 + o)) atomicAdd(a.err + 1, 1u);
        }
    }
    if (acc == 0x12345678u) a.sink[0] = acc;
}

__global__ __launch_bounds__(256) void phase_kernel(Phase p, unsigned* sink) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    u32x4 pre[LPR];
    unsigned acc = stream_phase(p, blockIdx.x * 4 + wv, gridDim.x * 4, lane, pre, false);
    if (acc == 0x12345678u) sink[0] = acc;
}

int main(int argc, char** argv) {
    const int G = argc > 1 ? atoi(argv[1]) : 512;
    hipDeviceProp_t prop; CHECK(hipGetDeviceProperties(&prop, 0));
    int per_cu = 0;
    CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, persist_kernel, 256, 0));
    printf("CUs %d, persist blocks per CU %d, grid %d, coop %d\n", prop.multiProcessorCount, per_cu, G, prop.cooperativeLaunch);
    if (per_cu * prop.multiProcessorCount < G) { printf("grid does not fit\n"); return 1; }
    // a decode layer's GEMV bytes (rounded to 4 KiB): QKV, O, gate/up, down
    const unsigned long long lay[4] = {8847360ull, 5898240ull, 28016640ull, 20428800ull};
    const int NL = 36, NP = NL * 4;
    std::vector<Phase> ph(NP);
    std::vector<uint8_t*> bufs;
    for (int l = 0; l < NL; l++)
        for (int j = 0; j < 4; j++) {
            uint8_t* b; const unsigned long long n = lay[j] / 4096 * 4096;
            CHECK(hipMalloc(&b, n)); CHECK(hipMemset(b, l + j, n));
            bufs.push_back(b); ph[l * 4 + j] = Phase{b, n};
        }
    Phase* dph; CHECK(hipMalloc(&dph, sizeof(Phase) * NP)); CHECK(hipMemcpy(dph, ph.data(), sizeof(Phase) * NP, hipMemcpyHostToDevice));
    unsigned *cnt, *flags, *gflags, *out, *err, *sink;
    CHECK(hipMalloc(&cnt, 4096 * 4)); CHECK(hipMalloc(&flags, 4096 * 4)); CHECK(hipMalloc(&gflags, 64 * 4));
    CHECK(hipMalloc(&out, 2 * 4096 * 4)); CHECK(hipMalloc(&err, 64)); CHECK(hipMalloc(&sink, 64));
    hipStream_t st; CHECK(hipStreamCreate(&st));
    hipEvent_t e0, e1; CHECK(hipEventCreate(&e0)); CHECK(hipEventCreate(&e1));
    double total_bytes = 0; for (auto& p : ph) total_bytes += p.bytes;

    // (A) one launch per phase, captured in a graph
    hipGraph_t gr; hipGraphExec_t ge;
    CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (int p = 0; p < NP; p++) hipLaunchKernelGGL(phase_kernel, dim3(G), dim3(256), 0, st, ph[p], sink);
    CHECK(hipStreamEndCapture(st, &gr)); CHECK(hipGraphInstantiate(&ge, gr, nullptr, nullptr, 0));
    for (int w = 0; w < 3; w++) CHECK(hipGraphLaunch(ge, st));
    CHECK(hipEventRecord(e0, st));
    for (int w = 0; w < 5; w++) CHECK(hipGraphLaunch(ge, st));
    CHECK(hipEventRecord(e1, st)); CHECK(hipEventSynchronize(e1));
    float ms; CHECK(hipEventElapsedTime(&ms, e0, e1)); ms /= 5;
    printf("launches: %.3f ms per 144 phases = %.2f us/phase, %.0f GB/s\n", ms, ms * 1e3 / NP, total_bytes / (ms * 1e-3) / 1e9);
    fflush(stdout);

    for (int mode = 0; mode < 3; mode++)
        for (int pf = 0; pf < 2; pf++) {
            for (int nph : {NP, 1}) {
                CHECK(hipMemset(cnt, 0, 4096 * 4)); CHECK(hipMemset(flags, 0, 4096 * 4)); CHECK(hipMemset(gflags, 0, 64 * 4));
                CHECK(hipMemset(err, 0, 64)); CHECK(hipMemset(out, 0xff, 2 * 4096 * 4));
                CHECK(hipDeviceSynchronize());
                Args a{dph, nph, cnt, flags, gflags, out, err, sink, mode, pf};
                void* kargs[] = {&a};
                CHECK(hipEventRecord(e0, st));
                CHECK(hipLaunchCooperativeKernel((void*)persist_kernel, dim3(G), dim3(256), kargs, 0, st));
                CHECK(hipEventRecord(e1, st)); CHECK(hipEventSynchronize(e1));
                CHECK(hipEventElapsedTime(&ms, e0, e1));
                unsigned herr[2]; CHECK(hipMemcpy(herr, err, 8, hipMemcpyDeviceToHost));
                if (nph == NP) {
                    double by = total_bytes;
                    printf("persist mode %d prefetch %d: %.3f ms = %.2f us/phase, %.0f GB/s, timeouts %u mismatches %u\n",
                           mode, pf, ms, ms * 1e3 / NP, by / (ms * 1e-3) / 1e9, herr[0], herr[1]);
                }
                fflush(stdout);
                if (herr[0]) { printf("spin timeout: stopping\n"); return 2; }
            }
        }
    // pure barrier cost: phases of zero bytes
    std::vector<Phase> z(NP, Phase{bufs[0], 0});
    CHECK(hipMemcpy(dph, z.data(), sizeof(Phase) * NP, hipMemcpyHostToDevice));
    for (int mode = 0; mode < 3; mode++) {
        CHECK(hipMemset(cnt, 0, 4096 * 4)); CHECK(hipMemset(flags, 0, 4096 * 4)); CHECK(hipMemset(gflags, 0, 64 * 4));
        CHECK(hipMemset(err, 0, 64)); CHECK(hipDeviceSynchronize());
        Args a{dph, NP, cnt, flags, gflags, out, err, sink, mode, 0};
        void* kargs[] = {&a};
        CHECK(hipEventRecord(e0, st));
        CHECK(hipLaunchCooperativeKernel((void*)persist_kernel, dim3(G), dim3(256), kargs, 0, st));
        CHECK(hipEventRecord(e1, st)); CHECK(hipEventSynchronize(e1));
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        unsigned herr[2]; CHECK(hipMemcpy(herr, err, 8, hipMemcpyDeviceToHost));
        printf("empty phases mode %d: %.2f us per barrier, timeouts %u mismatches %u\n", mode, ms * 1e3 / NP, herr[0], herr[1]);
        fflush(stdout);
        if (herr[0]) return 2;
    }
    return 0;
}
