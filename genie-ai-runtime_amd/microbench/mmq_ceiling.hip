// mmq_ceiling.hip -- register-only microbenchmark of the MMQ inner step on
// gfx950: what the matrix cores plus the per-sub-block fp32 epilogue that
// the K-quant format forces can reach, with no memory traffic at all.
//
// Each wave repeats, ITER times, the work of one 32 x 32 (rows x tokens)
// output tile for one 32-wide K sub-block, in one of these forms:
//   mode 0  int8 MFMA only (v_mfma_i32_32x32x32_i8), int32 result kept
//   mode 1  int8 MFMA + epilogue acc += S * float(C), S per element in
//           registers (2 VALU ops per element: cvt, fma)
//   mode 2  int8 MFMA + epilogue acc += ax[r] * (bx * float(C))
//           (3 VALU ops: cvt, mul, fma; S formed from row and token scales)
//   mode 3  two f16 MFMAs (v_mfma_f32_32x32x16_f16, K = 32 with exact
//           integer-valued operands) + acc += S * C (1 VALU op)
//   mode 4  f16 MFMAs only
//   mode 5  int8 MFMA 16x16x64 only (two instructions = one 32x32x32 in MACs)
//   mode 6  Q6_K-style, int8: two v_mfma_i32_32x32x16_i8 (the two 16-groups
//           of a 32-block) + C0*sc0 + C1*sc1 (mul, mad) + cvt + fma
//   mode 7  Q6_K-style, int8: (q-32)*sc split into two int8 planes, two
//           v_mfma_i32_32x32x32_i8 + (hi << 6) + lo, cvt, fma (lane scale)
//   mode 8  Q6_K-style, f16: two f16 MFMAs + fma (lane scale)
//   mode 9  f16 MFMA 16x16x32 only (four instructions = one 32x32x32 tile)
//   mode 10 Q4_K-style, f16 16x16 tiles: per 16x16 tile one v_mfma_f32_16x16x32_f16
//           (K = 32 = one sub-block, exact dots) + 4 fma with S in registers
//   mode 11 Q4_K-style, int8 with S from the matrix cores: int8 MFMA +
//           v_mfma_f32_32x32x8_f16 outer product (S) + cvt + fma
//   mode 12 Q4_K-style, f16 16x16 tiles with S = ax[row] * bx in the VALU
//           (mul + fma per element)
//   mode 13 Q4_K-style, f16 16x16 tiles with S from a v_mfma_f32_16x16x16_f16
//           outer product (K slot 0) + fma
//   mode 14 mode 1 with the int->float conversion done by the matrix core:
//           the int32 accumulator starts at the bits of 12582912.0f, so the
//           result bits are the float 12582912 + C (exact, |C| < 2^22), and
//           one subtract replaces the cvt
//   mode 15 mode 11 (S from the matrix cores) with that conversion
//           (__int_as_float of the element: hipcc 7.2 compiles
//           __builtin_bit_cast(float, v[i]) of a vector element as element 0)
//   mode 16 Q4_K-style, f16 32x32 tiles with S from the matrix cores: two
//           v_mfma_f32_32x32x16_f16 (exact dots) + v_mfma_f32_32x32x8_f16
//           outer product (S) + fma (no cvt)
//   mode 17 f16 MFMA 32x32x16 only, accumulating in place (two instructions
//           per step, no VALU: mode 4 adds every result into acc as well)
// Throughput is reported as int8-equivalent TOPS (2 * 32 * 32 * 32 per tile
// step) and as a fraction of the 5.0 POPS dense int8 peak.
//
// Build: hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang
//        -packed-fp32-ops -o mmq_ceiling mmq_ceiling.hip
// Run:   ./mmq_ceiling   (one line per mode and waves-per-SIMD setting)
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

constexpr int ITER = 4096;

template <int MODE>
__global__ __launch_bounds__(256) void ceiling_kernel(float* out, int seed) {
#pragma clang fp contract(off)
    const int l = threadIdx.x & 63;
    i32x4 a = {seed + l, seed * 3 + l, l ^ seed, l * 7};
    i32x4 b = {l * 5, seed - l, l + 11, seed ^ 0x01010101};
    h8 ah, bh;
    for (int e = 0; e < 8; e++) { ah[e] = (_Float16)((l + e) & 15); bh[e] = (_Float16)(((l * 3 + e) & 255) - 127); }
    float ax[16], S[16];
    for (int r = 0; r < 16; r++) { ax[r] = 1.0f + 0.001f * (r + l); S[r] = ax[r] * 0.5f; }
    float bx = 0.25f + 0.0001f * l;
    f32x16 acc = {};
    i32x16 iacc = {};
    for (int it = 0; it < ITER; it++) {
        if (MODE == 0) {
            iacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, iacc, 0, 0, 0);
            a.x += 1;
        } else if (MODE == 1 || MODE == 2) {
            const i32x16 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, i32x16{}, 0, 0, 0);
            a.x += 1;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                if (MODE == 1) acc[r] = __builtin_fmaf(S[r], (float)c[r], acc[r]);
                else acc[r] = __builtin_fmaf(ax[r], bx * (float)c[r], acc[r]);
            }
            bx += 1e-7f;
        } else if (MODE == 3 || MODE == 4) {
            f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, f32x16{}, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(bh, ah, c, 0, 0, 0);
            ah[0] += (_Float16)1.0f;
            if (MODE == 3) {
#pragma unroll
                for (int r = 0; r < 16; r++) acc[r] = __builtin_fmaf(S[r], c[r], acc[r]);
            } else {
                acc += c;
            }
        } else if (MODE == 6) {
            const i32x16 c0 = __builtin_amdgcn_mfma_i32_32x32x16_i8(
                __builtin_bit_cast(long, i32x2{a.x, a.y}), __builtin_bit_cast(long, i32x2{b.x, b.y}), i32x16{}, 0, 0, 0);
            const i32x16 c1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(
                __builtin_bit_cast(long, i32x2{a.z, a.w}), __builtin_bit_cast(long, i32x2{b.z, b.w}), i32x16{}, 0, 0, 0);
            a.x += 1;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int sc0 = (int)(ax[r] * 7.0f), sc1 = r - 8;   // loop-invariant row scales
                acc[r] = __builtin_fmaf((float)(c0[r] * sc0 + c1[r] * sc1), bx, acc[r]);
            }
            bx += 1e-7f;
        } else if (MODE == 7) {
            const i32x16 chi = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, i32x16{}, 0, 0, 0);
            const i32x16 clo = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, i32x16{}, 0, 0, 0);
            a.x += 1;
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = __builtin_fmaf((float)((chi[r] << 6) + clo[r]), bx, acc[r]);
            bx += 1e-7f;
        } else if (MODE == 8) {
            f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, f32x16{}, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(bh, ah, c, 0, 0, 0);
            ah[0] += (_Float16)1.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = __builtin_fmaf(c[r], bx, acc[r]);
            bx += 1e-7f;
        } else if (MODE == 10) {
            typedef float f32x4l __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const f32x4l c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(q & 1 ? bh : ah, q & 1 ? ah : bh,
                                                                        f32x4l{}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[4 * q + r] = __builtin_fmaf(S[4 * q + r], c4[r], acc[4 * q + r]);
            }
            ah[0] += (_Float16)1.0f;
        } else if (MODE == 11) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            const i32x16 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, i32x16{}, 0, 0, 0);
            const h4 as = {(_Float16)bx, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
            const h4 bs = {(_Float16)ax[it & 15], (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
            const f32x16 sm = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs, f32x16{}, 0, 0, 0);
            a.x += 1;
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = __builtin_fmaf(sm[r], (float)c[r], acc[r]);
            bx += 1e-7f;
        } else if (MODE == 12 || MODE == 13) {
            typedef float f32x4l __attribute__((ext_vector_type(4)));
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const f32x4l c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(q & 1 ? bh : ah, q & 1 ? ah : bh,
                                                                        f32x4l{}, 0, 0, 0);
                if (MODE == 12) {
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[4 * q + r] = __builtin_fmaf(ax[4 * q + r] * bx, c4[r], acc[4 * q + r]);
                } else {
                    const h4 as = {(_Float16)ax[q], (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
                    const h4 bs = {(_Float16)bx, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
                    const f32x4l s4 = __builtin_amdgcn_mfma_f32_16x16x16f16(as, bs, f32x4l{}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[4 * q + r] = __builtin_fmaf(s4[r], c4[r], acc[4 * q + r]);
                }
            }
            ah[0] += (_Float16)1.0f;
            bx += 1e-7f;
        } else if (MODE == 14 || MODE == 15) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            i32x16 magic;
#pragma unroll
            for (int r = 0; r < 16; r++) magic[r] = 0x4B400000;
            const i32x16 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, magic, 0, 0, 0);
            f32x16 sm;
            if (MODE == 15) {
                const h4 as = {(_Float16)bx, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
                const h4 bs = {(_Float16)ax[it & 15], (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
                sm = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs, f32x16{}, 0, 0, 0);
            }
            a.x += 1;
#pragma unroll
            for (int r = 0; r < 16; r++)
                acc[r] = __builtin_fmaf(MODE == 15 ? sm[r] : S[r], __int_as_float(c[r]) - 12582912.0f, acc[r]);
            bx += 1e-7f;
        } else if (MODE == 16) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, f32x16{}, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(bh, ah, c, 0, 0, 0);
            const h4 as = {(_Float16)bx, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
            const h4 bs = {(_Float16)ax[it & 15], (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
            const f32x16 sm = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs, f32x16{}, 0, 0, 0);
            ah[0] += (_Float16)1.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = __builtin_fmaf(sm[r], c[r], acc[r]);
            bx += 1e-7f;
        } else if (MODE == 17) {
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(bh, ah, acc, 0, 0, 0);
        } else if (MODE == 9) {
            typedef float f32x4l __attribute__((ext_vector_type(4)));
            f32x4l c4 = {acc[0], acc[1], acc[2], acc[3]};
            c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, c4, 0, 0, 0);
            c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bh, ah, c4, 0, 0, 0);
            c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, c4, 0, 0, 0);
            c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bh, ah, c4, 0, 0, 0);
            acc[0] = c4.x; acc[1] = c4.y; acc[2] = c4.z; acc[3] = c4.w;
            ah[0] += (_Float16)1.0f;
        } else {
            // two 16x16x64 steps cover 32x32 outputs of K = 32 ... per 16x16 tile: K = 64,
            // so one 32x32x32 tile step equals two 16x16x64 instructions in MACs
            i32x4 r4 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, i32x4{iacc[0], iacc[1], iacc[2], iacc[3]}, 0, 0, 0);
            r4 = __builtin_amdgcn_mfma_i32_16x16x64_i8(b, a, r4, 0, 0, 0);
            iacc[0] = r4.x; iacc[1] = r4.y; iacc[2] = r4.z; iacc[3] = r4.w;
            a.x += 1;
        }
    }
    float s = 0.0f;
    for (int r = 0; r < 16; r++) s += acc[r] + (float)iacc[r];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

template <int MODE>
static void run(int wps, float* buf) {
    const int blocks = 256 * wps;          // 4 waves per block; wps waves per SIMD
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    hipLaunchKernelGGL(ceiling_kernel<MODE>, dim3(blocks), dim3(256), 0, 0, buf, 1);
    (void)hipEventRecord(e0);
    const int reps = 5;
    for (int i = 0; i < reps; i++) hipLaunchKernelGGL(ceiling_kernel<MODE>, dim3(blocks), dim3(256), 0, 0, buf, 2 + i);
    (void)hipEventRecord(e1);
    (void)hipEventSynchronize(e1);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    const double ops = 2.0 * 32 * 32 * 32 * (double)ITER * blocks * 4 * reps;
    const double tops = ops / (ms * 1e-3) / 1e12;
    printf("mode %d waves/SIMD %d: %.1f us per launch, %.0f int8-equivalent TOPS = %.3f of 5000\n", MODE, wps,
           ms * 1e3 / reps, tops, tops / 5000.0);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
}

int main() {
    float* buf = nullptr;
    if (hipMalloc(&buf, (size_t)256 * 8 * 256 * sizeof(float)) != hipSuccess) return 1;
    for (int wps = 1; wps <= 4; wps *= 2) {
        run<0>(wps, buf);
        run<1>(wps, buf);
        run<2>(wps, buf);
        run<3>(wps, buf);
        run<4>(wps, buf);
        run<5>(wps, buf);
        run<6>(wps, buf);
        run<7>(wps, buf);
        run<8>(wps, buf);
        run<9>(wps, buf);
        run<10>(wps, buf);
        run<11>(wps, buf);
        run<12>(wps, buf);
        run<13>(wps, buf);
        run<14>(wps, buf);
        run<15>(wps, buf);
        run<16>(wps, buf);
        run<17>(wps, buf);
    }
    (void)hipFree(buf);
    return 0;
}
