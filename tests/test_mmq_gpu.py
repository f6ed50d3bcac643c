"""GPU parity of the prefill path: MMQ activation quantiser (bit-exact), the
exact sub-block dots the MMQ kernels form on the matrix cores (bit-exact
against the reference's int32 dots) and the fp32 /
fp16 GEMM outputs (rel_inf <= 1e-3 against the CPU oracle; BASELINE
config 3 shapes are checked on a sampled row subset at full token count)."""
import numpy as np
import pytest
import torch

import jllm
import oracle
import synth
from gpu_util import f16_to_f64, from_dev, print_case, rel_inf, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _npad(n):
    return (n + 63) // 64 * 64


def _quantize_dev(x, N, K, Npad, ds4, dev):
    q8 = torch.zeros((K // 128) * Npad * 144, dtype=torch.uint8, device=dev)
    jllm.call("jllm_hip_quantize_mmq_q8_1", to_dev(x), q8, N, K, Npad, 1 if ds4 else 0)
    return q8


@pytest.mark.parametrize("ds4", [True, False])
@pytest.mark.parametrize("N,K", [(1, 256), (5, 512), (64, 2560), (100, 2560), (130, 9728)])
def test_quantize_mmq_bit_exact(dev, ds4, N, K):
    print_case("quantize_mmq", ds4, N, K)
    x = synth.x_f16(synth.rng(N * 7 + K), (N, K))
    x[0, :32] = 0                                        # an all-zero block
    Npad = _npad(N)
    got = from_dev(_quantize_dev(x, N, K, Npad, ds4, dev))
    want = oracle.quantize_mmq(x, N, K, Npad, ds4)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("ds4", [True, False])
@pytest.mark.parametrize("N,K", [(1, 256), (70, 512), (130, 2560)])
def test_kernel_layout_quantizer_matches_reference_layout(dev, ds4, N, K):
    """The production quantiser (fp16 codes, packed scale words) holds the
    same codes, d and sum bits as the reference-layout quantiser (which is
    bit-exact against the oracle)."""
    print_case("quantize_mmq_f16", ds4, N, K)
    x = synth.x_f16(synth.rng(N + K + ds4), (N, K))
    x[0, 32:64] = 0
    Npad = _npad(N)
    codes = torch.zeros(K * Npad, dtype=torch.int16, device=dev)
    scl = torch.zeros(K // 32 * Npad, dtype=torch.int32, device=dev)
    jllm.call("jllm_hip_quantize_mmq_f16", to_dev(x), codes, scl, N, K, Npad, 1 if ds4 else 0)
    c = f16_to_f64(from_dev(codes, np.uint16)).reshape(K // 256, Npad, 256)
    sw = from_dev(scl).view(np.uint32).reshape(K // 32, Npad)
    ref = oracle.quantize_mmq(x, N, K, Npad, ds4).reshape(K // 128, Npad, 144)
    rq = ref[:, :, 16:].view(np.int8).astype(np.float64)           # [K/128][Npad][128]
    want_c = rq.reshape(K // 256, 2, Npad, 128).transpose(0, 2, 1, 3).reshape(K // 256, Npad, 256)
    assert np.array_equal(c, want_c)
    rs = ref[:, :, 0:16].copy().view(np.uint32)                    # [K/128][Npad][4]
    want_s = rs.transpose(0, 2, 1).reshape(K // 32, Npad)
    assert np.array_equal(sw, want_s)


@pytest.mark.parametrize("N,K", [(64, 256), (70, 2560), (1, 512)])
def test_quantize_mmq_i8_layout_bit_exact(dev, N, K):
    """The Q4_K kernel's int8 code layout [K/256][Npad][256] holds the
    reference quantiser's codes, and the same DS4 scale words."""
    print_case("quantize_mmq_i8", N, K)
    x = synth.x_f16(synth.rng(N + K + 7), (N, K))
    x[0, 32:64] = 0
    Npad = _npad(N)
    codes = torch.zeros(K * Npad, dtype=torch.int8, device=dev)
    scl = torch.zeros(K // 32 * Npad, dtype=torch.int32, device=dev)
    jllm.call("jllm_hip_quantize_mmq_i8", to_dev(x), codes, scl, N, K, Npad, 1)
    c = from_dev(codes).reshape(K // 256, Npad, 256)
    sw = from_dev(scl).view(np.uint32).reshape(K // 32, Npad)
    ref = oracle.quantize_mmq(x, N, K, Npad, True).reshape(K // 128, Npad, 144)
    rq = ref[:, :, 16:].view(np.int8)
    assert np.array_equal(c, rq.reshape(K // 256, 2, Npad, 128).transpose(0, 2, 1, 3).reshape(K // 256, Npad, 256))
    assert np.array_equal(sw, ref[:, :, 0:16].copy().view(np.uint32).transpose(0, 2, 1).reshape(K // 32, Npad))


@pytest.mark.parametrize("t", [12, 14])
@pytest.mark.parametrize("M,N,K", [(128, 64, 256), (200, 70, 512), (33, 5, 2560), (64, 129, 768)])
def test_mmq_int32_dots_bit_exact(dev, t, M, N, K):
    print_case("mmq_subdots", t, M, N, K)
    g = synth.rng(M + N + K + t)
    W = synth.weights(g, t, M, K)
    x = synth.x_f16(g, (N, K))
    Npad = _npad(N)
    G = 32 if t == 12 else 16
    out = torch.zeros(N * M * (K // G), dtype=torch.int32, device=dev)
    jllm.call("jllm_hip_mmq_subdots", out, to_dev(W), t, to_dev(x), M, N, K)
    got = from_dev(out).reshape(N, M, K // G)
    want = oracle.mmq_subdots(W, t, oracle.quantize_mmq(x, N, K, Npad, t == 12), M, N, K, Npad)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("t", [12, 14])
@pytest.mark.parametrize("M,N,K", [(300, 70, 2560), (128, 64, 1024), (97, 130, 512), (256, 2, 256),
                                   (70, 66, 28672)])      # the largest K: 112 super-blocks, many split ranges
def test_mmq_f32_and_f16(dev, t, M, N, K):
    print_case("mmq", t, M, N, K)
    g = synth.rng(1000 + M + N + K + t)
    W = synth.weights(g, t, M, K)
    x = synth.x_f16(g, (N, K))
    Wd, xd = to_dev(W), to_dev(x)
    y32 = torch.empty(N * M, dtype=torch.float32, device=dev)
    jllm.call("jllm_hip_gemm_quant_batched_f32", y32, Wd, t, xd, M, N, K)
    want = oracle.mmq(W, t, oracle.quantize_mmq(x, N, K, _npad(N), t == 12), M, N, K, _npad(N))
    assert rel_inf(from_dev(y32).reshape(N, M), want) <= TOL
    y16 = torch.empty(N * M, dtype=torch.int16, device=dev)
    jllm.call("jllm_hip_gemm_quant_batched", y16, Wd, t, xd, M, N, K)
    got = f16_to_f64(from_dev(y16, np.uint16)).reshape(N, M)
    err = np.abs(got - want)
    assert np.all(err <= TOL * np.abs(want).max() + np.abs(want) * 2 ** -10)


@pytest.mark.parametrize("t,M,K", [(12, 9728, 2560), (14, 2560, 9728)])
@pytest.mark.parametrize("N", [64, 512, 1261])
def test_mmq_baseline_shapes_sampled(dev, t, M, K, N):
    """full GEMM on the GPU, oracle on 48 sampled rows."""
    print_case("mmq_full", t, M, N, K)
    g = synth.rng(2000 + N + t)
    W = synth.weights(g, t, M, K)
    x = synth.x_f16(g, (N, K))
    y32 = torch.empty(N * M, dtype=torch.float32, device=dev)
    jllm.call("jllm_hip_gemm_quant_batched_f32", y32, to_dev(W), t, to_dev(x), M, N, K)
    got = from_dev(y32).reshape(N, M)
    rows = np.sort(g.choice(M, 48, replace=False))
    rows[-1] = M - 1
    q8 = oracle.quantize_mmq(x, N, K, _npad(N), t == 12)
    want = oracle.mmq(W[rows], t, q8, len(rows), N, K, _npad(N))
    assert rel_inf(got[:, rows], want) <= TOL


def test_gemm_n1_routes_to_gemv(dev):
    K, M = 2560, 512
    g = synth.rng(3)
    W = synth.q4k(g, M, K)
    x = synth.x_f16(g, K)
    y = torch.empty(M, dtype=torch.int16, device=dev)
    jllm.call("jllm_hip_gemm_quant_batched", y, to_dev(W), 12, to_dev(x), M, 1, K)
    want = oracle.mmvq(W, 12, oracle.quantize_q8_1(x, K), M, K)
    got = f16_to_f64(from_dev(y, np.uint16))
    assert np.all(np.abs(got - want) <= TOL * np.abs(want).max() + np.abs(want) * 2 ** -10)


# ---- Q5_K batched GEMM (fp16 activation, float-dequant arithmetic) --------------

def _oracle_q5_batched(W, x, M, N, K):
    """gemm_quant_batched_q5k_kernel (gemv_q4.cu:1703-1762) per token is the
    row arithmetic of gemv_quant_cpu's Q5_K branch."""
    return np.stack([oracle.gemv_quant_cpu(W, 13, x[t], M, K) for t in range(N)])


@pytest.mark.parametrize("M,N,K", [(300, 70, 2560), (128, 64, 1024), (97, 130, 512), (256, 2, 256), (1, 3, 256),
                                   (130, 65, 4096), (40, 3, 28672)])
def test_q5k_batched_f32_and_f16(dev, M, N, K):
    print_case("q5k_gemm", M, N, K)
    g = synth.rng(3000 + M + N + K)
    W = synth.q5k(g, M, K)
    x = synth.x_f16(g, (N, K))
    Wd, xd = to_dev(W), to_dev(x)
    want = _oracle_q5_batched(W, x, M, N, K)
    y32 = torch.empty(N * M, dtype=torch.float32, device=dev)
    jllm.call("jllm_hip_gemm_quant_batched_f32", y32, Wd, 13, xd, M, N, K)
    got = from_dev(y32).reshape(N, M)
    assert rel_inf(got, want) <= TOL
    # every product is exact and the sums are fp32: far inside the bar
    assert rel_inf(got, want) <= 2e-5
    y16 = torch.empty(N * M, dtype=torch.int16, device=dev)
    jllm.call("jllm_hip_gemm_quant_batched", y16, Wd, 13, xd, M, N, K)
    got16 = f16_to_f64(from_dev(y16, np.uint16)).reshape(N, M)
    assert np.all(np.abs(got16 - want) <= TOL * np.abs(want).max() + np.abs(want) * 2 ** -10)


def test_q5k_batched_column_probe(dev):
    """Token t = e_k(t): row t of y is column k(t) of the dequantised matrix,
    which pins the K order of the matrix-core mapping and the min term."""
    M, K = 160, 512
    W = synth.q5k(synth.rng(3100), M, K)
    ks = np.array([0, 1, 7, 8, 15, 16, 31, 32, 33, 47, 48, 63, 64, 100, 127, 128, 200, 255, 256, 300, 383, 511])
    N = len(ks)
    x = np.zeros((N, K), np.uint16)
    x[np.arange(N), ks] = 0x3C00
    y = torch.empty(N * M, dtype=torch.float32, device=dev)
    print_case("q5k_gemm_probe", M, N, K)
    jllm.call("jllm_hip_gemm_quant_batched_f32", y, to_dev(W), 13, to_dev(x), M, N, K)
    got = from_dev(y).reshape(N, M)
    Wd = oracle.dequant(W, 13, M, K)
    assert np.allclose(got, Wd[:, ks].T, rtol=2e-6, atol=1e-9)


@pytest.mark.parametrize("N", [512, 1261])
def test_q5k_batched_baseline_shape_sampled(dev, N):
    M, K = 9728, 2560
    print_case("q5k_gemm_full", M, N, K)
    g = synth.rng(3200 + N)
    W = synth.q5k(g, M, K)
    x = synth.x_f16(g, (N, K))
    y32 = torch.empty(N * M, dtype=torch.float32, device=dev)
    jllm.call("jllm_hip_gemm_quant_batched_f32", y32, to_dev(W), 13, to_dev(x), M, N, K)
    got = from_dev(y32).reshape(N, M)
    rows = np.sort(g.choice(M, 24, replace=False))
    rows[-1] = M - 1
    want = _oracle_q5_batched(np.ascontiguousarray(W[rows]), x, len(rows), N, K)
    assert rel_inf(got[:, rows], want) <= 2e-5


def test_q5k_has_no_subdots(dev):
    x = to_dev(synth.x_f16(synth.rng(1), (2, 256)))
    W = to_dev(synth.q5k(synth.rng(2), 4, 256))
    out = torch.zeros(64, dtype=torch.int32, device=dev)
    assert jllm.lib().jllm_hip_mmq_subdots(jllm._ptr(out), jllm._ptr(W), 13, jllm._ptr(x), 4, 2, 256, None) != 0


# ---- the reference's own accuracy bar against the true fp16 x K-quant product -----

def _reference_style_weights(g, t, M, K):
    """Block distributions of the reference's MMQ tests: Q4_K d ~ U(0.005, 0.02),
    dmin ~ U(0.001, 0.004), random scale / qs bytes (test_mmq_q4k_int8.cu:434-445);
    Q6_K sc ~ U{-32..32}, d ~ U(0.001, 0.01) (test_mmq_q6k_int8.cu:257-266)."""
    nb = K // 256
    if t == 12:
        b = np.frombuffer(g.bytes(M * nb * 144), np.uint8).reshape(M, nb, 144).copy()
        b[:, :, 0:2] = g.uniform(0.005, 0.02, (M, nb, 1)).astype(np.float16).view(np.uint8)
        b[:, :, 2:4] = g.uniform(0.001, 0.004, (M, nb, 1)).astype(np.float16).view(np.uint8)
        return b.reshape(M, -1)
    b = np.frombuffer(g.bytes(M * nb * 210), np.uint8).reshape(M, nb, 210).copy()
    b[:, :, 192:208] = g.integers(-32, 33, (M, nb, 16)).astype(np.int8).view(np.uint8)
    b[:, :, 208:210] = g.uniform(0.001, 0.01, (M, nb, 1)).astype(np.float16).view(np.uint8)
    return b.reshape(M, -1)


@pytest.mark.parametrize("t,M,N,K", [(12, 256, 64, 2560), (14, 256, 64, 2560), (12, 512, 130, 4096)])
def test_mmq_vs_true_fp16_product(dev, t, M, N, K):
    """The q8_1 quantisation error against the unquantised product, with the
    reference's bar for its MMQ port (test_mmq_q4k_llama.cu:477-482): relRMS
    < 0.01 and no element with rel > 0.02 and abs > 0.05 sigma; x ~ U(-1, 1)
    (test_mmq_q4k_int8.cu:496-497)."""
    import np_ref
    print_case("mmq_vs_fp16", t, M, N, K)
    g = synth.rng(0xC0FFEE + t)
    W = _reference_style_weights(g, t, M, K)
    x = g.uniform(-1.0, 1.0, (N, K)).astype(np.float16).view(np.uint16)
    y = torch.empty(N * M, dtype=torch.float32, device=dev)
    jllm.call("jllm_hip_gemm_quant_batched_f32", y, to_dev(W), t, to_dev(x), M, N, K)
    got = from_dev(y).reshape(N, M).astype(np.float64)
    ref = np_ref.f16(x).reshape(N, K) @ np_ref.dequant(W, t, M, K).T
    err = got - ref
    sigma = ref.std()
    rel_rms = np.sqrt((err ** 2).mean()) / np.sqrt((ref ** 2).mean())
    assert rel_rms < 0.01, rel_rms
    bad = (np.abs(err) > 0.02 * np.abs(ref)) & (np.abs(err) > 0.05 * sigma)
    assert not bad.any(), int(bad.sum())


def _multi(outs, Ws, types, Ms, x, N, K):
    import ctypes
    n = len(Ws)
    ya = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    wa = (ctypes.c_void_p * n)(*[w.data_ptr() for w in Ws])
    ta = (ctypes.c_int * n)(*types)
    ma = (ctypes.c_int * n)(*Ms)
    jllm.call("jllm_hip_gemm_quant_batched_multi", ctypes.cast(ya, ctypes.c_void_p), ctypes.cast(wa, ctypes.c_void_p),
              ctypes.cast(ta, ctypes.c_void_p), ctypes.cast(ma, ctypes.c_void_p), n, x, N, K)


@pytest.mark.parametrize("Ms,types,N", [
    ((9728, 9728), (12, 12), 512),          # gate/up of a 512-token chunk: one launch, 1216 tiles
    ((4096, 1024, 1024), (12, 12, 12), 512),  # Q/K/V: one launch, 384 tiles
    ((4096, 1024, 1024), (12, 12, 12), 40),   # too few tiles: one launch per matrix (split-K)
    ((2560, 2560), (12, 14), 512),          # mixed types: one launch per matrix
])
def test_gemm_multi_matches_separate_products(dev, Ms, types, N):
    """The multi-matrix product equals each matrix's own gemm_quant_batched
    bit for bit where neither splits K; where the single launch splits K, the
    two agree within the fp32 parity bar (and the fp32 single launch is pinned
    against the oracle by the tests above)."""
    print_case("gemm_multi", Ms, types, N)
    K = 2560
    g = synth.rng(sum(Ms) + N)
    Ws = [to_dev(synth.weights(g, t, M, K)) for t, M in zip(types, Ms)]
    x = to_dev(synth.x_f16(g, (N, K)))
    outs = [torch.full((N * M,), 0x7C00, dtype=torch.int16, device=dev) for M in Ms]
    _multi(outs, Ws, types, Ms, x, N, K)
    for o, W, t, M in zip(outs, Ws, types, Ms):
        single = torch.empty(N * M, dtype=torch.int16, device=dev)
        jllm.call("jllm_hip_gemm_quant_batched", single, W, t, x, M, N, K)
        ref32 = torch.empty(N * M, dtype=torch.float32, device=dev)
        jllm.call("jllm_hip_gemm_quant_batched_f32", ref32, W, t, x, M, N, K)
        torch.cuda.synchronize()
        got = f16_to_f64(from_dev(o, np.uint16))
        sgl = f16_to_f64(from_dev(single, np.uint16))
        tiles = lambda m: ((m + 127) // 128) * _npad(N) // 64
        one_launch = all(tt == 12 for tt in types) and sum(tiles(m) for m in Ms) >= 384
        if not one_launch or tiles(M) >= 384:       # same arithmetic as the single launch
            assert np.array_equal(got, sgl)
        assert rel_inf(got, from_dev(ref32).astype(np.float64)) <= TOL
