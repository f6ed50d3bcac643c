"""GPU parity of the GEMV family (through the C ABI) against the CPU oracle.

Tolerance: rel_inf = max|y - y_oracle| / max|y_oracle| <= 1e-3 for fp32
outputs; fp16 outputs are compared after the oracle result is rounded to
fp16 with the same bound plus one fp16 ulp.  The activation quantiser is
compared bit-exactly.
"""
import numpy as np
import pytest
import torch

import jllm
import oracle
import synth
from gpu_util import empty_f16, empty_f32, f16_to_f64, from_dev, print_case, rel_inf, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-3

SHAPES = [  # (rows, K) -- BASELINE config 1/2 shapes, trimmed rows, plus odd row counts; K above
    # 10240 takes the second activation-staging pass, 28672 is the largest K accepted
    (9728, 2560), (4096, 2560), (1024, 2560), (2560, 4096), (2560, 9728), (37, 256), (1, 512), (203, 1280),
    (77, 12288), (40, 28672),
]


def _case(t, rows, K, seed):
    g = synth.rng(seed)
    return synth.weights(g, t, rows, K), synth.x_f16(g, K)


def _close_f16(got_bits, want_f32):
    got = f16_to_f64(got_bits)
    want = np.asarray(want_f32, np.float64)
    err = np.abs(got - want)
    bound = TOL * np.abs(want).max() + np.abs(want) * 2 ** -10
    return bool(np.all(err <= bound)), float(err.max())


@pytest.mark.parametrize("t", [12, 14])
def test_quantize_q8_1_bit_exact(dev, t):
    for K in (256, 2560, 9728):
        print_case("q8_1", K)
        x = synth.x_f16(synth.rng(K), K)
        x[:32] = 0                                  # an all-zero block
        xd = to_dev(x)
        y = torch.zeros(K // 32 * 36, dtype=torch.uint8, device=dev)
        jllm.quantize_q8_1(xd, y, K)
        assert np.array_equal(from_dev(y), oracle.quantize_q8_1(x, K))


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("rows,K", SHAPES)
def test_gemv_dequant_f32_vs_host_scalar(dev, t, rows, K):
    """float-dequant fp32 GEMV vs gemv_quant_cpu (the reference host path)."""
    print_case("dequant_f32", t, rows, K)
    W, x = _case(t, rows, K, 100 + rows)
    y = empty_f32(rows)
    jllm.gemv_quant_dequant_f32(y, to_dev(W), t, to_dev(x), rows, K)
    want = oracle.gemv_quant_cpu(W, t, x, rows, K)
    assert rel_inf(from_dev(y), want) <= TOL


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("rows,K", SHAPES)
def test_gemv_f32(dev, t, rows, K):
    """gemv_quant_f32: Q4_K via MMVQ (oracle mmvq), Q5_K / Q6_K via float dequant."""
    print_case("gemv_f32", t, rows, K)
    W, x = _case(t, rows, K, 200 + rows)
    y = empty_f32(rows)
    jllm.gemv_quant_f32(y, to_dev(W), t, to_dev(x), rows, K)
    if t == 12:
        want = oracle.mmvq(W, t, oracle.quantize_q8_1(x, K), rows, K)
    else:
        want = oracle.gemv_quant_cpu(W, t, x, rows, K)
    assert rel_inf(from_dev(y), want) <= TOL


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("rows,K", SHAPES)
def test_gemv_half_mmvq(dev, t, rows, K):
    """gemv_quant: MMVQ for Q4_K / Q6_K, float dequant for Q5_K (gemv_q4.cu:1263-1290)."""
    print_case("gemv_half", t, rows, K)
    W, x = _case(t, rows, K, 300 + rows)
    y = empty_f16(rows)
    jllm.gemv_quant(y, to_dev(W), t, to_dev(x), rows, K)
    if t == 13:
        want = oracle.gemv_quant_cpu(W, t, x, rows, K)
    else:
        want = oracle.mmvq(W, t, oracle.quantize_q8_1(x, K), rows, K)
    ok, err = _close_f16(from_dev(y, np.uint16), want)
    assert ok, err


@pytest.mark.parametrize("t", [12, 13, 14])
def test_gemv_add(dev, t):
    rows, K = 2560, 9728 if t == 14 else 4096
    print_case("gemv_add", t, rows, K)
    W, x = _case(t, rows, K, 400)
    res = synth.x_f16(synth.rng(401), rows)
    y = empty_f16(rows)
    jllm.gemv_quant_add(y, to_dev(W), t, to_dev(x), to_dev(res), rows, K)
    proj = oracle.gemv_quant_cpu(W, t, x, rows, K).astype(np.float16).astype(np.float32)
    want = proj + f16_to_f64(res).astype(np.float32)
    ok, err = _close_f16(from_dev(y, np.uint16), want)
    assert ok, err


@pytest.mark.parametrize("t,rows,K", [(12, 1, 256), (12, 7, 768), (12, 100, 1024), (14, 333, 2560),
                                      (13, 1000, 4096), (12, 2560, 9728), (14, 4096, 1280), (12, 5000, 2560)])
def test_gemv_add_shapes(dev, t, rows, K):
    """Residual GEMV at ragged shapes: one row, rows that do not fill a
    workgroup's waves (rounds dealt round-robin), both workgroup sizes (the
    Q4_K 2560 x 9728 down takes 512 threads, the larger Q6_K ones 256)."""
    print_case("gemv_add_shape", t, rows, K)
    W, x = _case(t, rows, K, 410 + rows)
    res = synth.x_f16(synth.rng(411 + rows), rows)
    y = empty_f16(rows)
    jllm.gemv_quant_add(y, to_dev(W), t, to_dev(x), to_dev(res), rows, K)
    proj = oracle.gemv_quant_cpu(W, t, x, rows, K).astype(np.float16).astype(np.float32)
    want = proj + f16_to_f64(res).astype(np.float32)
    ok, err = _close_f16(from_dev(y, np.uint16), want)
    assert ok, err


def test_gemv_pair_and_triple(dev):
    K = 2560
    g = synth.rng(500)
    x = synth.x_f16(g, K)
    Wg, Wu = synth.q4k(g, 9728, K), synth.q4k(g, 9728, K)
    xq = oracle.quantize_q8_1(x, K)
    y0, y1 = empty_f16(9728), empty_f16(9728)
    print_case("pair q4k/q4k")
    jllm.gemv_quant_pair(y0, to_dev(Wg), 12, 9728, y1, to_dev(Wu), 12, 9728, to_dev(x), K)
    for y, W in ((y0, Wg), (y1, Wu)):
        ok, err = _close_f16(from_dev(y, np.uint16), oracle.mmvq(W, 12, xq, 9728, K))
        assert ok, err
    # mixed pair -> float dequant
    Wm = synth.q6k(g, 1000, K)
    print_case("pair q4k/q6k")
    y2 = empty_f16(1000)
    jllm.gemv_quant_pair(y0, to_dev(Wg), 12, 9728, y2, to_dev(Wm), 14, 1000, to_dev(x), K)
    ok, err = _close_f16(from_dev(y2, np.uint16), oracle.gemv_quant_cpu(Wm, 14, x, 1000, K))
    assert ok, err
    # QKV triple, Q4_K / Q4_K / Q6_K (Qwen3 Q4_K_M layout)
    Wq, Wk, Wv = synth.q4k(g, 4096, K), synth.q4k(g, 1024, K), synth.q6k(g, 1024, K)
    yq, yk, yv = empty_f16(4096), empty_f16(1024), empty_f16(1024)
    print_case("triple q4k/q4k/q6k")
    jllm.gemv_quant_triple(yq, to_dev(Wq), 12, 4096, yk, to_dev(Wk), 12, 1024, yv, to_dev(Wv), 14, 1024, to_dev(x), K)
    for y, W, t, M in ((yq, Wq, 12, 4096), (yk, Wk, 12, 1024), (yv, Wv, 14, 1024)):
        ok, err = _close_f16(from_dev(y, np.uint16), oracle.mmvq(W, t, xq, M, K))
        assert ok, (t, M, err)


def test_q5k_in_fused_launches(dev):
    """Launches holding Q5_K rows run in float mode for every segment
    (gemv_q4.cu:1391-1441, :1527-1559); Q4_K + Q5_K segments in one call are
    split over two launches of the same kernel family."""
    K = 2560
    g = synth.rng(520)
    x = synth.x_f16(g, K)
    Wa, Wb, Wc = synth.q5k(g, 4096, K), synth.q4k(g, 1024, K), synth.q6k(g, 1024, K)
    ys = [empty_f16(4096), empty_f16(1024), empty_f16(1024)]
    print_case("triple q5k/q4k/q6k")
    jllm.gemv_quant_triple(ys[0], to_dev(Wa), 13, 4096, ys[1], to_dev(Wb), 12, 1024, ys[2], to_dev(Wc), 14, 1024,
                           to_dev(x), K)
    for y, W, t, M in zip(ys, (Wa, Wb, Wc), (13, 12, 14), (4096, 1024, 1024)):
        ok, err = _close_f16(from_dev(y, np.uint16), oracle.gemv_quant_cpu(W, t, x, M, K))
        assert ok, (t, M, err)
    print_case("pair q5k/q5k")
    Wg, Wu = synth.q5k(g, 9728, K), synth.q5k(g, 9728, K)
    y0, y1 = empty_f16(9728), empty_f16(9728)
    jllm.gemv_quant_pair(y0, to_dev(Wg), 13, 9728, y1, to_dev(Wu), 13, 9728, to_dev(x), K)
    for y, W in ((y0, Wg), (y1, Wu)):
        ok, err = _close_f16(from_dev(y, np.uint16), oracle.gemv_quant_cpu(W, 13, x, 9728, K))
        assert ok, err
    print_case("triple_rmsnorm q5k/q5k/q6k")
    w = (1.0 + 0.02 * g.standard_normal(K)).astype(np.float32)
    xn = oracle.rmsnorm(x, None, w, 1, K, 1e-6, True)
    Wk = synth.q5k(g, 1024, K)
    jllm.call("jllm_hip_gemv_quant_triple_rmsnorm", ys[0], to_dev(Wa), 13, 4096, ys[1], to_dev(Wk), 13, 1024,
              ys[2], to_dev(Wc), 14, 1024, to_dev(x), to_dev(w), 1, 1e-6, K)
    for y, W, t, M in zip(ys, (Wa, Wk, Wc), (13, 13, 14), (4096, 1024, 1024)):
        ok, err = _close_f16(from_dev(y, np.uint16), oracle.gemv_quant_cpu(W, t, xn, M, K))
        assert ok, (t, M, err)


def test_triple_routes_like_the_reference(dev):
    """A Q4_K/Q6_K triple outside the four MMVQ instantiations
    (gemv_q4.cu:1475-1490), e.g. (Q4_K, Q6_K, Q4_K), runs in float mode."""
    K = 2560
    g = synth.rng(530)
    x = synth.x_f16(g, K)
    Ws = (synth.q4k(g, 512, K), synth.q6k(g, 256, K), synth.q4k(g, 256, K))
    ys = [empty_f16(512), empty_f16(256), empty_f16(256)]
    print_case("triple q4k/q6k/q4k")
    jllm.gemv_quant_triple(ys[0], to_dev(Ws[0]), 12, 512, ys[1], to_dev(Ws[1]), 14, 256, ys[2], to_dev(Ws[2]), 12, 256,
                           to_dev(x), K)
    for y, W, t, M in zip(ys, Ws, (12, 14, 12), (512, 256, 256)):
        got = f16_to_f64(from_dev(y, np.uint16))
        fl = oracle.gemv_quant_cpu(W, t, x, M, K)
        mq = oracle.mmvq(W, t, oracle.quantize_q8_1(x, K), M, K)
        assert _close_f16(from_dev(y, np.uint16), fl)[0]
        # and it is the float result, not the MMVQ one: closer to the former
        assert np.abs(got - fl).max() < np.abs(got - mq).max()


def test_gemv_errors(dev):
    x = to_dev(synth.x_f16(synth.rng(1), 512))
    W = to_dev(synth.q4k(synth.rng(2), 4, 512))
    y = empty_f16(4)
    for bad in (11, 15, 0):
        with pytest.raises(jllm.JllmError, match="unsupported"):
            jllm.gemv_quant(y, W, bad, x, 4, 512)
    with pytest.raises(jllm.JllmError, match="invalid"):
        jllm.gemv_quant(y, W, 12, x, 4, 300)
    xl = to_dev(synth.x_f16(synth.rng(3), 28928))
    Wl = to_dev(synth.q4k(synth.rng(4), 1, 28928))
    with pytest.raises(jllm.JllmError, match="invalid"):           # K above 28672
        jllm.gemv_quant(empty_f16(1), Wl, 12, xl, 1, 28928)
    host = torch.zeros(4 * 2 * 144, dtype=torch.uint8)           # plain host memory: no fallback
    with pytest.raises(jllm.JllmError, match="visible"):
        jllm.gemv_quant(y, host, 12, x, 4, 512)


# ---- fused activation prologues ---------------------------------------------------

def _rms_case(seed, K):
    g = synth.rng(seed)
    x = synth.x_f16(g, K)
    w = (1.0 + 0.02 * g.standard_normal(K)).astype(np.float32)
    return g, x, w


def test_triple_and_pair_rmsnorm(dev):
    K, eps = 2560, 1e-6
    g, x, w = _rms_case(700, K)
    xn = oracle.rmsnorm(x, None, w, 1, K, eps, True)
    xq = oracle.quantize_q8_1(xn, K)
    Wq, Wk, Wv = synth.q4k(g, 4096, K), synth.q4k(g, 1024, K), synth.q6k(g, 1024, K)
    ys = [empty_f16(4096), empty_f16(1024), empty_f16(1024)]
    print_case("triple_rmsnorm")
    jllm.call("jllm_hip_gemv_quant_triple_rmsnorm", ys[0], to_dev(Wq), 12, 4096, ys[1], to_dev(Wk), 12, 1024,
              ys[2], to_dev(Wv), 14, 1024, to_dev(x), to_dev(w), 1, eps, K)
    for y, W, t, M in zip(ys, (Wq, Wk, Wv), (12, 12, 14), (4096, 1024, 1024)):
        ok, err = _close_f16(from_dev(y, np.uint16), oracle.mmvq(W, t, xq, M, K))
        assert ok, (t, M, err)
    print_case("pair_rmsnorm fp16 weight")
    w16 = w.astype(np.float16).view(np.uint16)
    xn16 = oracle.rmsnorm(x, None, w16, 1, K, eps, False)
    xq16 = oracle.quantize_q8_1(xn16, K)
    Wg, Wu = synth.q4k(g, 9728, K), synth.q4k(g, 9728, K)
    y0, y1 = empty_f16(9728), empty_f16(9728)
    jllm.call("jllm_hip_gemv_quant_pair_rmsnorm", y0, to_dev(Wg), 12, 9728, y1, to_dev(Wu), 12, 9728, to_dev(x),
              to_dev(w16), 0, eps, K)
    for y, W in ((y0, Wg), (y1, Wu)):
        ok, err = _close_f16(from_dev(y, np.uint16), oracle.mmvq(W, 12, xq16, 9728, K))
        assert ok, err


@pytest.mark.parametrize("t", [12, 13, 14])
def test_f32_rmsnorm_lm_head(dev, t):
    K, M, eps = 2560, {12: 4000, 13: 20000, 14: 151936}[t], 1e-6
    print_case("f32_rmsnorm", t, M)
    g, x, w = _rms_case(710 + t, K)
    W = synth.weights(g, t, M, K)
    xn = oracle.rmsnorm(x, None, w, 1, K, eps, True)
    y = empty_f32(M)
    jllm.call("jllm_hip_gemv_quant_f32_rmsnorm", y, to_dev(W), t, to_dev(x), to_dev(w), 1, eps, M, K)
    want = oracle.mmvq(W, t, oracle.quantize_q8_1(xn, K), M, K) if t == 12 else oracle.gemv_quant_cpu(W, t, xn, M, K)
    assert rel_inf(from_dev(y), want) <= TOL


def test_fused_prologue_argument_checks(dev):
    l = jllm.lib()
    x = to_dev(synth.x_f16(synth.rng(1), 4352))
    y = empty_f32(16)
    W = to_dev(synth.q4k(synth.rng(2), 16, 4352))
    w = to_dev(np.ones(4352, np.float32))
    # K above the single-pass staging limit of the fused RMSNorm
    assert l.jllm_hip_gemv_quant_f32_rmsnorm(jllm._ptr(y), jllm._ptr(W), 12, jllm._ptr(x), jllm._ptr(w), 1,
                                             1e-6, 16, 4352, None) == -1


# ---- gate/up pair with the SwiGLU epilogue ----------------------------------------

@pytest.mark.parametrize("t,M,K,rms", [(12, 9728, 2560, True), (12, 9728, 2560, False), (13, 9728, 2560, True),
                                       (12, 37, 512, False), (13, 1000, 1280, True), (12, 4000, 4096, True)])
def test_pair_swiglu_matches_pair_then_swiglu(dev, t, M, K, rms):
    """Bit-identical to the unfused pair (+ RMSNorm) followed by the SwiGLU
    kernel, and within the GEMV bar of the oracle composition."""
    print_case("pair_swiglu", t, M, K, rms)
    g = synth.rng(800 + M + t)
    x = synth.x_f16(g, K)
    w = (1.0 + 0.02 * g.standard_normal(K)).astype(np.float32)
    # block scales 20x below the BASELINE ones, so that silu(g) * u stays in fp16 range
    mk = (lambda: synth.q4k(g, M, K, 1e-3, 1e-3)) if t == 12 else (lambda: synth.q5k(g, M, K, 5e-4, 1e-3))
    Wg, Wu = mk(), mk()
    Wgd, Wud, xd, wd = to_dev(Wg), to_dev(Wu), to_dev(x), to_dev(w)
    act = empty_f16(M)
    y0, y1, act2 = empty_f16(M), empty_f16(M), empty_f16(M)
    if rms:
        jllm.call("jllm_hip_gemv_quant_pair_rmsnorm_swiglu", act, Wgd, t, Wud, t, M, xd, wd, 1, 1e-6, K)
        jllm.call("jllm_hip_gemv_quant_pair_rmsnorm", y0, Wgd, t, M, y1, Wud, t, M, xd, wd, 1, 1e-6, K)
    else:
        jllm.call("jllm_hip_gemv_quant_pair_swiglu", act, Wgd, t, Wud, t, M, xd, K)
        jllm.gemv_quant_pair(y0, Wgd, t, M, y1, Wud, t, M, xd, K)
    jllm.call("jllm_hip_fused_swiglu", act2, y0, y1, 1, M)
    got = from_dev(act, np.uint16)
    assert np.array_equal(got, from_dev(act2, np.uint16))
    xn = oracle.rmsnorm(x, None, w, 1, K, 1e-6, True) if rms else x
    if t == 12:
        xq = oracle.quantize_q8_1(xn, K)
        gy, uy = oracle.mmvq(Wg, t, xq, M, K), oracle.mmvq(Wu, t, xq, M, K)
    else:
        gy, uy = oracle.gemv_quant_cpu(Wg, t, xn, M, K), oracle.gemv_quant_cpu(Wu, t, xn, M, K)
    want = f16_to_f64(oracle.swiglu(gy.astype(np.float16).view(np.uint16), uy.astype(np.float16).view(np.uint16)))
    # gate/up carry the GEMV bar; silu(g)*u then scales it by at most ~|u| + |g|
    assert np.all(np.isfinite(want))
    err = np.abs(f16_to_f64(got) - want)
    bound = 4 * TOL * np.abs(want).max() + np.abs(want) * 2 ** -9
    assert np.all(err <= bound), float(err.max())


def test_pair_swiglu_rejects_mixed_types(dev):
    K, M = 512, 64
    x = to_dev(synth.x_f16(synth.rng(1), K))
    Wg, Wu = to_dev(synth.q4k(synth.rng(2), M, K)), to_dev(synth.q6k(synth.rng(3), M, K))
    act = empty_f16(M)
    l = jllm.lib()
    assert l.jllm_hip_gemv_quant_pair_swiglu(jllm._ptr(act), jllm._ptr(Wg), 12, jllm._ptr(Wu), 14, M, jllm._ptr(x),
                                             K, None) == -2     # JLLM_ERR_UNSUPPORTED
    W6 = to_dev(synth.q6k(synth.rng(4), M, K))
    assert l.jllm_hip_gemv_quant_pair_swiglu(jllm._ptr(act), jllm._ptr(W6), 14, jllm._ptr(W6), 14, M, jllm._ptr(x),
                                             K, None) == -2
