"""GPU checks of the drop-in boundary beyond the hot-path kernels:

* the device-position (graph-capturable) entry points -- decode attention,
  RoPE, RoPE + fp16 KV store -- give the same bits as their host-position
  forms, also when one captured HIP graph is replayed for several positions;
* the batched RoPE + fp16 KV store with row strides, and the Gemma-family /
  logits kernels (GeGLU, vec_scale, soft-cap, softmax, dense projections)
  against the CPU oracle;
* the namespace jllm C++ layer (tests/cxx/libengine_calls.so calls it with
  the engine's argument types): same bits as the C ABI, zero-filled output
  on an error, and the engine's mapped-weight registry found through the
  library's weak reference.

Bars as in the other GPU tests: bit-exact where the arithmetic is the same
expression (vec_scale, the position variants against their fixed forms);
one fp16 ulp where a libm function or a reduction order differs (GeGLU,
dense projections); 4 fp32 ulps for the soft-cap; for softmax 2e-4 relative to the oracle's
serial fp32 sum and 2e-5 to float64.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import jllm
import oracle
import synth
from gpu_util import f16_to_f64, from_dev, print_case, to_dev

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EC_PATH = os.path.join(ROOT, "tests", "cxx", "libengine_calls.so")
H, KV, HD = 32, 8, 128


def ulps(a, b):
    def key(x):
        x = np.asarray(x, np.uint16).astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)
    return np.abs(key(a) - key(b))


def dev16(n):
    return torch.empty(n, dtype=torch.int16, device="cuda:0")


def pos_tensor(p):
    return torch.tensor([p], dtype=torch.int32, device="cuda:0")


_ec = None


def ec():
    global _ec
    if _ec is None:
        if not os.path.exists(EC_PATH):
            pytest.fail(f"{EC_PATH} is not built (tests/cxx/build.py)")
        _ec = ctypes.CDLL(EC_PATH)
        _ec.ec_get_splitk_partials.restype = ctypes.c_void_p
    return _ec


def P(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def S():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def F(x):
    return ctypes.c_float(x)


def _kv_case(seed, ctx, int8):
    g = synth.rng(seed)
    q = synth.x_f16(g, H * HD)
    if int8:
        k, v = synth.kv_int8(g, ctx, KV, HD), synth.kv_int8(g, ctx, KV, HD)
        ks, vs = synth.kv_scales(g, ctx, KV), synth.kv_scales(g, ctx, KV)
        return to_dev(q), to_dev(k), to_dev(v), to_dev(ks), to_dev(vs)
    k = (g.standard_normal((ctx, KV, HD)) * 0.5).astype(np.float16).view(np.uint16)
    v = g.standard_normal((ctx, KV, HD)).astype(np.float16).view(np.uint16)
    return to_dev(q), to_dev(k), to_dev(v), None, None


# ---- device-position entry points ---------------------------------------------------

@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("seq,splits,window", [(1, 1, 0), (37, 8, 0), (300, 8, 0), (1000, 32, 0), (1000, 64, 256),
                                               (20, 128, 0)])
def test_attention_dyn_equals_static(dev, int8, seq, splits, window):
    print_case("attn_dyn", int8, seq, splits, window)
    q, k, v, ks, vs = _kv_case(seq + splits, 1024, int8)
    scale = 1.0 / np.sqrt(HD)
    a, b = dev16(H * HD), dev16(H * HD)
    jllm.call("jllm_hip_flash_attention_decode_splits", a, q, k, v, H, KV, HD, HD, seq, scale, int(int8), ks, vs,
              window, splits)
    jllm.call("jllm_hip_flash_attention_decode_dyn", b, q, k, v, H, KV, HD, HD, pos_tensor(seq - 1), scale,
              int(int8), ks, vs, window, splits)
    assert torch.equal(a, b)


@pytest.mark.parametrize("S_", [16, 128])        # 128 key ranges run as workgroups of 4 waves
def test_attention_dyn_graph_replays(dev, S_):
    """One captured graph (d_pos read at execution time) replayed for several
    positions equals the eager host-position call at each of them."""
    q, k, v, ks, vs = _kv_case(3, 2048, True)
    scale = 1.0 / np.sqrt(HD)
    assert jllm.lib().jllm_hip_get_splitk_partials(H, S_, HD)
    d_pos = pos_tensor(0)
    out, ref = dev16(H * HD), dev16(H * HD)
    jllm.call("jllm_hip_flash_attention_decode_dyn", out, q, k, v, H, KV, HD, HD, d_pos, scale, 1, ks, vs, 0, S_)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        jllm.call("jllm_hip_flash_attention_decode_dyn", out, q, k, v, H, KV, HD, HD, d_pos, scale, 1, ks, vs, 0, S_)
    for p in (0, 31, 32, 500, 2047, 100):
        print_case("attn_dyn_graph", S_, p)
        d_pos.fill_(p)
        gr.replay()
        jllm.call("jllm_hip_flash_attention_decode_splits", ref, q, k, v, H, KV, HD, HD, p + 1, scale, 1, ks, vs, 0,
                  S_)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), p
        want = oracle.attn_decode_int8(from_dev(q, np.uint16), from_dev(k), from_dev(v), H, KV, HD, HD, p + 1, scale,
                                       from_dev(ks), from_dev(vs), 0, oracle.decode_attn_splits(p + 1))
        w = f16_to_f64(want)
        g = f16_to_f64(from_dev(out, np.uint16))
        assert np.all(np.abs(g - w) <= 1e-3 * np.abs(w).max() + np.abs(w) * 2 ** -10)


@pytest.mark.parametrize("pos,with_k", [(0, True), (777, True), (40000, True), (5, False)])
def test_rope_dyn_equals_static(dev, pos, with_k):
    print_case("rope_dyn", pos, with_k)
    g = synth.rng(pos + 1)
    q, k = synth.x_f16(g, H * HD), synth.x_f16(g, KV * HD)
    q1, k1, q2, k2 = to_dev(q), to_dev(k), to_dev(q), to_dev(k)
    nkv = KV if with_k else 0
    jllm.call("jllm_hip_rope_inplace", q1, k1 if with_k else None, H, nkv, HD, pos, 1e6, 1)
    jllm.call("jllm_hip_rope_inplace_dyn", q2, k2 if with_k else None, H, nkv, HD, pos_tensor(pos), 1e6, 1)
    assert torch.equal(q1, q2) and torch.equal(k1, k2)
    if not with_k:
        assert torch.equal(k2, to_dev(k))


@pytest.mark.parametrize("chd", [128, 160])
def test_rope_store_kv_fp16_dyn(dev, chd):
    """The device-position store writes k (rotated) and v at
    base + pos * n_kv * cache_head_dim, head h at h * cache_head_dim: the
    oracle's fused front without norms and with an fp16 cache."""
    pos, ctx = 300, 512
    print_case("rope_store_dyn", chd)
    g = synth.rng(chd)
    q, k, v = synth.x_f16(g, H * HD), synth.x_f16(g, KV * HD), synth.x_f16(g, KV * HD)
    kc, vc = np.zeros((ctx, KV, chd), np.uint16), np.zeros((ctx, KV, chd), np.uint16)
    wq, wk = oracle.qk_post(q, k, v, None, None, True, 1e-6, kc, vc, None, None, H, KV, HD, chd, pos, 1, 1e6, True,
                            False)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    kcd, vcd = to_dev(np.zeros_like(kc)), to_dev(np.zeros_like(vc))
    jllm.call("jllm_hip_rope_inplace_store_kv_fp16_dyn", qd, kd, vd, kcd, vcd, H, KV, HD, chd, pos_tensor(pos), 1e6, 1)
    # the fixed-position form (reference rope_inplace_store_kv_fp16) at the same row: same bits
    q2, k2 = to_dev(q), to_dev(k)
    kr, vr = dev16(KV * HD), dev16(KV * HD)
    jllm.call("jllm_hip_qk_norm_rope_store_kv", q2, k2, vd, None, None, 1, 1e-6, kr, vr, None, None, KV * HD, H, KV,
              HD, HD, pos, 1, 1e6, 1, 0)
    assert torch.equal(qd, q2) and torch.equal(kd, k2)
    gkc, gvc = from_dev(kcd).view(np.uint16), from_dev(vcd).view(np.uint16)
    assert np.array_equal(gkc[pos][:, :HD].ravel(), from_dev(kr, np.uint16))
    assert np.array_equal(gvc, vc)
    assert np.max(ulps(gkc[pos][:, :HD], kc[pos][:, :HD])) <= 1 and np.max(ulps(from_dev(qd, np.uint16), wq)) <= 1
    others = np.ones(ctx, bool)
    others[pos] = False
    assert not gkc[others].any() and not gvc[others].any()
    if chd > HD:
        assert not gkc[..., HD:].any()


def test_rope_store_kv_fp16_batched_strided(dev):
    """rope_inplace_store_kv_fp16_batched: q/k/v rows with strides wider than
    the heads (fused QKV layout), cache rows of kv_slot halves; the padding
    columns stay untouched."""
    N, start, qs, kvs, slot = 9, 100, H * HD + 64, KV * HD + 32, KV * HD + 8
    g = synth.rng(77)
    q, k, v = synth.x_f16(g, N * qs), synth.x_f16(g, N * kvs), synth.x_f16(g, N * kvs)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    kb, vb = to_dev(np.zeros(N * slot, np.uint16)), to_dev(np.zeros(N * slot, np.uint16))
    jllm.call("jllm_hip_rope_inplace_store_kv_fp16_batched", qd, kd, vd, kb, vb, slot, H, KV, HD, start, N, qs, kvs,
              1e6, 1)
    qp, kp = q.reshape(N, qs)[:, :H * HD], k.reshape(N, kvs)[:, :KV * HD]
    wq, wk = oracle.rope(qp, kp, H, KV, HD, start, N, 1e6, True)
    gq, gk = from_dev(qd, np.uint16).reshape(N, qs), from_dev(kd, np.uint16).reshape(N, kvs)
    assert ulps(gq[:, :H * HD].ravel(), wq).max() <= 1 and ulps(gk[:, :KV * HD].ravel(), wk).max() <= 1
    assert np.array_equal(gq[:, H * HD:], q.reshape(N, qs)[:, H * HD:])
    gkb, gvb = from_dev(kb, np.uint16).reshape(N, slot), from_dev(vb, np.uint16).reshape(N, slot)
    assert np.array_equal(gkb[:, :KV * HD], gk[:, :KV * HD])
    assert np.array_equal(gvb[:, :KV * HD], v.reshape(N, kvs)[:, :KV * HD])
    assert not gkb[:, KV * HD:].any() and not gvb[:, KV * HD:].any()


# ---- Gemma-family / logits kernels -------------------------------------------------------

@pytest.mark.parametrize("n", [1, 1001, 9728 * 3])
def test_geglu(dev, n):
    print_case("geglu", n)
    g = synth.rng(n + 5)
    a, b = synth.x_f16(g, n), synth.x_f16(g, n)
    out = dev16(n)
    jllm.call("jllm_hip_fused_geglu", out, to_dev(a), to_dev(b), 1, n)
    assert ulps(from_dev(out, np.uint16), oracle.geglu(a, b)).max() <= 1


@pytest.mark.parametrize("n", [1, 2, 2561, 2560 * 7])
def test_vec_scale_bit_exact(dev, n):
    print_case("vec_scale", n)
    x = synth.x_f16(synth.rng(n), n)
    for s in (0.70710678, 50.596443, 1.0 / 3.0):
        xd = to_dev(x)
        jllm.call("jllm_hip_vec_scale", xd, n, s)
        assert np.array_equal(from_dev(xd, np.uint16), oracle.vec_scale(x, s))


def test_logit_softcap(dev):
    x = (synth.rng(3).standard_normal(151936) * 40).astype(np.float32)
    xd = to_dev(x)
    jllm.call("jllm_hip_logit_softcap", xd, x.size, 30.0)
    got, want = from_dev(xd), oracle.logit_softcap(x, 30.0)
    assert np.all(np.abs(got - want) <= 4 * np.spacing(np.abs(want)) + 1e-7)


@pytest.mark.parametrize("n", [1, 1000, 151936])
def test_softmax(dev, n):
    print_case("softmax", n)
    x = (synth.rng(n).standard_normal(n) * 6).astype(np.float32)
    xd = to_dev(x)
    jllm.call("jllm_hip_softmax_inplace", xd, n)
    got, want = from_dev(xd), oracle.softmax(x)
    # the oracle sums the n exponentials serially in fp32 (error ~1e-4 at the
    # vocabulary size), the kernel in a tree: both against float64 too
    e = np.exp(x.astype(np.float64) - x.max())
    assert np.all(np.abs(got - want) <= 2e-4 * want + 1e-12)
    assert np.all(np.abs(got - e / e.sum()) <= 2e-5 * e / e.sum() + 1e-12)


@pytest.mark.parametrize("wtype,M,N,K", [(0, 2560, 1, 256), (30, 256 * 35, 1, 2560), (1, 333, 5, 2560),
                                        (0, 64, 17, 520), (30, 7, 3, 13)])
def test_dense(dev, wtype, M, N, K):
    print_case("dense", wtype, M, N, K)
    g = synth.rng(M + N + K + wtype)
    wf = (g.standard_normal((M, K)) * 0.05).astype(np.float32)
    if wtype == 0:
        W = wf
    elif wtype == 1:
        W = wf.astype(np.float16).view(np.uint16)
    else:
        W = torch.from_numpy(wf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    x = synth.x_f16(g, (N, K))
    out = dev16(N * M)
    if N == 1:
        jllm.call("jllm_hip_gemv_dense", out, to_dev(W), wtype, to_dev(x), M, K)
    else:
        jllm.call("jllm_hip_gemm_dense_batched", out, to_dev(W), wtype, to_dev(x), M, N, K)
    got, want = from_dev(out, np.uint16), oracle.dense(W, wtype, x, M, N, K)
    gw, ww = f16_to_f64(got), f16_to_f64(want)
    assert np.all((ulps(got, want) <= 1) | (np.abs(gw - ww) <= 1e-4 * np.abs(ww).max()))


# ---- the namespace jllm C++ layer ----------------------------------------------------------

def test_cxx_layer_matches_c_abi(dev):
    """The C++ entry points the engine calls give the C ABI's bits."""
    l = ec()
    g = synth.rng(11)
    M, K, N = 1024, 2560, 7
    W4, W6 = to_dev(synth.q4k(g, M, K)), to_dev(synth.q6k(g, M, K))
    x, xs = to_dev(synth.x_f16(g, K)), to_dev(synth.x_f16(g, N * K))
    r = to_dev(synth.x_f16(g, M))
    for t, W in ((12, W4), (14, W6)):
        a, b = dev16(M), dev16(M)
        jllm.call("jllm_hip_gemv_quant", a, W, t, x, M, K)
        l.ec_gemv_quant(P(b), P(W), t, P(x), M, K, S())
        assert torch.equal(a, b)
        jllm.call("jllm_hip_gemv_quant_add", a, W, t, x, r, M, K)
        l.ec_gemv_quant_add(P(b), P(W), t, P(x), P(r), M, K, S())
        assert torch.equal(a, b)
        af, bf = torch.empty(M, device=dev), torch.empty(M, device=dev)
        jllm.call("jllm_hip_gemv_quant_f32", af, W, t, x, M, K)
        l.ec_gemv_quant_f32(P(bf), P(W), t, P(x), M, K, S())
        assert torch.equal(af, bf)
        a, b = dev16(N * M), dev16(N * M)
        jllm.call("jllm_hip_gemm_quant_batched", a, W, t, xs, M, N, K)
        l.ec_gemm_quant_batched(P(b), P(W), t, P(xs), M, N, K, S())
        assert torch.equal(a, b)
    a0, a1, a2, b0, b1, b2 = (dev16(M) for _ in range(6))
    jllm.call("jllm_hip_gemv_quant_triple", a0, W4, 12, M, a1, W4, 12, M, a2, W6, 14, M, x, K)
    l.ec_gemv_quant_triple(P(b0), P(W4), 12, M, P(b1), P(W4), 12, M, P(b2), P(W6), 14, M, P(x), K, S())
    assert torch.equal(a0, b0) and torch.equal(a1, b1) and torch.equal(a2, b2)
    jllm.call("jllm_hip_gemv_quant_pair", a0, W4, 12, M, a1, W4, 12, M, x, K)
    l.ec_gemv_quant_pair(P(b0), P(W4), 12, M, P(b1), P(W4), 12, M, P(x), K, S())
    assert torch.equal(a0, b0) and torch.equal(a1, b1)
    # attention (static and both dyn forms) and the KV quantiser
    q, k, v, ks, vs = _kv_case(2, 700, True)
    a, b, c = dev16(H * HD), dev16(H * HD), dev16(H * HD)
    jllm.call("jllm_hip_flash_attention_decode", a, q, k, v, H, KV, HD, HD, 700, 0.0884, 1, ks, vs, 0)
    l.ec_flash_attention_decode(P(b), P(q), P(k), P(v), H, KV, HD, HD, 700, F(0.0884), 1, P(ks), P(vs), 0, S())
    n_s = l.ec_decode_attn_splits(700)
    assert l.ec_get_splitk_partials(H, n_s, HD)
    l.ec_flash_attention_decode_dyn2(P(c), P(q), P(k), P(v), H, KV, HD, HD, P(pos_tensor(699)), F(0.0884), 1, P(ks),
                                     P(vs), 0, n_s, S())
    assert torch.equal(a, b) and torch.equal(a, c)
    qf, kf, vf, _, _ = _kv_case(4, 300, False)
    jllm.call("jllm_hip_flash_attention_decode_splits", a, qf, kf, vf, H, KV, HD, HD, 300, 0.0884, 0, None, None, 0, 8)
    l.ec_flash_attention_decode_dyn1(P(b), P(qf), P(kf), P(vf), H, KV, HD, HD, P(pos_tensor(299)), F(0.0884), 0,
                                     None, 0, 8, S())
    assert torch.equal(a, b)
    src = to_dev(synth.x_f16(g, 8 * HD))
    i8a, i8b = torch.empty(8 * HD, dtype=torch.int8, device=dev), torch.empty(8 * HD, dtype=torch.int8, device=dev)
    sa, sb = torch.empty(8, device=dev), torch.empty(8, device=dev)
    jllm.call("jllm_hip_fp16_to_int8", i8a, sa, src, 8, HD)
    l.ec_fp16_to_int8(P(i8b), P(sb), P(src), 8, HD, S())
    assert torch.equal(i8a, i8b) and torch.equal(sa, sb)
    # element-wise and norm kernels
    w = to_dev((1 + 0.02 * g.standard_normal(K)).astype(np.float32))
    a, b = dev16(K), dev16(K)
    jllm.call("jllm_hip_fused_rmsnorm_residual", a, x, x, w, 1, K, 1e-6, 1)
    l.ec_fused_rmsnorm_residual(P(b), P(x), P(x), P(w), 1, K, F(1e-6), 1, S())
    assert torch.equal(a, b)
    for fn in ("fused_swiglu", "fused_geglu"):
        jllm.call("jllm_hip_" + fn, a, x, x, 1, K)
        getattr(l, "ec_" + fn)(P(b), P(x), P(x), 1, K, S())
        assert torch.equal(a, b)
    torch.cuda.synchronize()


def _filled(n, dtype=torch.int16):
    return torch.full((n,), 0x3C00 if dtype == torch.int16 else 1, dtype=dtype, device="cuda:0")


def test_cxx_layer_errors_zero_fill(dev):
    """On an error the C++ layer prints and zero-fills the output (the
    reference's unsupported-type behaviour, gemv_q4.cu:2667-2669); in-place
    operations leave their data unchanged."""
    l = ec()
    g = synth.rng(12)
    M, K = 256, 2560
    W, x = to_dev(synth.q4k(g, M, K)), to_dev(synth.x_f16(g, K))
    y = _filled(M)
    l.ec_gemv_quant(P(y), P(W), 2, P(x), M, K, S())                     # unsupported type (Q4_0)
    assert not from_dev(y).any()
    y = _filled(4 * M)
    l.ec_gemm_quant_batched(P(y), P(W), 12, P(x), M, 4, 300, S())       # K not a multiple of 256
    assert not from_dev(y).any()
    yf = _filled(M, torch.float32)
    l.ec_gemv_quant_f32(P(yf), P(W), 12, P(x), M, K + 1, S())
    assert not from_dev(yf).any()
    q, k, v, ks, vs = _kv_case(5, 64, True)
    out = _filled(H * HD)
    l.ec_flash_attention_decode_dyn1(P(out), P(q), P(k), P(v), H, KV, HD, HD, P(pos_tensor(10)), F(0.1), 1, P(ks), 0,
                                     8, S())                             # INT8 with one scales pointer: refused
    assert not from_dev(out).any()
    out = _filled(H * HD)
    l.ec_flash_attention_decode(P(out), P(q), P(k), P(v), H, KV, HD, 64, 10, F(0.1), 1, P(ks), P(vs), 0, S())
    assert not from_dev(out).any()
    qq = to_dev(synth.x_f16(g, H * 130))
    before = qq.clone()
    l.ec_rope_inplace(P(qq), None, H, 0, 130, 5, F(1e6), 1, S())        # head_dim > 128: unchanged
    assert torch.equal(qq, before)
    dst = _filled(K)
    assert l.ec_dequant_embedding_row(P(dst), P(W), 13, 0, K, S()) == 0  # Q5_K single row: refused, as the reference
    assert not from_dev(dst).any()
    sm = torch.ones(10, device=dev)
    l.ec_softmax_inplace(P(sm), 0, S())                                # n = 0: nothing changes
    assert torch.equal(sm, torch.ones(10, device=dev))


def test_cxx_layer_negative_sizes_write_nothing(dev):
    """A negative (or overflowing) size is rejected and the C++ layer's error
    path writes nothing -- the zero fill is sized by fill_bytes, 0 for such
    shapes -- so a canary buffer handed in as the output stays as it was
    (the reference's invalid sizes fail at launch and write nothing,
    gemv_q4.cu:2633-2775)."""
    l = ec()
    g = synth.rng(14)
    M, K = 256, 2560
    W, x = to_dev(synth.q4k(g, M, K)), to_dev(synth.x_f16(g, K))
    c0, c1, c2 = _filled(4096), _filled(4096), _filled(4096)
    cf = _filled(4096, torch.float32)
    ref16, reff = c0.clone(), cf.clone()
    l.ec_gemv_quant(P(c0), P(W), 12, P(x), -M, K, S())
    l.ec_gemv_quant_add(P(c0), P(W), 12, P(x), P(x), -M, K, S())
    l.ec_gemv_quant_pair(P(c0), P(W), 12, -M, P(c1), P(W), 12, -1, P(x), K, S())
    l.ec_gemv_quant_triple(P(c0), P(W), 12, -M, P(c1), P(W), 12, -2, P(c2), P(W), 14, -3, P(x), K, S())
    l.ec_gemv_quant_f32(P(cf), P(W), 12, P(x), -M, K, S())
    l.ec_gemm_quant_batched(P(c0), P(W), 12, P(x), -M, 4, K, S())
    l.ec_gemm_quant_batched(P(c0), P(W), 12, P(x), M, -4, K, S())
    l.ec_gemm_quant_batched(P(c0), P(W), 12, P(x), 1 << 30, 1 << 30, 300, S())   # M*N*2 = 2^61 bytes
    l.ec_quantize_q8_1(P(x), P(c0), -2560, S())
    q, k, v, ks, vs = _kv_case(6, 64, True)
    l.ec_flash_attention_decode(P(c0), P(q), P(k), P(v), -H, KV, HD, HD, 10, F(0.1), 1, P(ks), P(vs), 0, S())
    l.ec_flash_attention_decode(P(c0), P(q), P(k), P(v), H, KV, -HD, HD, 10, F(0.1), 1, P(ks), P(vs), 0, S())
    l.ec_flash_attention_prefill_batched(P(c0), P(q), P(k), P(v), H, KV, HD, HD, -3, 0, F(0.1), 1, P(ks), P(vs),
                                         0, S())
    l.ec_fused_rmsnorm_residual(P(c0), P(x), P(x), P(x), -1, K, F(1e-6), 1, S())
    l.ec_fused_swiglu(P(c0), P(x), P(x), 1, -K, S())
    assert l.ec_dequant_embedding_row(P(c0), P(W), 12, 0, -K, S()) == 0
    i8 = torch.ones(4096, dtype=torch.int8, device=dev)
    sc = torch.ones(64, device=dev)
    l.ec_fp16_to_int8(P(i8), P(sc), P(x), -8, 128, S())
    torch.cuda.synchronize()
    for t in (c0, c1, c2):
        assert torch.equal(t, ref16)
    assert torch.equal(cf, reff)
    assert bool((i8 == 1).all()) and bool((sc == 1).all())


def test_cxx_fp16_to_int8_error_fill_is_byte_exact(dev):
    """On a rejected call with a valid shape (src missing), fp16_to_int8 zero
    fills exactly rows x cols bytes of dst -- an odd count included -- and the
    rows scales; the bytes after them are untouched."""
    l = ec()
    rows, cols = 8, 127
    i8 = torch.ones(1024, dtype=torch.int8, device=dev)
    sc = torch.ones(16, device=dev)
    l.ec_fp16_to_int8(P(i8), P(sc), None, rows, cols, S())
    torch.cuda.synchronize()
    got, gs = from_dev(i8), from_dev(sc)
    assert not got[:rows * cols].any() and (got[rows * cols:] == 1).all()
    assert not gs[:rows].any() and (gs[rows:] == 1).all()


def test_oversized_requests_refused(dev):
    """Sizes beyond what the kernels address are refused up front, with no
    allocation attempt: a GEMM whose quantised activation or weight matrix
    exceeds the kernels' 2 GiB buffer ranges, a partials buffer beyond the
    decode kernels' limits (2^30 heads x 2^30 splits once overflowed the
    scratch size and never returned)."""
    x = torch.zeros(4096, dtype=torch.int16, device=dev)
    y = torch.zeros(64, dtype=torch.int16, device=dev)
    W = torch.zeros(4096, dtype=torch.uint8, device=dev)
    lib = jllm.lib()
    for M, N, K in ((64, 1 << 20, 1536), (1 << 22, 64, 2560), (1 << 30, 1 << 30, 256)):
        for t in (12, 14):
            st = lib.jllm_hip_gemm_quant_batched(y.data_ptr(), W.data_ptr(), t, x.data_ptr(), M, N, K, None)
            assert st == -1, (M, N, K, t, st)
    assert not lib.jllm_hip_get_splitk_partials(1 << 30, 1 << 30, 128)
    assert not lib.jllm_hip_get_splitk_partials(32, 257, 128)
    assert not lib.jllm_hip_get_splitk_partials(32, 8, 256)
    assert lib.jllm_hip_get_splitk_partials(32, 256, 128)
    torch.cuda.synchronize()


SPLITK_CHILD = r"""
import ctypes, sys
sys.path[:0] = [sys.argv[1]]
ec = ctypes.CDLL(sys.argv[2])
print("splits", [ec.ec_decode_attn_splits(s) for s in (1, 63, 64, 700, 8192)])
"""


@pytest.mark.parametrize("env,want", [(None, [1, 2, 2, 22, 128]), ("1", [1, 2, 2, 22, 128]),
                                      ("0", [1, 1, 1, 1, 1])])
def test_splitk_switch(dev, env, want):
    """JLLM_SPLITK=0 makes decode_attn_splits return 1 for every length (the
    reference's splitk_enabled, attention.cu:990-1005); read once per
    process, so each setting runs in a child process of its own."""
    e = dict(os.environ)
    e.pop("JLLM_SPLITK", None)
    if env is not None:
        e["JLLM_SPLITK"] = env
    r = subprocess.run([sys.executable, "-c", SPLITK_CHILD, os.path.join(ROOT, "genie-ai-runtime_amd"), EC_PATH],
                       capture_output=True, text=True, timeout=120, env=e)
    assert r.returncode == 0, r.stderr[-2000:]
    assert f"splits {want}" in r.stdout, r.stdout


SPLITK_ATTN_CHILD = r"""
import ctypes, sys
import numpy as np
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import torch, jllm, synth
from gpu_util import to_dev
H, KV, HD, ctx = 32, 8, 128, 700
g = synth.rng(21)
q, k, v = synth.x_f16(g, H * HD), synth.kv_int8(g, ctx, KV, HD), synth.kv_int8(g, ctx, KV, HD)
ks, vs = synth.kv_scales(g, ctx, KV), synth.kv_scales(g, ctx, KV)
out = torch.zeros(H * HD, dtype=torch.int16, device="cuda:0")
jllm.call("jllm_hip_flash_attention_decode", out, to_dev(q), to_dev(k), to_dev(v), H, KV, HD, HD, ctx,
          1.0 / np.sqrt(HD), 1, to_dev(ks), to_dev(vs), 0)
one = torch.zeros_like(out)
jllm.call("jllm_hip_flash_attention_decode_splits", one, to_dev(q), to_dev(k), to_dev(v), H, KV, HD, HD, ctx,
          1.0 / np.sqrt(HD), 1, to_dev(ks), to_dev(vs), 0, 1)
torch.cuda.synchronize()
print("same_as_one_split", bool(torch.equal(out, one)))
"""


@pytest.mark.parametrize("env,same", [("0", True), (None, False)])
def test_splitk_switch_static_entry(dev, env, same):
    """With JLLM_SPLITK=0 the static decode entry runs one split: its output
    is bit-identical to an explicit one-split call (and, with split-K on,
    it is not -- 22 key ranges combine in another order)."""
    e = dict(os.environ)
    e.pop("JLLM_SPLITK", None)
    if env is not None:
        e["JLLM_SPLITK"] = env
    r = subprocess.run([sys.executable, "-c", SPLITK_ATTN_CHILD, os.path.join(ROOT, "genie-ai-runtime_amd"),
                        os.path.dirname(os.path.abspath(__file__))], capture_output=True, text=True, timeout=300,
                       env=e)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert f"same_as_one_split {same}" in r.stdout, r.stdout


REGISTRY_CHILD = r"""
import ctypes, sys
import numpy as np
sys.path[:0] = [sys.argv[1], sys.argv[2]]
ec = ctypes.CDLL(sys.argv[3], mode=ctypes.RTLD_GLOBAL)    # the engine side first, as a linked engine would be
import torch, jllm, synth, oracle
g = synth.rng(13)
M, K = 512, 2560
Wh = np.ascontiguousarray(synth.q4k(g, M, K))             # plain host memory, unknown to HIP
x = synth.x_f16(g, K)
Wd = torch.from_numpy(Wh).cuda()                          # its device copy
xd = torch.from_numpy(x.view(np.int16)).cuda()
y = torch.empty(M, dtype=torch.float32, device="cuda:0")
st = jllm.lib().jllm_hip_gemv_quant_f32(y.data_ptr(), Wh.ctypes.data, 12, xd.data_ptr(), M, K, None)
assert st != 0, "an unregistered host pointer must be refused"
ec.ec_register_mapped_weight_region(ctypes.c_void_p(Wh.ctypes.data), ctypes.c_void_p(Wd.data_ptr()),
                                    ctypes.c_int64(Wh.nbytes))
ec.ec_gemv_quant_f32(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(Wh.ctypes.data), 12,
                     ctypes.c_void_p(xd.data_ptr()), M, K, None)
torch.cuda.synchronize()
want = oracle.mmvq(Wh, 12, oracle.quantize_q8_1(x, K), M, K)
err = float(np.abs(y.cpu().numpy() - want).max() / np.abs(want).max())
assert err <= 1e-3, err
ec.ec_clear_mapped_weight_region(ctypes.c_void_p(Wh.ctypes.data))
print("registry ok")
"""


def test_engine_registry_through_weak_reference(dev):
    """A host weight pointer registered in the ENGINE's registry (model.cpp's
    functions, here tests/cxx/model_registry_stub.cpp) resolves to its device
    alias inside the library, which only holds a weak reference to it.  Run
    in a child process so the engine side is loaded before the library, as
    in a linked engine."""
    r = subprocess.run([sys.executable, "-c", REGISTRY_CHILD, os.path.join(ROOT, "genie-ai-runtime_amd"),
                        os.path.join(ROOT, "oracle"), EC_PATH], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "registry ok" in r.stdout, r.stdout[-3000:] + r.stderr[-3000:]
