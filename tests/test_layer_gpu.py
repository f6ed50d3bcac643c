"""GPU parity of the decoder-layer kernels around the matmuls and of the
prefill attention, through the C ABI, against the CPU oracle.

Bars: bit-exact for the integer / exactly-rounded operations (residual add,
embedding dequant, argmax, the KV int8 store when its fp16 input is exact);
at most one fp16 ulp for the fp16 outputs whose fp32 intermediate comes from
a reduction in another order or from a libm function (RMSNorm, SwiGLU);
for RoPE outputs (a rotation, whose cancellation magnifies an input ulp)
one ulp plus 2^-10 of the row's largest magnitude; int8 codes within 1
where the fp16 value they quantise may differ; attention |out - oracle| <= 1e-3 * max|oracle| + one fp16 ulp.
"""
import numpy as np
import pytest
import torch

import jllm
import np_ref
import oracle
import synth
from gpu_util import f16_to_f64, from_dev, print_case, to_dev

pytestmark = pytest.mark.gpu


def ulps(a, b):
    """fp16 ulp distance of two bit arrays (same-sign monotone mapping)."""
    def key(x):
        x = np.asarray(x, np.uint16).astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)
    return np.abs(key(a) - key(b))


def close_rows(got, want, width):
    """fp16 outputs of a chain of rounded stages (norm -> fp16 -> rotation ->
    fp16): |got - want| <= one fp16 ulp of the value + 2^-10 of the largest
    magnitude in its row (the rotation's cancellation turns an ulp of an
    input into several ulps of a small output)."""
    g, w = f16_to_f64(got).reshape(-1, width), f16_to_f64(want).reshape(-1, width)
    tol = np.abs(w) * 2.0 ** -10 + np.abs(w).max(axis=1, keepdims=True) * 2.0 ** -10
    return bool(np.all(np.abs(g - w) <= tol))


def dev16(n, dev):
    return torch.empty(n, dtype=torch.int16, device=dev)


# ---- RMSNorm -------------------------------------------------------------------

@pytest.mark.parametrize("rows,dim,res,w_fp32,inplace", [
    (1, 2560, False, True, False), (1, 2560, True, True, False), (32, 128, False, True, True),
    (8, 128, False, False, True), (512, 2560, False, True, False), (5, 250, True, False, False),
    (3, 1030, True, True, False), (7, 4096, True, False, False)])
def test_rmsnorm(dev, rows, dim, res, w_fp32, inplace):
    print_case("rmsnorm", rows, dim, res, w_fp32, inplace)
    g = synth.rng(rows * 7 + dim)
    x = synth.x_f16(g, rows * dim)
    r = synth.x_f16(g, rows * dim) if res else None
    w = (1.0 + 0.02 * g.standard_normal(dim)).astype(np.float32)
    wb = w if w_fp32 else w.astype(np.float16).view(np.uint16)
    xd = to_dev(x)
    out = xd if inplace else dev16(rows * dim, dev)
    jllm.call("jllm_hip_fused_rmsnorm_residual", out, xd, to_dev(r) if res else None, to_dev(wb), rows, dim,
              1e-6, 1 if w_fp32 else 0)
    got = from_dev(out, np.uint16)
    want = oracle.rmsnorm(x, r, wb, rows, dim, 1e-6, w_fp32)
    assert ulps(got, want).max() <= 1


# ---- SwiGLU / residual add -----------------------------------------------------

@pytest.mark.parametrize("n", [9728, 512 * 9728, 1001])
def test_swiglu(dev, n):
    print_case("swiglu", n)
    g = synth.rng(n)
    a, b = synth.x_f16(g, n), synth.x_f16(g, n)
    out = dev16(n, dev)
    jllm.call("jllm_hip_fused_swiglu", out, to_dev(a), to_dev(b), 1, n)
    got = from_dev(out, np.uint16)
    want = oracle.swiglu(a, b)
    d = ulps(got, want)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


@pytest.mark.parametrize("n,offset", [(2560, 0), (512 * 2560, 0), (1001, 1)])
def test_vec_add_bit_exact(dev, n, offset):
    print_case("vec_add", n, offset)
    g = synth.rng(n + 1)
    a, b = synth.x_f16(g, n + offset), synth.x_f16(g, n + offset)
    ad, bd = to_dev(a), to_dev(b)
    out = dev16(n + offset, dev)
    jllm.call("jllm_hip_vec_add", out[offset:], ad[offset:], bd[offset:], n)
    got = from_dev(out, np.uint16)[offset:]
    assert np.array_equal(got, oracle.vec_add(a[offset:], b[offset:]))


# ---- RoPE ------------------------------------------------------------------------

@pytest.mark.parametrize("hd,pos,neox,with_k", [(128, 0, True, True), (128, 1234, True, True), (64, 77, False, True),
                                                (128, 40000, True, False), (96, 5, True, True)])
def test_rope_inplace(dev, hd, pos, neox, with_k):
    print_case("rope", hd, pos, neox, with_k)
    H, KV = 32, 8
    g = synth.rng(hd + pos)
    q, k = synth.x_f16(g, H * hd), synth.x_f16(g, KV * hd)
    qd, kd = to_dev(q), to_dev(k)
    jllm.call("jllm_hip_rope_inplace", qd, kd if with_k else None, H, KV, hd, pos, 1e6, 1 if neox else 0)
    wq, wk = oracle.rope(q, k if with_k else None, H, KV, hd, pos, 1, 1e6, neox)
    assert close_rows(from_dev(qd, np.uint16), wq, hd)
    if with_k:
        assert close_rows(from_dev(kd, np.uint16), wk, hd)
    else:
        assert np.array_equal(from_dev(kd, np.uint16), k)
    if pos == 0:
        assert np.array_equal(from_dev(qd, np.uint16), q)


def test_rope_batched_strided(dev):
    print_case("rope_batched")
    H, KV, hd, N = 8, 2, 128, 37
    qs, ks = H * hd + 64, KV * hd + 32                       # row strides with padding
    g = synth.rng(21)
    q, k = synth.x_f16(g, N * qs), synth.x_f16(g, N * ks)
    qd, kd = to_dev(q), to_dev(k)
    jllm.call("jllm_hip_rope_inplace_batched", qd, kd, H, KV, hd, 100, N, qs, ks, 1e6, 1)
    wq, wk = oracle.rope(q, k, H, KV, hd, 100, N, 1e6, True, qs, ks)
    assert close_rows(from_dev(qd, np.uint16).reshape(N, qs)[:, :H * hd], wq.reshape(N, qs)[:, :H * hd], hd)
    assert close_rows(from_dev(kd, np.uint16).reshape(N, ks)[:, :KV * hd], wk.reshape(N, ks)[:, :KV * hd], hd)
    # padding untouched
    gq = from_dev(qd, np.uint16).reshape(N, qs)
    assert np.array_equal(gq[:, H * hd:], q.reshape(N, qs)[:, H * hd:])


# ---- fused attention front ---------------------------------------------------------

@pytest.mark.parametrize("N,pos0,norm,kv_int8,chd", [(1, 0, False, True, 128), (1, 777, True, True, 128),
                                                      (64, 0, True, True, 128), (5, 300, True, False, 128),
                                                      (3, 10, True, True, 160)])
def test_qk_post(dev, N, pos0, norm, kv_int8, chd):
    print_case("qk_post", N, pos0, norm, kv_int8, chd)
    H, KV, hd, eps, theta = 32, 8, 128, 1e-6, 1e6
    g = synth.rng(N * 3 + pos0)
    q, k, v = synth.x_f16(g, N * H * hd), synth.x_f16(g, N * KV * hd), synth.x_f16(g, N * KV * hd)
    qn = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32) if norm else None
    kn = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32) if norm else None
    ctx = pos0 + N
    et = np.int8 if kv_int8 else np.uint16
    kc, vc = np.zeros((ctx, KV, chd), et), np.zeros((ctx, KV, chd), et)
    ksc, vsc = np.zeros((ctx, KV), np.float32), np.zeros((ctx, KV), np.float32)
    wq, wk = oracle.qk_post(q, k, v, qn, kn, True, eps, kc, vc, ksc, vsc, H, KV, hd, chd, pos0, N, theta, True,
                            kv_int8)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    kcd, vcd = to_dev(np.zeros_like(kc)), to_dev(np.zeros_like(vc))
    ksd, vsd = to_dev(np.zeros_like(ksc)), to_dev(np.zeros_like(vsc))
    row = KV * chd
    jllm.call("jllm_hip_qk_norm_rope_store_kv", qd, kd, vd, to_dev(qn) if norm else None,
              to_dev(kn) if norm else None, 1, eps, kcd[pos0:], vcd[pos0:], ksd[pos0:], vsd[pos0:], row, H, KV, hd,
              chd, pos0, N, theta, 1, 1 if kv_int8 else 0)
    assert close_rows(from_dev(qd, np.uint16), wq, hd)
    gk = from_dev(kd, np.uint16)
    assert close_rows(gk, wk, hd)
    gkc, gvc = from_dev(kcd), from_dev(vcd)
    if kv_int8:
        # v is quantised from the unmodified input: bit-exact
        assert np.array_equal(gvc, vc) and np.array_equal(from_dev(vsd), vsc)
        # k: exact where the fp16 rotated keys agree, else codes within 1
        assert np.abs(gkc.astype(np.int32) - kc.astype(np.int32)).max() <= 1
        assert np.allclose(from_dev(ksd), ksc, rtol=1e-3)
        same = np.array_equal(gk, wk)
        if same:
            assert np.array_equal(gkc, kc)
    else:
        assert np.array_equal(gvc.view(np.uint16), vc)
        assert close_rows(gkc.view(np.uint16)[..., :hd], kc[..., :hd], hd)
    assert not np.any(gkc[:pos0]) and not np.any(gvc[:pos0])
    if chd > hd:
        assert not np.any(gkc[..., hd:])


# ---- embedding / argmax -------------------------------------------------------------

@pytest.mark.parametrize("t", [12, 13, 14])
def test_embedding_rows_bit_exact(dev, t):
    """Q4_K / Q6_K: dequant_embedding_q4k/q6k_kernel; Q5_K rows: the engine's
    host dequant (decode.cu:230-266) -- the single-row entry point keeps the
    reference's Q4_K/Q6_K-only contract (gemv_q4.cu:2777-2810)."""
    print_case("embedding", t)
    vocab, hidden = 300, 2560
    g = synth.rng(t)
    W = synth.weights(g, t, vocab, hidden)
    Wd = to_dev(W)
    toks = np.array([0, 299, 17, 17, 150, -1, 300], np.int32)
    out = dev16(len(toks) * hidden, dev)
    jllm.call("jllm_hip_dequant_embedding_rows", out, Wd, t, to_dev(toks), len(toks), hidden, vocab)
    got = from_dev(out, np.uint16).reshape(len(toks), hidden)
    for i, tok in enumerate(toks):
        want = oracle.embed_row(W, t, tok, hidden) if 0 <= tok < vocab else np.zeros(hidden, np.uint16)
        assert np.array_equal(got[i], want), (i, tok)
    one = dev16(hidden, dev)
    if t == 13:
        assert jllm.lib().jllm_hip_dequant_embedding_row(jllm._ptr(one), jllm._ptr(Wd), 13, 123, hidden, None) != 0
        return
    jllm.call("jllm_hip_dequant_embedding_row", one, Wd, t, 123, hidden)
    assert np.array_equal(from_dev(one, np.uint16), oracle.embed_row(W, t, 123, hidden))


@pytest.mark.parametrize("n", [151936, 1000, 7, 4099, 262144, 262145])
def test_argmax(dev, n):
    print_case("argmax", n)
    g = synth.rng(n)
    x = g.standard_normal(n).astype(np.float32)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    for case in range(7):
        if case == 1:
            x[n // 3] = x[n - 1] = 50.0                      # tie: the lower index wins
        if case == 2:
            x[min(2, n - 1)] = np.inf
            x[0] = np.nan
        if case == 3:
            x[:] = np.nan
        if case == 4:
            # ties inside one wave of the first workgroup, across the lane
            # rows and halves the reduction merges (element 4 t is lane t's)
            x = g.standard_normal(n).astype(np.float32)
            for i in (4 * 50, 4 * 3, 4 * 33, 4 * 17):
                if i < n:
                    x[i] = 60.0
        if case == 5:
            x = np.full(n, -np.inf, np.float32)              # no finite value: index 0
        if case == 6:
            # ties in different workgroups and waves, the highest index first
            x = g.standard_normal(n).astype(np.float32)
            for i in (4 * (1024 * 9 + 700) + 2, 4 * (1024 * 3 + 5) + 1, 4 * 1000 + 3, 4 * 70):
                if i < n:
                    x[i] = 70.0
        jllm.call("jllm_hip_argmax_f32", out, to_dev(x), n)
        assert int(from_dev(out)[0]) == oracle.argmax(x), case


def test_argmax_unaligned(dev):
    x = synth.rng(3).standard_normal(1001).astype(np.float32)
    xd = to_dev(x)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    jllm.call("jllm_hip_argmax_f32", out, xd[1:], 1000)
    assert int(from_dev(out)[0]) == oracle.argmax(x[1:])


# ---- prefill attention -----------------------------------------------------------------

def _close(got, want):
    err = np.abs(got - want)
    return bool(np.all(err <= 1e-3 * np.abs(want).max() + np.abs(want) * 2 ** -10)), float(err.max())


@pytest.mark.parametrize("H,KV,hd,start,N,window", [(32, 8, 128, 0, 1, 0), (32, 8, 128, 0, 40, 0),
                                                     (32, 8, 128, 100, 64, 0), (32, 8, 128, 0, 512, 0),
                                                     (16, 2, 64, 30, 33, 16), (8, 8, 96, 0, 17, 0),
                                                     (32, 2, 128, 7, 41, 0), (24, 8, 128, 0, 70, 32)])
def test_prefill_attention(dev, H, KV, hd, start, N, window):
    print_case("prefill_attn", H, KV, hd, start, N, window)
    g = synth.rng(start + N + hd)
    ctx = start + N
    q = synth.x_f16(g, N * H * hd)
    k, v = synth.kv_int8(g, ctx, KV, hd), synth.kv_int8(g, ctx, KV, hd)
    ks, vs = synth.kv_scales(g, ctx, KV), synth.kv_scales(g, ctx, KV)
    scale = 1.0 / np.sqrt(hd)
    out = dev16(N * H * hd, dev)
    jllm.call("jllm_hip_flash_attention_prefill_batched", out, to_dev(q), to_dev(k), to_dev(v), H, KV, hd, hd, N,
              start, scale, 1, to_dev(ks), to_dev(vs), window)
    got = f16_to_f64(from_dev(out, np.uint16))
    want = f16_to_f64(oracle.attn_prefill_int8(q, k, v, H, KV, hd, hd, N, start, scale, ks, vs, window))
    ok, err = _close(got, want)
    assert ok, err
    # the last token of a prefill equals a decode step at the same length
    dq = dev16(H * hd, dev)
    jllm.call("jllm_hip_flash_attention_decode", dq, to_dev(q[(N - 1) * H * hd:]), to_dev(k), to_dev(v), H, KV, hd,
              hd, ctx, scale, 1, to_dev(ks), to_dev(vs), window)
    ok, err = _close(f16_to_f64(from_dev(dq, np.uint16)), want[(N - 1) * H * hd:])
    assert ok, err
