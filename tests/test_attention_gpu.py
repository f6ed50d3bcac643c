"""GPU parity of INT8-KV split-K decode attention and the KV quantiser.

Attention outputs are fp16; the bar is |out - oracle| <= 1e-3 * max|oracle|
+ one fp16 ulp of the value, against the CPU restatement of the reference's
split-K partial/reduce kernels (and, independently, float64 softmax
attention).  The KV quantiser is compared bit-exactly.
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
TOL = 1e-3
H, KV, HD = 32, 8, 128


def _case(seed, ctx, n_heads=H, n_kv=KV, hd=HD, chd=None):
    chd = chd or hd
    g = synth.rng(seed)
    q = synth.x_f16(g, n_heads * hd)
    k = np.zeros((ctx, n_kv, chd), np.int8)
    v = np.zeros((ctx, n_kv, chd), np.int8)
    k[:, :, :hd] = synth.kv_int8(g, ctx, n_kv, hd)
    v[:, :, :hd] = synth.kv_int8(g, ctx, n_kv, hd)
    ks = synth.kv_scales(g, ctx, n_kv)
    vs = synth.kv_scales(g, ctx, n_kv)
    return q, k, v, ks, vs


def _run(dev, q, k, v, ks, vs, n_heads, n_kv, hd, chd, seq, window, splits=None):
    out = torch.empty(n_heads * hd, dtype=torch.int16, device=dev)
    args = [out, to_dev(q), to_dev(k), to_dev(v), n_heads, n_kv, hd, chd, seq, 1.0 / np.sqrt(hd), 1,
            to_dev(ks), to_dev(vs), window]
    if splits is None:
        jllm.call("jllm_hip_flash_attention_decode", *args)
    else:
        jllm.call("jllm_hip_flash_attention_decode_splits", *args, splits)
    return f16_to_f64(from_dev(out, np.uint16))


def _close(got, want):
    err = np.abs(got - want)
    return bool(np.all(err <= TOL * np.abs(want).max() + np.abs(want) * 2 ** -10)), float(err.max())


@pytest.mark.parametrize("ctx,window", [(1, 0), (37, 0), (64, 0), (100, 0), (512, 0), (4096, 0), (8192, 0),
                                        (4096, 512), (8192, 512), (300, 64), (200, 500),
                                        # ragged key ranges around the 4-wave groups (64 ranges) and the
                                        # 128-range cap: a partial last range, a partial last group
                                        (2047, 0), (2049, 0), (6001, 0), (8193, 0), (5000, 1000)])
def test_attention_vs_oracle(dev, ctx, window):
    print_case("attn", ctx, window)
    q, k, v, ks, vs = _case(ctx + window, ctx)
    got = _run(dev, q, k, v, ks, vs, H, KV, HD, HD, ctx, window)
    want = f16_to_f64(oracle.attn_decode_int8(q, k, v, H, KV, HD, HD, ctx, 1.0 / np.sqrt(HD), ks, vs, window,
                                              oracle.decode_attn_splits(ctx)))
    ok, err = _close(got, want)
    assert ok, err
    if ctx <= 4096:
        ref64 = np_ref.attention_f64(q, k, v, ks, vs, H, KV, HD, ctx, 1.0 / np.sqrt(HD), window).reshape(-1)
        ok, err = _close(got, ref64)
        assert ok, err


@pytest.mark.parametrize("splits", [1, 3, 8, 32, 64, 200, 256])
def test_attention_split_invariance(dev, splits):
    ctx = 2000
    print_case("attn_splits", splits)
    q, k, v, ks, vs = _case(5, ctx)
    base = _run(dev, q, k, v, ks, vs, H, KV, HD, HD, ctx, 0, splits=1)
    got = _run(dev, q, k, v, ks, vs, H, KV, HD, HD, ctx, 0, splits=splits)
    ok, err = _close(got, base)
    assert ok, err


@pytest.mark.parametrize("n_heads,n_kv,hd,chd", [(8, 8, 64, 64), (16, 2, 128, 160), (12, 1, 96, 96), (32, 4, 128, 128)])
def test_attention_shapes(dev, n_heads, n_kv, hd, chd):
    ctx = 333
    print_case("attn_shape", n_heads, n_kv, hd, chd)
    q, k, v, ks, vs = _case(7, ctx, n_heads, n_kv, hd, chd)
    got = _run(dev, q, k, v, ks, vs, n_heads, n_kv, hd, chd, ctx, 0)
    want = f16_to_f64(oracle.attn_decode_int8(q, k, v, n_heads, n_kv, hd, chd, ctx, 1.0 / np.sqrt(hd), ks, vs, 0,
                                              oracle.decode_attn_splits(ctx)))
    ok, err = _close(got, want)
    assert ok, err


def test_attention_fp16_kv(dev):
    ctx, n_heads, n_kv, hd = 700, 16, 4, 128
    g = synth.rng(9)
    q = synth.x_f16(g, n_heads * hd)
    k = (g.standard_normal((ctx, n_kv, hd)) * 0.5).astype(np.float16)
    v = g.standard_normal((ctx, n_kv, hd)).astype(np.float16)
    out = torch.empty(n_heads * hd, dtype=torch.int16, device=dev)
    jllm.call("jllm_hip_flash_attention_decode", out, to_dev(q), to_dev(k.view(np.uint16)), to_dev(v.view(np.uint16)),
              n_heads, n_kv, hd, hd, ctx, 1.0 / np.sqrt(hd), 0, None, None, 0)
    got = f16_to_f64(from_dev(out, np.uint16))
    ones = np.ones((ctx, n_kv), np.float32)
    want = np_ref.attention_f64(q, k.astype(np.float64), v.astype(np.float64), ones, ones, n_heads, n_kv, hd, ctx,
                                1.0 / np.sqrt(hd), 0).reshape(-1)
    ok, err = _close(got, want)
    assert ok, err


def test_attention_empty_sequence(dev):
    q = synth.x_f16(synth.rng(1), H * HD)
    out = torch.full((H * HD,), 123, dtype=torch.int16, device=dev)
    kv = torch.zeros(16, dtype=torch.int8, device=dev)
    jllm.call("jllm_hip_flash_attention_decode", out, to_dev(q), kv, kv, H, KV, HD, HD, 0, 0.1, 1, None, None, 0)
    assert not from_dev(out).any()


def test_splits_policy_and_partials(dev):
    assert [jllm.lib().jllm_hip_decode_attn_splits(s) for s in (1, 32, 33, 512, 4096, 20000)] == [1, 1, 2, 16, 128, 128]
    assert jllm.lib().jllm_hip_get_splitk_partials(32, 32, 128)


@pytest.mark.parametrize("rows,cols", [(8, 128), (1, 64), (3, 1000)])
def test_fp16_to_int8_bit_exact(dev, rows, cols):
    src = synth.x_f16(synth.rng(rows * cols), (rows, cols))
    src[0] = 0                                                   # all-zero row -> scale 0, codes 0
    dst = torch.empty(rows * cols, dtype=torch.int8, device=dev)
    sc = torch.empty(rows, dtype=torch.float32, device=dev)
    jllm.call("jllm_hip_fp16_to_int8", dst, sc, to_dev(src), rows, cols)
    q, s = oracle.fp16_to_int8(src, rows, cols)
    assert np.array_equal(from_dev(dst).reshape(rows, cols), q)
    assert np.array_equal(from_dev(sc).view(np.uint32), s.view(np.uint32))


def test_fp16_to_int8_known_answer(dev):
    # test_kernels.cu:91-110
    src = np.concatenate([np.full(128, np.float16(0.5)), np.full(128, np.float16(-0.5))]).view(np.uint16)
    dst = torch.empty(256, dtype=torch.int8, device=dev)
    sc = torch.empty(2, dtype=torch.float32, device=dev)
    jllm.call("jllm_hip_fp16_to_int8", dst, sc, to_dev(src), 2, 128)
    s = from_dev(sc)
    assert abs(s[0] - 0.5 / 127) < 1e-3
    d = from_dev(dst)
    assert np.all(d[:128] == 127) and np.all(d[128:] == -127)


@pytest.mark.parametrize("rows,cols", [(8, 128), (1, 64), (300, 1024)])
def test_kv_int8_round_trip(dev, rows, cols):
    """The reference's round-trip bar (test_kv_int8_convert.cu:154): codes
    times scale reproduce every value within 2 % of its row's max |v|
    (rounding error <= scale / 2 = max / 254)."""
    print_case("kv_roundtrip", rows, cols)
    g = synth.rng(rows + cols)
    x = (g.uniform(-1.0, 1.0, (rows, cols)) * g.uniform(0.01, 10.0, (rows, 1))).astype(np.float16)
    dst = torch.empty(rows * cols, dtype=torch.int8, device=dev)
    sc = torch.empty(rows, dtype=torch.float32, device=dev)
    jllm.call("jllm_hip_fp16_to_int8", dst, sc, to_dev(x.view(np.uint16)), rows, cols)
    back = from_dev(dst).reshape(rows, cols).astype(np.float64) * from_dev(sc).astype(np.float64)[:, None]
    xf = x.astype(np.float64)
    amax = np.abs(xf).max(axis=1, keepdims=True)
    assert np.all(np.abs(back - xf) <= 0.02 * amax)
    assert np.all(np.abs(back - xf) <= amax / 254 * (1 + 1e-5))


def test_attention_repeats_and_graph_replays(dev):
    """Back-to-back split-K calls sharing the partials scratch, and graph
    replays of them with eager work in between, give the eager result every
    time."""
    ctx = 500                                        # 16 splits
    print_case("attn_repeat_graph", ctx)
    q, k, v, ks, vs = _case(11, ctx)
    qd, kd, vd, ksd, vsd = to_dev(q), to_dev(k), to_dev(v), to_dev(ks), to_dev(vs)
    outs = [torch.zeros(H * HD, dtype=torch.int16, device=dev) for _ in range(2)]

    def calls():
        for i, o in enumerate(outs):
            jllm.call("jllm_hip_flash_attention_decode", o, qd, kd, vd, H, KV, HD, HD, ctx - 37 * i,
                      1.0 / np.sqrt(HD), 1, ksd, vsd, 0)
    calls()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    want = f16_to_f64(oracle.attn_decode_int8(q, k, v, H, KV, HD, HD, ctx, 1.0 / np.sqrt(HD), ks, vs, 0,
                                              oracle.decode_attn_splits(ctx)))
    assert _close(f16_to_f64(from_dev(eager[0], np.uint16)), want)[0]
    for _ in range(3):
        calls()
    torch.cuda.synchronize()
    for o, e in zip(outs, eager):
        assert torch.equal(o, e)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        calls()
    for r in range(4):
        for o in outs:
            o.zero_()
        gr.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), r
        calls()                                      # eager work between replays
        torch.cuda.synchronize()


def test_captured_graph_survives_scratch_growth(dev):
    """A graph captured with the library's split-K partials keeps valid memory
    when a later, larger call grows that scratch: the old buffer is retired,
    not freed, so the graph's replays still give the eager result."""
    print_case("attn_graph_scratch_growth")
    ctx = 512
    q, k, v, ks, vs = _case(77, ctx)
    qd, kd, vd, ksd, vsd = to_dev(q), to_dev(k), to_dev(v), to_dev(ks), to_dev(vs)
    out = torch.empty(H * HD, dtype=torch.int16, device=dev)
    args = [out, qd, kd, vd, H, KV, HD, HD, ctx, 1.0 / np.sqrt(HD), 1, ksd, vsd, 0]
    jllm.call("jllm_hip_flash_attention_decode", *args)
    want = from_dev(out, np.uint16).copy()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        jllm.call("jllm_hip_flash_attention_decode", *args)
    out.zero_()
    gr.replay()
    assert np.array_equal(from_dev(out, np.uint16), want)
    # a larger request (64 heads x 256 splits) grows the partials buffer
    big = 64
    qb = to_dev(synth.x_f16(synth.rng(78), big * HD))
    outb = torch.empty(big * HD, dtype=torch.int16, device=dev)
    jllm.call("jllm_hip_flash_attention_decode_splits", outb, qb, kd, vd, big, KV, HD, HD, ctx, 1.0 / np.sqrt(HD), 1,
              ksd, vsd, 0, 256)
    torch.cuda.synchronize()
    filler = torch.full((64 << 20,), 7, dtype=torch.uint8, device=dev)     # reuse of freed memory would show
    for _ in range(3):
        out.zero_()
        gr.replay()
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(out, np.uint16), want)
    del filler
