"""Pins the CPU oracle (oracle/kquant_oracle.c) independently of itself.

Each oracle function is checked against something that does not share its
code: numpy's IEEE fp16 conversions, a vectorised float64/int64 numpy
restatement written from the GGUF block spec (np_ref.py), closed-form
answers, the reference's own known-answer tests, and algebraic identities.
Runs on the CPU.
"""
import numpy as np
import pytest

import np_ref
import oracle
import synth


# ---- fp16 conversions -------------------------------------------------------

def test_f16_to_f32_all_patterns():
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.f16_bits_to_f32(b) for b in bits], dtype=np.float32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy():
    g = synth.rng(7)
    vals = np.concatenate([
        g.standard_normal(20000).astype(np.float32) * (10.0 ** g.integers(-9, 6, 20000)).astype(np.float32),
        (np.arange(-4096, 4096, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),   # subnormal ties
        np.array([65504, 65519.99, 65520, 1e9, -1e9, 0.0, -0.0, 2.0 ** -25, 2.0 ** -26], np.float32),
        (np.arange(1, 2049, dtype=np.float32) + 0.5),                                  # ties at 2048+
    ]).astype(np.float32)
    got = np.array([oracle.f32_to_f16_bits(v) for v in vals], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- dequant / scale unpack -----------------------------------------------------

@pytest.mark.parametrize("t", [12, 13, 14])
def test_dequant_matches_spec_restatement(t):
    rows, K = 16, 1024
    W = synth.weights(synth.rng(1), t, rows, K)
    got = oracle.dequant(W, t, rows, K).astype(np.float64)
    want = np_ref.dequant(W, t, rows, K)
    assert np.allclose(got, want, rtol=2e-7, atol=1e-12)


def test_q4k_scale_fields_each_bit_once():
    # setting a single bit of the 12 scale bytes changes exactly one 6-bit field
    W = np.zeros((1, 144), np.uint8)
    seen = set()
    for byte in range(12):
        for bit in range(8):
            W[:] = 0
            W[0, 4 + byte] = 1 << bit
            _, _, sc, mn, _ = np_ref.q4k_fields(W, 1, 256)
            nz = [("sc", j, int(sc[0, 0, j])) for j in range(8) if sc[0, 0, j]] + \
                 [("m", j, int(mn[0, 0, j])) for j in range(8) if mn[0, 0, j]]
            assert len(nz) == 1
            seen.add((nz[0][0], nz[0][1], nz[0][2]))
    assert len(seen) == 96          # 16 fields x 6 bits, all distinct


# ---- host scalar GEMV (gemv_quant_cpu) ------------------------------------------

@pytest.mark.parametrize("t", [12, 13, 14])
def test_gemv_cpu_vs_float64(t):
    rows, K = 64, 2560
    g = synth.rng(2)
    W = synth.weights(g, t, rows, K)
    x = synth.x_f16(g, K)
    y = oracle.gemv_quant_cpu(W, t, x, rows, K).astype(np.float64)
    Wd = np_ref.dequant(W, t, rows, K)
    xf = np_ref.f16(x)
    want = Wd @ xf
    bound = np.abs(Wd) @ np.abs(xf)
    assert np.all(np.abs(y - want) <= 2e-6 * bound + 1e-12)


@pytest.mark.parametrize("t", [12, 13, 14])
def test_gemv_cpu_column_probe(t):
    # x = e_k  =>  y = column k of the dequantised matrix (checks element order)
    rows, K = 8, 512
    W = synth.weights(synth.rng(3), t, rows, K)
    Wd = np_ref.dequant(W, t, rows, K)
    for k in (0, 1, 31, 32, 63, 64, 100, 127, 128, 255, 256, 300, 511):
        x = np.zeros(K, np.uint16)
        x[k] = 0x3C00  # 1.0
        y = oracle.gemv_quant_cpu(W, t, x, rows, K)
        assert np.allclose(y, Wd[:, k], rtol=1e-6, atol=0), k


def test_gemv_cpu_closed_form_zero_d():
    # d = 0  =>  y = -sum dmin*m*x
    rows, K = 4, 512
    W = synth.q4k(synth.rng(4), rows, K)
    W.reshape(rows, -1, 144)[:, :, 0:2] = 0
    x = synth.x_f16(synth.rng(5), K)
    d, dmin, sc, mn, q = np_ref.q4k_fields(W, rows, K)
    want = -(dmin[..., None, None] * mn[..., None] * np_ref.f16(x).reshape(1, -1, 8, 32)).sum(axis=(1, 2, 3))
    y = oracle.gemv_quant_cpu(W, 12, x, rows, K)
    assert np.allclose(y, want, rtol=1e-5)


def test_gemv_cpu_multithread_identical():
    rows, K = 97, 512
    g = synth.rng(6)
    W = synth.q6k(g, rows, K)
    x = synth.x_f16(g, K)
    a = oracle.gemv_quant_cpu(W, 14, x, rows, K)
    b = oracle.gemv_quant_cpu(W, 14, x, rows, K, threads=4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("t", [11, 15, 8])
def test_gemv_cpu_rejects_unsupported_type(t):
    with pytest.raises(ValueError):
        oracle.gemv_quant_cpu(np.zeros(256, np.uint8), t, np.zeros(256, np.uint16), 1, 256)


def _q5_as_q4(W5, rows, K):
    """The Q4_K tensor with the header and qs of a Q5_K tensor (qh dropped)."""
    b = W5.reshape(rows, -1, 176)
    return np.concatenate([b[:, :, 0:16], b[:, :, 48:176]], axis=2).reshape(rows, -1)


@pytest.mark.parametrize("fill", [0x00, 0xFF])
def test_q5k_closed_forms_vs_q4k(fill):
    # qh = 0: the Q5_K row is the Q4_K row of the same header and qs.
    # qh = 0xFF: every code gains 16, so y gains 16 * sum_j d*sc_j*sum(x over sub-block j).
    rows, K = 6, 768
    g = synth.rng(40)
    W5 = synth.q5k(g, rows, K)
    W5.reshape(rows, -1, 176)[:, :, 16:48] = fill
    x = synth.x_f16(g, K)
    y5 = oracle.gemv_quant_cpu(W5, 13, x, rows, K).astype(np.float64)
    W4 = _q5_as_q4(W5, rows, K)
    y4 = oracle.gemv_quant_cpu(W4, 12, x, rows, K).astype(np.float64)
    if fill == 0:
        assert np.array_equal(y5, y4)
    else:
        d, _, sc, _, _ = np_ref.q4k_fields(W4, rows, K)
        xs = np_ref.f16(x).reshape(1, -1, 8, 32).sum(axis=3)
        extra = 16 * (d[..., None] * sc * xs).sum(axis=(1, 2))
        bound = np.abs(np_ref.dequant(W5, 13, rows, K)) @ np.abs(np_ref.f16(x))
        assert np.all(np.abs(y5 - (y4 + extra)) <= 4e-6 * bound)


def test_q5k_high_bit_positions():
    # one qh bit b of byte l sets +16 on the code of sub-block b at position l
    rows, K = 1, 256
    W5 = np.zeros((rows, 176), np.uint8)
    W5[0, 0:2] = np.array([0x3C00], np.uint16).view(np.uint8)     # d = 1
    W5[0, 4:16] = 0x01                                             # sc = 1 for j < 4; j >= 4 gets low nibble 1
    for bit in range(8):
        for l in (0, 5, 31):
            W5[0, 16:48] = 0
            W5[0, 16 + l] = 1 << bit
            w = oracle.dequant(W5, 13, rows, K)[0]
            nz = np.nonzero(w)[0]
            assert list(nz) == [32 * bit + l], (bit, l, nz)
            assert w[32 * bit + l] == 16.0


# ---- q8_1 quantisers -------------------------------------------------------------

def _q8_1_unpack(buf, K):
    b = buf.reshape(K // 32, 36)
    d = b[:, 0:2].copy().view(np.uint16)[:, 0]
    s = b[:, 2:4].copy().view(np.uint16)[:, 0]
    q = b[:, 4:].view(np.int8)
    return d, s, q


def test_q8_1_matches_ieee_restatement():
    K = 4096
    x = synth.x_f16(synth.rng(8), K)
    d, s, q = _q8_1_unpack(oracle.quantize_q8_1(x, K), K)
    qn, dn = np_ref.q8_1_blocks(x, K)
    assert np.array_equal(q.astype(np.int64), qn)
    assert np.array_equal(d, dn.astype(np.float16).view(np.uint16))
    s_want = (dn.astype(np.float32) * qn.sum(axis=1).astype(np.float32)).astype(np.float16).view(np.uint16)
    assert np.array_equal(s, s_want)


def test_q8_1_closed_forms():
    K = 64
    x = np.zeros(K, np.uint16)                      # block 0: all zero
    x[32:64] = np.float16(0.25).view(np.uint16)     # block 1: constant -> all codes 127
    x[40] = np.float16(-0.5).view(np.uint16)        # amax element -> -127
    d, s, q = _q8_1_unpack(oracle.quantize_q8_1(x, K), K)
    assert d[0] == 0 and s[0] == 0 and not q[0].any()
    assert q[1][8] == -127
    assert np.all(q[1][np.arange(32) != 8] == 64)   # 0.25 / (0.5/127) = 63.5 -> 64 (ties to even)
    assert np.float16(d[1].view(np.float16)) == np.float16(np.float32(0.5) / np.float32(127))


@pytest.mark.parametrize("ds4", [True, False])
def test_mmq_quantizer_layout_and_values(ds4):
    N, K, Npad = 5, 512, 64
    x = synth.x_f16(synth.rng(9), (N, K))
    buf = oracle.quantize_mmq(x, N, K, Npad, ds4).reshape(K // 128, Npad, 144)
    assert not buf[:, N:, :].any()                  # padded token columns are zero
    xf = np_ref.f16(x).reshape(N, K // 32, 32)
    amax = np.abs(xf).max(axis=2).astype(np.float32)
    d = amax / np.float32(127)
    with np.errstate(divide="ignore"):
        dinv = np.where(d > 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    qn = np.rint((xf.astype(np.float32) * dinv[..., None]).astype(np.float32)).astype(np.int64)
    for kb in range(K // 128):
        for t in range(N):
            blk = buf[kb, t]
            q = blk[16:].view(np.int8).reshape(4, 32)
            assert np.array_equal(q, qn[t, kb * 4:(kb + 1) * 4])
            if ds4:
                h = blk[:16].copy().view(np.uint16).reshape(4, 2)
                assert np.array_equal(h[:, 0], d[t, kb * 4:(kb + 1) * 4].astype(np.float16).view(np.uint16))
                ssum = xf[t, kb * 4:(kb + 1) * 4].sum(axis=1)
                got = h[:, 1].view(np.float16).astype(np.float64)
                assert np.all(np.abs(got - ssum) <= np.abs(ssum) * 2 ** -10 + 2 ** -24 * 8)
            else:
                f = blk[:16].copy().view(np.float32)
                assert np.array_equal(f, d[t, kb * 4:(kb + 1) * 4])


# ---- MMVQ / MMQ -----------------------------------------------------------------

@pytest.mark.parametrize("t", [12, 14])
def test_mmvq_vs_exact_int_dots(t):
    rows, K = 32, 1024
    g = synth.rng(10)
    W = synth.weights(g, t, rows, K)
    x = synth.x_f16(g, K)
    xq = oracle.quantize_q8_1(x, K)
    y = oracle.mmvq(W, t, xq, rows, K).astype(np.float64)
    d8, s8, q8 = _q8_1_unpack(xq, K)
    d8 = np_ref.f16(d8); s8 = np_ref.f16(s8)
    c = np_ref.codes(W, t, rows, K)
    if t == 12:
        d, dmin, sc, mn, _ = np_ref.q4k_fields(W, rows, K)
        dots = (c.reshape(rows, -1, 32) * q8.astype(np.int64)[None]).sum(axis=2)   # [rows, K/32]
        want = ((d[..., None] * sc).reshape(rows, -1) * d8 * dots
                - (dmin[..., None] * mn).reshape(rows, -1) * s8).sum(axis=1)
    else:
        d, sc, _ = np_ref.q6k_fields(W, rows, K)
        dots = (c.reshape(rows, -1, 16) * q8.astype(np.int64).reshape(1, -1, 16)).sum(axis=2)  # [rows, K/16]
        scale = (d[..., None] * sc).reshape(rows, -1)
        want = (scale * np.repeat(d8, 2)[None] * dots).sum(axis=1)
    assert np.allclose(y, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


@pytest.mark.parametrize("t", [12, 14])
def test_mmq_subdots_bruteforce(t):
    M, N, K, Npad = 24, 7, 512, 64
    g = synth.rng(11)
    W = synth.weights(g, t, M, K)
    x = synth.x_f16(g, (N, K))
    q8 = oracle.quantize_mmq(x, N, K, Npad, ds4=(t == 12))
    sub = oracle.mmq_subdots(W, t, q8, M, N, K, Npad)
    qa = q8.reshape(K // 128, Npad, 144)[:, :N, 16:].view(np.int8).transpose(1, 0, 2).reshape(N, K).astype(np.int64)
    c = np_ref.codes(W, t, M, K)
    G = 32 if t == 12 else 16
    want = np.einsum("mgk,ngk->nmg", c.reshape(M, -1, G), qa.reshape(N, -1, G))
    assert np.array_equal(sub, want)


@pytest.mark.parametrize("t,expected", [(12, 127 * 2 * sum(range(16))), (14, 127 * sum(range(16)))])
def test_mmq_diag_probe(t, expected):
    # DIAG probe (test_mmq_q4k_int8.cu:195-201): A = k, B = 1 => C = sum k
    K, M, N, Npad = 256, 1, 1, 64
    if t == 12:
        W = np.zeros((1, 144), np.uint8)
        W[0, 16:144] = np.tile(np.arange(16, dtype=np.uint8), 8) | (np.tile(np.arange(16, dtype=np.uint8), 8) << 4)
    else:
        W = np.zeros((1, 210), np.uint8)
        # codes q-32 = k mod 16 for element k: raw q6 = 32 + (k % 16)
        raw = 32 + (np.arange(256) % 16)
        for e in range(256):
            h, p = divmod(e, 128)
            g, r = divmod(p, 32)
            lo_byte = h * 64 + r + (32 if g & 1 else 0)
            W[0, lo_byte] |= (raw[e] & 15) << (4 if g >= 2 else 0)
            W[0, 128 + h * 32 + r] |= (raw[e] >> 4) << (2 * g)
    x = np.full((1, K), np.float16(1.0).view(np.uint16), np.uint16)
    q8 = oracle.quantize_mmq(x, N, K, Npad, ds4=(t == 12))
    sub = oracle.mmq_subdots(W, t, q8, M, N, K, Npad)
    assert np.all(sub == expected)


@pytest.mark.parametrize("t", [12, 14])
def test_mmq_epilogue_vs_exact(t):
    M, N, K, Npad = 16, 5, 512, 64
    g = synth.rng(12)
    W = synth.weights(g, t, M, K)
    x = synth.x_f16(g, (N, K))
    q8 = oracle.quantize_mmq(x, N, K, Npad, ds4=(t == 12))
    y = oracle.mmq(W, t, q8, M, N, K, Npad).astype(np.float64)
    sub = oracle.mmq_subdots(W, t, q8, M, N, K, Npad).astype(np.float64)
    blk = q8.reshape(K // 128, Npad, 144)[:, :N, :16]
    if t == 12:
        h = blk.copy().view(np.uint16).reshape(K // 128, N, 4, 2)
        d8 = np_ref.f16(h[..., 0]).transpose(1, 0, 2).reshape(N, -1)
        sx = np_ref.f16(h[..., 1]).transpose(1, 0, 2).reshape(N, -1)
        d, dmin, sc, mn, _ = np_ref.q4k_fields(W, M, K)
        ax = (d[..., None] * sc).reshape(M, -1).astype(np.float16).astype(np.float64)   # half(d*sc)
        ay = (-dmin[..., None] * mn).reshape(M, -1).astype(np.float16).astype(np.float64)
        want = np.einsum("mg,ng,nmg->nm", ax, d8, sub) + np.einsum("mg,ng->nm", ay, sx)
    else:
        d4 = blk.copy().view(np.float32).reshape(K // 128, N, 4).transpose(1, 0, 2).reshape(N, -1).astype(np.float64)
        d, sc, _ = np_ref.q6k_fields(W, M, K)
        isum = sub.reshape(N, M, -1, 2) * sc.reshape(1, M, -1, 2)
        per32 = isum.sum(axis=3) * d4[:, None, :]                        # [N, M, K/32]
        want = (per32.reshape(N, M, K // 256, 8).sum(axis=3) * d[None]).sum(axis=2)
    assert np.allclose(y, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


@pytest.mark.parametrize("t", [12, 14])
def test_mmq_is_a_matmul(t):
    # loose: the int8 result approximates W_dequant @ x within q8 error
    M, N, K, Npad = 32, 6, 1024, 64
    g = synth.rng(13)
    W = synth.weights(g, t, M, K)
    x = synth.x_f16(g, (N, K))
    q8 = oracle.quantize_mmq(x, N, K, Npad, ds4=(t == 12))
    y = oracle.mmq(W, t, q8, M, N, K, Npad)
    want = np_ref.f16(x) @ np_ref.dequant(W, t, M, K).T
    rel = np.sqrt(((y - want) ** 2).mean()) / np.sqrt((want ** 2).mean())
    assert rel < 0.02


# ---- KV quantiser ---------------------------------------------------------------

def test_fp16_to_int8_known_answer():
    # test_kernels.cu:91-110: rows of +0.5 / -0.5 -> scale 0.5/127, codes +-127
    src = np.concatenate([np.full(128, np.float16(0.5)), np.full(128, np.float16(-0.5))]).view(np.uint16)
    q, sc = oracle.fp16_to_int8(src, 2, 128)
    assert abs(sc[0] - 0.5 / 127) < 1e-3 and sc[0] == np.float32(0.5) / np.float32(127)
    assert np.all(q[0] == 127) and np.all(q[1] == -127)


def test_fp16_to_int8_vs_numpy():
    rows, cols = 8, 128
    src = synth.x_f16(synth.rng(14), (rows, cols))
    q, sc = oracle.fp16_to_int8(src, rows, cols)
    v = np_ref.f16(src).astype(np.float32)
    mx = np.abs(v).max(axis=1)
    assert np.array_equal(sc, mx / np.float32(127))
    inv = (np.float32(127) / mx).astype(np.float32)
    assert np.array_equal(q, np.clip(np.rint(v * inv[:, None]), -127, 127).astype(np.int8))


# ---- attention -----------------------------------------------------------------

def _attn_case(seed, seq, n_heads=8, n_kv=2, hd=64):
    g = synth.rng(seed)
    q = synth.x_f16(g, n_heads * hd)
    k = synth.kv_int8(g, seq, n_kv, hd)
    v = synth.kv_int8(g, seq, n_kv, hd)
    ks = synth.kv_scales(g, seq, n_kv)
    vs = synth.kv_scales(g, seq, n_kv)
    return q, k, v, ks, vs, n_heads, n_kv, hd


@pytest.mark.parametrize("seq,window,splits", [(1, 0, 1), (63, 0, 1), (100, 0, 4), (300, 0, 8), (300, 64, 8), (300, 500, 8)])
def test_attention_vs_float64(seq, window, splits):
    q, k, v, ks, vs, H, KV, hd = _attn_case(15, seq)
    scale = 1.0 / np.sqrt(hd)
    out = oracle.attn_decode_int8(q, k, v, H, KV, hd, hd, seq, scale, ks, vs, window, splits)
    want = np_ref.attention_f64(q, k, v, ks, vs, H, KV, hd, seq, scale, window)
    got = np_ref.f16(out).reshape(H, hd)
    assert np.allclose(got, want, rtol=2e-3, atol=2e-3 * np.abs(want).max())


def test_attention_identities():
    q, k, v, ks, vs, H, KV, hd = _attn_case(16, 200)
    scale = 0.125
    # seq = 1 -> out = V[0] * vs
    out = np_ref.f16(oracle.attn_decode_int8(q, k, v, H, KV, hd, hd, 1, scale, ks, vs, 0, 1)).reshape(H, hd)
    for h in range(H):
        want = (v[0, h // (H // KV)].astype(np.float32) * vs[0, h // (H // KV)]).astype(np.float16)
        assert np.array_equal(out[h].astype(np.float16), want)
    # identical keys -> uniform weights -> mean of V
    k2 = np.repeat(k[:1], 200, axis=0)
    ks2 = np.repeat(ks[:1], 200, axis=0)
    out = np_ref.f16(oracle.attn_decode_int8(q, k2, v, H, KV, hd, hd, 200, scale, ks2, vs, 0, 8)).reshape(H, hd)
    for h in range(H):
        kvh = h // (H // KV)
        want = (v[:, kvh].astype(np.float64) * vs[:, kvh, None]).mean(axis=0)
        assert np.allclose(out[h], want, rtol=3e-3, atol=3e-3 * np.abs(want).max())
    # window W == plain attention over the last W positions
    a = oracle.attn_decode_int8(q, k, v, H, KV, hd, hd, 200, scale, ks, vs, 50, 8)
    b = oracle.attn_decode_int8(q, k[150:], v[150:], H, KV, hd, hd, 50, scale, ks[150:], vs[150:], 0, 1)
    assert np.allclose(np_ref.f16(a), np_ref.f16(b), rtol=2e-3, atol=1e-3)
    # split count does not change the result beyond fp32 rounding
    s1 = np_ref.f16(oracle.attn_decode_int8(q, k, v, H, KV, hd, hd, 200, scale, ks, vs, 0, 1))
    s8 = np_ref.f16(oracle.attn_decode_int8(q, k, v, H, KV, hd, hd, 200, scale, ks, vs, 0, 8))
    assert np.allclose(s1, s8, rtol=2e-3, atol=1e-3)


def test_attention_split_policy():
    # decode_attn_splits, attention.cu:1000-1005
    assert [oracle.decode_attn_splits(s) for s in (1, 63, 64, 127, 128, 8192)] == [1, 1, 4, 4, 8, 8]
