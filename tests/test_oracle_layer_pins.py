"""Pins the decoder-layer oracle (oracle/layer_oracle.c) independently of itself.

Checks come from the reference's own known-answer tests (tests/test_kernels.cu
of genie-ai-runtime: RMSNorm of x + residual = 2 is 1.0, silu(1) * 2 =
1.4621, RoPE at position 0 is the identity), closed forms, float64 numpy
restatements written from the textbook definitions, and identities (pair
norm, rotation composition).  Runs on the CPU.
"""
import numpy as np
import pytest

import np_ref
import oracle
import synth


def f16b(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def f64(bits):
    return np_ref.f16(bits)


# ---- RMSNorm ---------------------------------------------------------------

def test_rmsnorm_known_answer():
    # test_kernels.cu: x = 1, residual = 1, weight = 1 -> 1.0 (sum is 2)
    x = f16b(np.ones(256))
    out = f64(oracle.rmsnorm(x, x, np.ones(256, np.float32), 1, 256, 1e-6, True))
    assert np.all(np.abs(out - 1.0) < 1e-3)


@pytest.mark.parametrize("w_fp32", [True, False])
def test_rmsnorm_closed_forms(w_fp32):
    dim, eps = 512, 1e-2
    g = synth.rng(3)
    w = (1.0 + 0.5 * g.standard_normal(dim)).astype(np.float32)
    wbits = w if w_fp32 else f16b(w)
    wv = w.astype(np.float64) if w_fp32 else f64(wbits)
    # constant row c with residual r: every element is (c+r)/sqrt((c+r)^2 + eps) * w
    c, r = 0.375, 0.125
    out = f64(oracle.rmsnorm(f16b(np.full(dim, c)), f16b(np.full(dim, r)), wbits, 1, dim, eps, w_fp32))
    want = (c + r) / np.sqrt((c + r) ** 2 + eps) * wv
    assert np.allclose(out, want, rtol=1e-3, atol=1e-6)
    # one-hot row a*e_k: a / sqrt(a^2/dim + eps) * w_k at k, 0 elsewhere
    k, a = 137, 3.0
    x = np.zeros(dim); x[k] = a
    out = f64(oracle.rmsnorm(f16b(x), None, wbits, 1, dim, eps, w_fp32))
    want = np.zeros(dim); want[k] = a / np.sqrt(a * a / dim + eps) * wv[k]
    assert np.allclose(out, want, rtol=1e-3, atol=1e-6)


def test_rmsnorm_random_rows_vs_float64():
    rows, dim, eps = 7, 2560, 1e-6
    g = synth.rng(4)
    x, res = synth.x_f16(g, rows * dim), synth.x_f16(g, rows * dim)
    w = (1.0 + 0.02 * g.standard_normal(dim)).astype(np.float32)
    out = f64(oracle.rmsnorm(x, res, w, rows, dim, eps, True)).reshape(rows, dim)
    v = (f64(x) + f64(res)).reshape(rows, dim)
    want = v / np.sqrt((v * v).mean(axis=1, keepdims=True) + eps) * w
    assert np.all(np.abs(out - want) <= 2.0 ** -10 * np.abs(want) + 1e-6)


# ---- SwiGLU / residual add ---------------------------------------------------

def test_swiglu_known_answers_and_float64():
    out = f64(oracle.swiglu(f16b([1.0, 0.0, 20.0, -20.0]), f16b([2.0, 5.0, 0.5, 3.0])))
    assert abs(out[0] - 1.4621) < 1e-3                        # test_kernels.cu
    assert out[1] == 0.0 and abs(out[2] - 10.0) < 1e-2 and abs(out[3]) < 1e-6
    g = synth.rng(5)
    a, b = synth.x_f16(g, 4096), synth.x_f16(g, 4096)
    ga, ub = f64(a), f64(b)
    want = ga / (1.0 + np.exp(-ga)) * ub
    got = f64(oracle.swiglu(a, b))
    assert np.all(np.abs(got - want) <= 2.0 ** -10 * np.abs(want) + 1e-7)


def test_vec_add_is_rounded_sum():
    g = synth.rng(6)
    a, b = synth.x_f16(g, 5000), synth.x_f16(g, 5000)
    want = (f64(a) + f64(b)).astype(np.float16).view(np.uint16)   # exact sum, one rounding
    assert np.array_equal(oracle.vec_add(a, b), want)


# ---- RoPE --------------------------------------------------------------------

@pytest.mark.parametrize("neox", [True, False])
def test_rope_position_zero_identity(neox):
    g = synth.rng(8)
    q, k = synth.x_f16(g, 4 * 128), synth.x_f16(g, 2 * 128)
    q2, k2 = oracle.rope(q, k, 4, 2, 128, 0, 1, 1e6, neox)
    assert np.array_equal(q2, q) and np.array_equal(k2, k)


@pytest.mark.parametrize("neox", [True, False])
def test_rope_one_hot_pairs(neox):
    hd, theta, pos = 64, 10000.0, 37
    h2 = hd // 2
    for i in (0, 1, 5, h2 - 1):
        x = np.zeros(hd); x[i if neox else 2 * i] = 1.0
        q2, _ = oracle.rope(f16b(x), None, 1, 0, hd, pos, 1, theta, neox)
        out = f64(q2)
        ang = pos * theta ** (-2.0 * i / hd)
        i0, i1 = (i, i + h2) if neox else (2 * i, 2 * i + 1)
        want = np.zeros(hd); want[i0], want[i1] = np.cos(ang), np.sin(ang)
        assert np.allclose(out, want, atol=2e-3), i


def test_rope_norm_and_composition():
    hd, theta = 128, 1e6
    g = synth.rng(9)
    q = synth.x_f16(g, 3 * hd)
    a, _ = oracle.rope(q, None, 3, 0, hd, 200, 1, theta, True)
    v, w = f64(q).reshape(3, 2, 64), f64(a).reshape(3, 2, 64)
    assert np.allclose(np.hypot(w[:, 0], w[:, 1]), np.hypot(v[:, 0], v[:, 1]), rtol=2e-3, atol=2e-3)
    # R(120) R(80) = R(200)
    b, _ = oracle.rope(q, None, 3, 0, hd, 80, 1, theta, True)
    c, _ = oracle.rope(b, None, 3, 0, hd, 120, 1, theta, True)
    assert np.allclose(f64(c), f64(a), atol=1e-2)


def test_rope_batched_is_per_token():
    hd, H, KV, N = 64, 4, 2, 5
    g = synth.rng(10)
    q, k = synth.x_f16(g, N * H * hd), synth.x_f16(g, N * KV * hd)
    qb, kb = oracle.rope(q, k, H, KV, hd, 11, N, 5e5, True)
    for t in range(N):
        qt, kt = oracle.rope(q[t * H * hd:(t + 1) * H * hd], k[t * KV * hd:(t + 1) * KV * hd], H, KV, hd,
                             11 + t, 1, 5e5, True)
        assert np.array_equal(qb[t * H * hd:(t + 1) * H * hd], qt)
        assert np.array_equal(kb[t * KV * hd:(t + 1) * KV * hd], kt)


# ---- attention front (q/k norm, rope, KV store) --------------------------------

def test_qk_post_composes_the_pinned_pieces():
    H, KV, hd, N, pos0, eps, theta = 4, 2, 128, 3, 5, 1e-6, 1e6
    g = synth.rng(11)
    q, k, v = synth.x_f16(g, N * H * hd), synth.x_f16(g, N * KV * hd), synth.x_f16(g, N * KV * hd)
    qn = (1 + 0.1 * g.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * g.standard_normal(hd)).astype(np.float32)
    kc = np.zeros((pos0 + N, KV, hd), np.int8); vc = np.zeros_like(kc)
    ksc = np.zeros((pos0 + N, KV), np.float32); vsc = np.zeros_like(ksc)
    q2, k2 = oracle.qk_post(q, k, v, qn, kn, True, eps, kc, vc, ksc, vsc, H, KV, hd, hd, pos0, N, theta, True, True)
    qr = oracle.rmsnorm(q, None, qn, N * H, hd, eps, True)
    kr = oracle.rmsnorm(k, None, kn, N * KV, hd, eps, True)
    qr, kr = oracle.rope(qr, kr, H, KV, hd, pos0, N, theta, True)
    assert np.array_equal(q2, qr) and np.array_equal(k2, kr)
    kq, ks = oracle.fp16_to_int8(kr, N * KV, hd)
    vq, vs = oracle.fp16_to_int8(v, N * KV, hd)
    assert np.array_equal(kc[pos0:].reshape(N * KV, hd), kq) and np.array_equal(ksc[pos0:].ravel(), ks)
    assert np.array_equal(vc[pos0:].reshape(N * KV, hd), vq) and np.array_equal(vsc[pos0:].ravel(), vs)
    assert not kc[:pos0].any()


# ---- embedding / argmax ----------------------------------------------------------

@pytest.mark.parametrize("t", [12, 14])
def test_embed_row_is_rounded_dequant(t):
    g = synth.rng(12)
    W = synth.weights(g, t, 20, 512)
    out = f64(oracle.embed_row(W, t, 13, 512))
    want = np_ref.dequant(W, t, 20, 512)[13]
    assert np.array_equal(out, want.astype(np.float16).astype(np.float64))


def test_argmax_first_finite_max():
    g = synth.rng(13)
    x = g.standard_normal(151936).astype(np.float32)
    assert oracle.argmax(x) == int(np.argmax(x))
    x[[5, 900]] = 100.0
    x[7] = np.inf
    x[8] = np.nan
    assert oracle.argmax(x) == 5
    assert oracle.argmax(np.full(10, np.nan, np.float32)) == 0


# ---- prefill attention -----------------------------------------------------------

@pytest.mark.parametrize("start,N,window", [(0, 9, 0), (40, 24, 0), (40, 24, 16)])
def test_prefill_attention_vs_float64(start, N, window):
    H, KV, hd = 8, 2, 64
    g = synth.rng(14)
    ctx = start + N
    q = synth.x_f16(g, N * H * hd)
    k, v = synth.kv_int8(g, ctx, KV, hd), synth.kv_int8(g, ctx, KV, hd)
    ks, vs = synth.kv_scales(g, ctx, KV), synth.kv_scales(g, ctx, KV)
    scale = 1.0 / np.sqrt(hd)
    out = f64(oracle.attn_prefill_int8(q, k, v, H, KV, hd, hd, N, start, scale, ks, vs, window)).reshape(N, H, hd)
    for t in range(N):
        want = np_ref.attention_f64(q[t * H * hd:(t + 1) * H * hd], k, v, ks, vs, H, KV, hd, start + t + 1, scale,
                                    window)
        assert np.allclose(out[t], want, rtol=2e-3, atol=2e-3 * np.abs(want).max()), t


# ---- the composed decoder loop ------------------------------------------------------

TINY = dict(n_layers=2, hidden_dim=512, n_heads=8, n_kv_heads=2, head_dim=64, intermediate_dim=1024,
            vocab_size=1000)


def test_decoder_oracle_prefill_chunking_and_steps():
    """Layer-major prefill is row-independent (chunked == whole, bit-exact),
    and it agrees with running the same prompt token by token through the
    decode path (a different arithmetic: MMQ vs MMVQ / float dequant), which
    catches a wrong KV position, causal bound or residual wiring."""
    import decoder
    import decoder_oracle
    shape = decoder.Shape(**TINY)
    model = decoder.synth_np(shape, 77)
    prompt = list(synth.rng(78).integers(0, shape.vocab_size, 12))
    a = decoder_oracle.OracleDecoder(shape, model, 32)
    ta = a.prefill(prompt)
    b = decoder_oracle.OracleDecoder(shape, model, 32)
    b.prefill(prompt[:5])
    tb = b.prefill(prompt[5:], start=5)
    assert ta == tb and np.array_equal(a.logits, b.logits)
    for l in range(shape.n_layers):
        assert np.array_equal(a.kc[l], b.kc[l]) and np.array_equal(a.vs[l], b.vs[l])
    c = decoder_oracle.OracleDecoder(shape, model, 32)
    for i, t in enumerate(prompt):
        tc = c.step(t, i)
    assert tc == ta
    rel = np.abs(c.logits - a.logits).max() / np.abs(a.logits).max()
    assert rel < 2e-2, rel
    assert np.abs(a.logits).max() > 0.5                   # the random model is not degenerate


def test_layer_functions_match_decoder_oracle():
    """The one-layer oracle functions the full-size per-layer GPU test uses
    (prefill_layer_rows on a subset of the prompt rows, decode_layer) give
    exactly the layers of OracleDecoder's prefill and decode step, KV rows
    included: the prefill layer is per token except for the attention, and
    the MMQ arithmetic of a token does not depend on the other tokens."""
    import decoder
    import decoder_oracle
    shape = decoder.Shape(**TINY)
    model = decoder.synth_np(shape, 81)
    prompt = list(synth.rng(82).integers(0, shape.vocab_size, 24))
    od = decoder_oracle.OracleDecoder(shape, model, 32)
    od.trace = []
    nxt = od.prefill(prompt)
    rows = [0, 5, 11, 23]
    H = shape.hidden_dim
    for l, x_in, x_out in od.trace:
        got, k, v, ks, vs = decoder_oracle.prefill_layer_rows(
            shape, model["layers"][l], x_in.reshape(-1, H)[rows], rows, od.kc[l], od.vc[l], od.ks[l], od.vs[l])
        assert np.array_equal(got, x_out.reshape(-1, H)[rows]), l
        assert np.array_equal(k, od.kc[l][rows]) and np.array_equal(v, od.vc[l][rows]), l
        assert np.array_equal(ks, od.ks[l][rows]) and np.array_equal(vs, od.vs[l][rows]), l
    before = [(od.kc[l].copy(), od.vc[l].copy(), od.ks[l].copy(), od.vs[l].copy()) for l in range(shape.n_layers)]
    od.trace = []
    od.step(nxt, 24)
    for l, x_in, x_out in od.trace:
        kc, vc, ks, vs = before[l]
        got = decoder_oracle.decode_layer(shape, model["layers"][l], x_in, 24, kc, vc, ks, vs)
        assert np.array_equal(got, x_out), l
        assert np.array_equal(kc, od.kc[l]) and np.array_equal(vs, od.vs[l]), l


def _qwen3_float64(shape, model, theta=None):
    """A Hugging Face transformers Qwen3ForCausalLM (an implementation of the
    architecture written independently of the reference engine and of this
    repository) in float64 over the DEQUANTISED weights of `model`."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    H, I = shape.hidden_dim, shape.intermediate_dim
    cfg = Qwen3Config(vocab_size=shape.vocab_size, hidden_size=H, intermediate_size=I,
                      num_hidden_layers=shape.n_layers, num_attention_heads=shape.n_heads,
                      num_key_value_heads=shape.n_kv_heads, head_dim=shape.head_dim, rms_norm_eps=shape.rms_eps,
                      rope_theta=theta or shape.rope_theta, tie_word_embeddings=False, attention_bias=False,
                      max_position_embeddings=4096, use_cache=False)
    cfg._attn_implementation = "eager"
    m = Qwen3ForCausalLM(cfg).to(torch.float64).eval()
    deq = {12: np_ref.q4k_dequant, 13: np_ref.q5k_dequant, 14: np_ref.q6k_dequant}

    def mat(W, t, M, K):
        return torch.from_numpy(np.ascontiguousarray(deq[t](W, M, K)))

    def vec(a):
        return torch.from_numpy(np.asarray(a, np.float64))
    sd = {"model.embed_tokens.weight": mat(model["tok_embd"], model["embd_type"], shape.vocab_size, H),
          "lm_head.weight": mat(model["output"], model["output_type"], shape.vocab_size, H),
          "model.norm.weight": vec(model["output_norm"])}
    names = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj", "wo": "self_attn.o_proj",
             "w_gate": "mlp.gate_proj", "w_up": "mlp.up_proj", "w_down": "mlp.down_proj"}
    for l, L in enumerate(model["layers"]):
        p = f"model.layers.{l}."
        for k, n in names.items():
            M, K = shape.mat_shape(k)
            sd[p + n + ".weight"] = mat(L[k], L["types"][k], M, K)
        sd[p + "input_layernorm.weight"] = vec(L["rms_attn"])
        sd[p + "post_attention_layernorm.weight"] = vec(L["rms_ffn"])
        sd[p + "self_attn.q_norm.weight"] = vec(L["q_norm"])
        sd[p + "self_attn.k_norm.weight"] = vec(L["k_norm"])
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m


def test_decoder_oracle_vs_float64_qwen3():
    """The decoder oracle's layer order (RMSNorm placement, q/k RMSNorm
    before a neox RoPE with base 1e6, GQA, SwiGLU, residuals, output norm)
    pinned against an independent float64 Qwen3 forward (transformers'
    Qwen3ForCausalLM) over the dequantised weights: the logits of the
    prefill's last row and of three teacher-forced decode steps agree within
    the quantisation error (q8 activations, int8 KV, fp16 intermediates),
    while the same forward with the RoPE base off (1e4) -- one plausible
    misreading -- misses by several times more."""
    import torch
    import decoder
    import decoder_oracle
    shape = decoder.Shape(**TINY)
    model = decoder.synth_np(shape, 83)
    prompt = list(synth.rng(84).integers(0, shape.vocab_size, 40))
    od = decoder_oracle.OracleDecoder(shape, model, 64)
    toks = [od.prefill(prompt)]
    got = [od.logits.copy()]
    for i in range(3):
        toks.append(od.step(toks[-1], len(prompt) + i))
        got.append(od.logits.copy())
    seq = prompt + toks[:3]

    def ref_logits(theta=None):
        m = _qwen3_float64(shape, model, theta)
        with torch.no_grad():
            lg = m(torch.tensor([seq])).logits[0].numpy()
        return [lg[len(prompt) - 1 + i] for i in range(4)]
    want = ref_logits()
    wrong = ref_logits(1e4)
    errs = [float(np.abs(g - w).max() / np.abs(w).max()) for g, w in zip(got, want)]
    miss = [float(np.abs(g - w).max() / np.abs(w).max()) for g, w in zip(got, wrong)]
    print("oracle vs float64 Qwen3:", errs, "with the RoPE base off:", miss)
    assert max(errs) < 0.05 and max(errs[1:]) < 0.02, errs
    assert min(miss) > 4 * max(errs), (errs, miss)
    assert all(int(np.argmax(w)) == t for w, t in zip(want, toks) if np.sort(w)[-1] - np.sort(w)[-2] >
               0.1 * np.abs(w).max())


# ---- kernels outside the Llama/Qwen decode path ------------------------------

def test_geglu_against_exact_gelu():
    from scipy.special import erf
    g = synth.rng(21)
    gate = f16b(np.concatenate([np.linspace(-8, 8, 4001), g.standard_normal(3000) * 3]))
    one = f16b(np.ones(gate.size))
    got = f64(oracle.geglu(gate, one))
    x = f64(gate)
    exact = x * 0.5 * (1.0 + erf(x / np.sqrt(2.0)))
    # the tanh form is within ~4.7e-4 of the erf GELU (plus one fp16 rounding)
    assert np.all(np.abs(got - exact) <= 5e-4 + np.abs(exact) * 2 ** -10)
    # odd part: gelu(x) - gelu(-x) = x  (one fp16 rounding each)
    neg = f64(oracle.geglu(f16b(-x), one))
    assert np.all(np.abs((got - neg) - x) <= 2 * 2 ** -10 * np.maximum(np.abs(got), np.abs(neg)) + 1e-6)
    # up = 0 -> 0; up scales the result
    assert np.all(f64(oracle.geglu(gate, f16b(np.zeros(gate.size)))) == 0)


def test_vec_scale_is_fp16_product():
    g = synth.rng(22)
    for n in (1, 2, 7, 1000, 1001):
        x = synth.x_f16(g, n)
        for s in (1.5, 0.1, 3.3333, 1.0 / 3.0):
            got = oracle.vec_scale(x, s).view(np.float16)
            xf = x.view(np.float16)
            m = n & ~1
            want = np.empty(n, np.float16)
            want[:m] = (xf[:m].astype(np.float32) * np.float32(np.float16(s))).astype(np.float16)
            want[m:] = (xf[m:].astype(np.float32) * np.float32(s)).astype(np.float16)
            assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # s = 2 doubles exactly
    x = synth.x_f16(g, 64)
    assert np.array_equal(oracle.vec_scale(x, 2.0).view(np.float16), x.view(np.float16) * np.float16(2))


def test_logit_softcap_vs_float64():
    g = synth.rng(23)
    x = (g.standard_normal(10000) * 40).astype(np.float32)
    got = oracle.logit_softcap(x, 30.0)
    want = 30.0 * np.tanh(x.astype(np.float64) / 30.0)
    assert np.all(np.abs(got - want) <= 4 * np.spacing(np.abs(want).astype(np.float32)) + 1e-7)
    small = np.float32([1e-3, -2e-3])
    assert np.allclose(oracle.logit_softcap(small, 30.0), small, rtol=1e-6)


def test_softmax_vs_float64():
    g = synth.rng(24)
    x = (g.standard_normal(151936) * 5).astype(np.float32)
    got = oracle.softmax(x).astype(np.float64)
    e = np.exp(x.astype(np.float64) - x.max())
    want = e / e.sum()
    assert np.abs(got.sum() - 1.0) < 1e-4
    assert np.all(np.abs(got - want) <= 1e-4 * want + 1e-12)
    assert np.allclose(oracle.softmax(x + np.float32(3.0)), got, rtol=1e-4, atol=1e-12)


@pytest.mark.parametrize("wtype", [0, 1, 30])
def test_dense_vs_float64(wtype):
    import torch
    g = synth.rng(25 + wtype)
    M, N, K = 37, 3, 520
    wf = (g.standard_normal((M, K)) * 0.05).astype(np.float32)
    if wtype == 0:
        W, wv = wf, wf.astype(np.float64)
    elif wtype == 1:
        W = f16b(wf)
        wv = f64(W).reshape(M, K)
    else:
        tb = torch.from_numpy(wf).to(torch.bfloat16)
        W = tb.view(torch.int16).numpy().view(np.uint16)
        wv = tb.to(torch.float64).numpy()
    x = synth.x_f16(g, (N, K))
    got = f64(oracle.dense(W, wtype, x, M, N, K)).reshape(N, M)
    want = f64(x).reshape(N, K) @ wv.T
    sabs = np.abs(f64(x).reshape(N, K)) @ np.abs(wv).T
    assert np.all(np.abs(got - want) <= 2 ** -11 * np.abs(want) + 1e-6 * sabs + 1e-7)
    # a transposed operand or a dropped term would miss by O(|want|)
    assert np.abs(want).max() > 0.1
