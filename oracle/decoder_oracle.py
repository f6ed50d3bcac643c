"""CPU restatement of the reference engine's greedy decoder loop, composed
from the pinned oracle kernels -- TEST INFRASTRUCTURE ONLY (tests/ use it
as the checker of the GPU decoder; no product path may import it).

Follows src/engine/decode.cu of genie-ai-runtime:
  decode step   Engine::decode_step :2101-2158 -> transformer_layer
                :1168-1246 -> transformer_layer_attn_compute :1437-1496,
                _attn_block :1498-1511, _ffn_block :1513-1522
  prefill       Path B :2779-2807 -> transformer_prefill :1760-1884, first
                token from the last prefill row :2950-2990
  sampling      sample_greedy, src/engine/sample.cpp:160-170
and the GEMV dispatch of gemv_q4.cu: gemv_quant of Q4_K / Q6_K (:1263-1290),
_pair of Q4_K+Q4_K (:1391), _triple of the four instantiated Q4_K/Q6_K
combinations (:1475-1490) and gemv_quant_f32 of Q4_K -> int8 MMVQ on the
q8_1-quantised activation; everything else (Q5_K anywhere, gemv_quant_add)
-> float dequant (gemv_quant_cpu arithmetic); gemm_quant_batched -> MMQ
for Q4_K / Q6_K with N > 1, the float Q5_K batched kernel (:1703-1762, per
token the gemv_quant_cpu arithmetic) for Q5_K, gemv_quant for N == 1.

A model is the dict of decoder.synth_np (raw GGUF block bytes as numpy).
"""
import numpy as np

import oracle


def _f16(a):
    """fp32 values -> fp16 bit patterns (RNE)."""
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def _f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def mmvq_f16(W, t, x, M, K):
    return _f16(oracle.mmvq(W, t, oracle.quantize_q8_1(x, K), M, K))


def float_f16(W, t, x, M, K):
    return _f16(oracle.gemv_quant_cpu(W, t, x, M, K, threads=None))


def pair(W0, t0, W1, t1, x, M, K):
    f = mmvq_f16 if (t0 == 12 and t1 == 12) else float_f16
    return f(W0, t0, x, M, K), f(W1, t1, x, M, K)


def triple_mmvq(t0, t1, t2):
    return (t0, t1, t2) in ((12, 12, 14), (12, 12, 12), (14, 14, 14), (14, 12, 12))


def gemv_add(W, t, x, res, M, K):
    """gemv_quant_add: half(half(W.x) + residual), float dequant."""
    proj = _f32(_f16(oracle.gemv_quant_cpu(W, t, x, M, K, threads=None)))
    return _f16(proj + _f32(res))


def gemm(W, t, x, M, N, K):
    """gemm_quant_batched: [N][M] fp16."""
    if N == 1:
        return (float_f16 if t == 13 else mmvq_f16)(W, t, x, M, K)
    if t == 13:
        xs = np.asarray(x, np.uint16).reshape(N, K)
        return np.concatenate([float_f16(W, t, xs[i], M, K) for i in range(N)])
    Npad = (N + 63) // 64 * 64
    q8 = oracle.quantize_mmq(x, N, K, Npad, t == 12)
    return _f16(oracle.mmq(W, t, q8, M, N, K, Npad)).ravel()


class OracleDecoder:
    def __init__(self, shape, model, max_seq, kv_int8=True):
        self.s, self.m = shape, model
        KV, hd = shape.n_kv_heads, shape.head_dim
        self.kc = [np.zeros((max_seq, KV, hd), np.int8) for _ in range(shape.n_layers)]
        self.vc = [np.zeros((max_seq, KV, hd), np.int8) for _ in range(shape.n_layers)]
        self.ks = [np.zeros((max_seq, KV), np.float32) for _ in range(shape.n_layers)]
        self.vs = [np.zeros((max_seq, KV), np.float32) for _ in range(shape.n_layers)]
        self.logits = None
        self.trace = None       # a list: every layer appends (layer, input, output) fp16 bits

    def _embed(self, tokens):
        s = self.s
        return np.concatenate([oracle.embed_row(self.m["tok_embd"], self.m["embd_type"], t, s.hidden_dim)
                               for t in tokens])

    def _head(self, xrow):
        s = self.s
        normed = oracle.rmsnorm(xrow, None, self.m["output_norm"], 1, s.hidden_dim, s.rms_eps, True)
        t = self.m["output_type"]
        if t == 12:
            self.logits = oracle.mmvq(self.m["output"], t, oracle.quantize_q8_1(normed, s.hidden_dim), s.vocab_size,
                                      s.hidden_dim)
        else:
            self.logits = oracle.gemv_quant_cpu(self.m["output"], t, normed, s.vocab_size, s.hidden_dim, threads=None)
        return oracle.argmax(self.logits)

    def _attn_front(self, l, L, q, k, v, start, N):
        s = self.s
        return oracle.qk_post(q, k, v, L["q_norm"], L["k_norm"], True, s.rms_eps, self.kc[l], self.vc[l],
                              self.ks[l], self.vs[l], s.n_heads, s.n_kv_heads, s.head_dim, s.head_dim, start, N,
                              s.rope_theta, True, True)

    def prefill(self, tokens, start=0):
        s = self.s
        H, QD, KVD, I = s.hidden_dim, s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim, s.intermediate_dim
        N = len(tokens)
        x = self._embed(tokens)
        for l, L in enumerate(self.m["layers"]):
            T = L["types"]
            normed = oracle.rmsnorm(x, None, L["rms_attn"], N, H, s.rms_eps, True)
            q = gemm(L["wq"], T["wq"], normed, QD, N, H)
            k = gemm(L["wk"], T["wk"], normed, KVD, N, H)
            v = gemm(L["wv"], T["wv"], normed, KVD, N, H)
            q, k = self._attn_front(l, L, q, k, v, start, N)
            attn = oracle.attn_prefill_int8(q, self.kc[l], self.vc[l], s.n_heads, s.n_kv_heads, s.head_dim,
                                            s.head_dim, N, start, 1.0 / np.sqrt(s.head_dim), self.ks[l], self.vs[l],
                                            0)
            x2 = oracle.vec_add(x, gemm(L["wo"], T["wo"], attn, H, N, QD))
            normed = oracle.rmsnorm(x2, None, L["rms_ffn"], N, H, s.rms_eps, True)
            gate = gemm(L["w_gate"], T["w_gate"], normed, I, N, H)
            up = gemm(L["w_up"], T["w_up"], normed, I, N, H)
            act = oracle.swiglu(gate, up)
            x_in, x = x, oracle.vec_add(x2, gemm(L["w_down"], T["w_down"], act, H, N, I))
            if self.trace is not None:
                self.trace.append((l, x_in, x))
        return self._head(x[(N - 1) * H:])

    def step(self, token, pos):
        s = self.s
        H, QD, KVD, I = s.hidden_dim, s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim, s.intermediate_dim
        x = self._embed([token])
        for l, L in enumerate(self.m["layers"]):
            T = L["types"]
            normed = oracle.rmsnorm(x, None, L["rms_attn"], 1, H, s.rms_eps, True)
            f = mmvq_f16 if triple_mmvq(T["wq"], T["wk"], T["wv"]) else float_f16
            q = f(L["wq"], T["wq"], normed, QD, H)
            k = f(L["wk"], T["wk"], normed, KVD, H)
            v = f(L["wv"], T["wv"], normed, KVD, H)
            q, k = self._attn_front(l, L, q, k, v, pos, 1)
            attn = oracle.attn_decode_int8(q, self.kc[l], self.vc[l], s.n_heads, s.n_kv_heads, s.head_dim,
                                           s.head_dim, pos + 1, 1.0 / np.sqrt(s.head_dim), self.ks[l], self.vs[l], 0,
                                           oracle.decode_attn_splits(pos + 1))
            x2 = gemv_add(L["wo"], T["wo"], attn, x, H, QD)
            normed = oracle.rmsnorm(x2, None, L["rms_ffn"], 1, H, s.rms_eps, True)
            gate, up = pair(L["w_gate"], T["w_gate"], L["w_up"], T["w_up"], normed, I, H)
            act = oracle.swiglu(gate, up)
            x_in, x = x, gemv_add(L["w_down"], T["w_down"], act, x2, H, I)
            if self.trace is not None:
                self.trace.append((l, x_in, x))
        return self._head(x)

    def generate(self, prompt, n_gen):
        out = [self.prefill(list(prompt))]
        for i in range(1, n_gen):
            out.append(self.step(out[-1], len(prompt) + i - 1))
        return out


# ---- one layer on a given input (per-layer checks of the GPU decoder) ----------

def prefill_front_rows(shape, L, x_rows, rows):
    """Attention front of the prefill layer at prompt positions `rows` (>= 2,
    so the projections take the MMQ path): RMSNorm, Q/K/V MMQ, q/k RMSNorm,
    RoPE, KV quantisation.  Returns (q rotated [n][QD] fp16 bits, k codes,
    v codes [n][KV][hd], k scales, v scales [n][KV])."""
    s = shape
    H, QD, KVD = s.hidden_dim, s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim
    n = len(rows)
    assert n >= 2
    T = L["types"]
    x = np.asarray(x_rows, np.uint16).reshape(n, H)
    normed = oracle.rmsnorm(x, None, L["rms_attn"], n, H, s.rms_eps, True)
    q = gemm(L["wq"], T["wq"], normed, QD, n, H).reshape(n, QD)
    k = gemm(L["wk"], T["wk"], normed, KVD, n, H).reshape(n, KVD)
    v = gemm(L["wv"], T["wv"], normed, KVD, n, H).reshape(n, KVD)
    KV, hd = s.n_kv_heads, s.head_dim
    own = (np.zeros((n, KV, hd), np.int8), np.zeros((n, KV, hd), np.int8), np.zeros((n, KV), np.float32),
           np.zeros((n, KV), np.float32))
    qr = np.empty((n, QD), np.uint16)
    for i, p in enumerate(rows):
        k1, v1 = np.zeros((1, KV, hd), np.int8), np.zeros((1, KV, hd), np.int8)
        ks1, vs1 = np.zeros((1, KV), np.float32), np.zeros((1, KV), np.float32)
        qr[i], _ = _qk_post_at(s, L, q[i], k[i], v[i], int(p), k1, v1, ks1, vs1)
        own[0][i], own[1][i], own[2][i], own[3][i] = k1[0], v1[0], ks1[0], vs1[0]
    return (qr,) + own


def prefill_attn_rows(shape, q_rows, rows, kc, vc, ks, vs):
    """Causal attention of the rotated q rows at prompt positions `rows`
    against the cache (kc, vc, ks, vs): token p attends to keys [0, p]."""
    s = shape
    return np.stack([oracle.attn_prefill_int8(q, kc, vc, s.n_heads, s.n_kv_heads, s.head_dim, s.head_dim, 1, int(p),
                                              1.0 / np.sqrt(s.head_dim), ks, vs, 0)
                     for q, p in zip(np.asarray(q_rows, np.uint16), rows)])


def prefill_o_rows(shape, L, attn_rows, x_rows):
    """x2 = x + O(attn) for n >= 2 rows (MMQ)."""
    s = shape
    H, QD = s.hidden_dim, s.n_heads * s.head_dim
    n = len(attn_rows)
    return oracle.vec_add(x_rows, gemm(L["wo"], L["types"]["wo"], attn_rows, H, n, QD)).reshape(n, H)


def prefill_ffn_rows(shape, L, x2_rows):
    """out = x2 + down(SwiGLU(gate(norm x2), up(norm x2))) for n >= 2 rows (MMQ)."""
    s = shape
    H, I = s.hidden_dim, s.intermediate_dim
    n = len(x2_rows)
    T = L["types"]
    normed = oracle.rmsnorm(x2_rows, None, L["rms_ffn"], n, H, s.rms_eps, True)
    gate = gemm(L["w_gate"], T["w_gate"], normed, I, n, H)
    up = gemm(L["w_up"], T["w_up"], normed, I, n, H)
    return oracle.vec_add(x2_rows, gemm(L["w_down"], T["w_down"], oracle.swiglu(gate, up), H, n, I)).reshape(n, H)


def prefill_layer_rows(shape, L, x_rows, rows, kc, vc, ks, vs):
    """One prefill layer (transformer_prefill, decode.cu:1760-1884) at the
    prompt positions `rows` only (>= 2 of them, so the projections take the
    MMQ path the prefill takes; every step of the layer is per token except
    the attention, whose keys come from the given cache).

    x_rows [len(rows)][H] fp16 bits: the layer's input rows at those
    positions.  kc, vc [max_seq][KV][hd] int8 and ks, vs [max_seq][KV] fp32:
    the KV cache after the layer wrote every prompt position (positions
    outside `rows` are taken as given).  Returns (out rows [len(rows)][H],
    k codes, v codes [len(rows)][KV][hd], k scales, v scales [len(rows)][KV])
    -- the oracle's own KV rows at `rows`, for comparison with the cache's."""
    x = np.asarray(x_rows, np.uint16).reshape(len(rows), shape.hidden_dim)
    q, ok, ov, oks, ovs = prefill_front_rows(shape, L, x, rows)
    attn = prefill_attn_rows(shape, q, rows, kc, vc, ks, vs)
    out = prefill_ffn_rows(shape, L, prefill_o_rows(shape, L, attn, x))
    return out, ok, ov, oks, ovs


def _qk_post_at(s, L, q, k, v, pos, k1, v1, ks1, vs1):
    """qk_post of one token at position pos (RoPE angle pos) whose KV row
    lands in the one-row cache (k1, v1, ks1, vs1): the oracle kernel indexes
    the cache by position, so it writes a cache of pos + 1 rows whose last
    row is copied out."""
    KV, hd = s.n_kv_heads, s.head_dim
    kc = np.zeros((pos + 1, KV, hd), np.int8)
    vc = np.zeros((pos + 1, KV, hd), np.int8)
    kss = np.zeros((pos + 1, KV), np.float32)
    vss = np.zeros((pos + 1, KV), np.float32)
    r = oracle.qk_post(q, k, v, L["q_norm"], L["k_norm"], True, s.rms_eps, kc, vc, kss, vss, s.n_heads, KV, hd, hd,
                       int(pos), 1, s.rope_theta, True, True)
    k1[0], v1[0], ks1[0], vs1[0] = kc[pos], vc[pos], kss[pos], vss[pos]
    return r


def decode_front(shape, L, x, pos, kc, vc, ks, vs):
    """Attention front of the decode layer for the token at position pos:
    RMSNorm, the QKV GEMV (MMVQ or float, as the triple dispatch routes),
    q/k RMSNorm, RoPE, and the KV row written into (kc, vc, ks, vs) at pos.
    Returns the rotated q [QD] fp16 bits."""
    s = shape
    H, QD, KVD = s.hidden_dim, s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim
    T = L["types"]
    normed = oracle.rmsnorm(x, None, L["rms_attn"], 1, H, s.rms_eps, True)
    f = mmvq_f16 if triple_mmvq(T["wq"], T["wk"], T["wv"]) else float_f16
    q = f(L["wq"], T["wq"], normed, QD, H)
    k = f(L["wk"], T["wk"], normed, KVD, H)
    v = f(L["wv"], T["wv"], normed, KVD, H)
    q, _ = oracle.qk_post(q, k, v, L["q_norm"], L["k_norm"], True, s.rms_eps, kc, vc, ks, vs, s.n_heads,
                          s.n_kv_heads, s.head_dim, s.head_dim, pos, 1, s.rope_theta, True, True)
    return q


def decode_attn(shape, q, pos, kc, vc, ks, vs):
    s = shape
    return oracle.attn_decode_int8(q, kc, vc, s.n_heads, s.n_kv_heads, s.head_dim, s.head_dim, pos + 1,
                                   1.0 / np.sqrt(s.head_dim), ks, vs, 0, oracle.decode_attn_splits(pos + 1))


def decode_o(shape, L, attn, x):
    """x2 = half(half(O . attn) + x), float dequant (gemv_quant_add)."""
    return gemv_add(L["wo"], L["types"]["wo"], attn, x, shape.hidden_dim, shape.n_heads * shape.head_dim)


def decode_ffn(shape, L, x2):
    s = shape
    H, I = s.hidden_dim, s.intermediate_dim
    T = L["types"]
    normed = oracle.rmsnorm(x2, None, L["rms_ffn"], 1, H, s.rms_eps, True)
    gate, up = pair(L["w_gate"], T["w_gate"], L["w_up"], T["w_up"], normed, I, H)
    return gemv_add(L["w_down"], T["w_down"], oracle.swiglu(gate, up), x2, H, I)


def decode_layer(shape, L, x, pos, kc, vc, ks, vs):
    """One decode-step layer (transformer_layer, decode.cu:1168-1246) for the
    token at position pos with input x [H] fp16 bits, over the KV cache
    (kc, vc, ks, vs) whose positions < pos are taken as given; the oracle
    writes row pos of these arrays itself (they are updated in place).
    Returns the layer's output [H] fp16 bits -- the computation of
    OracleDecoder.step for one layer."""
    q = decode_front(shape, L, x, pos, kc, vc, ks, vs)
    return decode_ffn(shape, L, decode_o(shape, L, decode_attn(shape, q, pos, kc, vc, ks, vs), x))


class perturbed_matmuls:
    """Context manager: every matmul output of the oracle (MMQ, MMVQ, float
    GEMV) is multiplied by (1 + rel * N(0, 1)) -- the size of the fp32
    summation-order differences between two correct implementations.  Used to
    measure how far the decoder's logits move under such differences (the
    int8 KV and q8 activation codes flip on ulp-level changes, and layers
    amplify the flips), which sets the parity bar of long generations."""

    NAMES = ("mmq", "mmvq", "gemv_quant_cpu")

    def __init__(self, seed, rel=1e-6):
        self.rng = np.random.default_rng(seed)
        self.rel = rel
        self.saved = {}

    def __enter__(self):
        for name in self.NAMES:
            fn = getattr(oracle, name)
            self.saved[name] = fn

            def wrapped(*a, _fn=fn, **kw):
                y = _fn(*a, **kw)
                return (y * (1.0 + self.rel * self.rng.standard_normal(y.shape))).astype(np.float32)
            setattr(oracle, name, wrapped)
        return self

    def __exit__(self, *exc):
        for name, fn in self.saved.items():
            setattr(oracle, name, fn)
        return False
