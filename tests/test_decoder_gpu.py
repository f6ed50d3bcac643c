"""GPU parity of the decoder loop (jllm_hip_decoder_*): random Q4_K_M and
Q5_K_M-style models run through the C ABI against the CPU restatement of the reference
engine's layer order (oracle/decoder_oracle.py).

Bars: with the oracle's tokens fed back (teacher forcing) every step's fp32
logits are within max(1e-2, 2 x envelope) * max|logits| of the oracle's,
where the envelope is how far the oracle's own logits move when 1e-6
relative noise (fp32 summation-order size) is put on its matmul outputs --
the int8 KV and q8 activation codes flip on ulp-level differences and the
layers amplify the flips, ~0 for short prompts, ~2 % for a 300-token one;
the greedy tokens of a free-running generation are identical to the
oracle's up to the first position whose top-2 margin is under that bar;
the chunked prefill and the one-call generate() are bit-identical to the
plain prefill / steps.
"""
import os

import numpy as np
import pytest
import torch

import decoder
import decoder_oracle
import synth
from gpu_util import from_dev, print_case

pytestmark = pytest.mark.gpu
TOL = 1e-2

TINY = decoder.Shape(n_layers=2, hidden_dim=512, n_heads=8, n_kv_heads=2, head_dim=64, intermediate_dim=1024,
                     vocab_size=1000)
# Qwen3-4B widths and vocabulary, 2 of the 36 layers (one Q6_K and one Q4_K down)
WIDE = decoder.Shape(n_layers=2)


def _tok(a, dev):
    return torch.tensor(np.asarray(a, np.int32), dtype=torch.int32, device=dev)


def _rel(got, want):
    return float(np.abs(got - want).max() / np.abs(want).max())


def _envelope(shape, model, prompt, tokens, max_seq):
    """Largest logit deviation / max|logits| of the oracle itself under
    1e-6 relative noise on its matmul outputs, teacher-forced with `tokens`
    (the generation is chaotic: see decoder_oracle.perturbed_matmuls)."""
    base, pert = decoder_oracle.OracleDecoder(shape, model, max_seq), decoder_oracle.OracleDecoder(shape, model, max_seq)
    base.prefill(list(prompt))
    with decoder_oracle.perturbed_matmuls(seed=len(prompt)):
        pert.prefill(list(prompt))
    env = [_rel(pert.logits, base.logits)]
    for i in range(1, len(tokens)):
        base.step(tokens[i - 1], len(prompt) + i - 1)
        with decoder_oracle.perturbed_matmuls(seed=len(prompt) + i):
            pert.step(tokens[i - 1], len(prompt) + i - 1)
        env.append(_rel(pert.logits, base.logits))
    return max(env)


# (WIDE, 300 tokens): the prefill's gate/up GEMMs run as one multi-product
# launch (>= 384 tiles) and the decode steps use multi-split attention
@pytest.mark.parametrize("shape,n_prompt,n_gen,seed,preset", [(TINY, 20, 8, 1, "q4km"), (TINY, 1, 4, 2, "q4km"),
                                                               (WIDE, 6, 3, 3, "q4km"), (TINY, 20, 6, 4, "q5km"),
                                                               (WIDE, 5, 3, 5, "q5km"), (WIDE, 300, 4, 6, "q4km")])
def test_decoder_vs_oracle(dev, shape, n_prompt, n_gen, seed, preset):
    """Logit bar: max(1e-2, 2 x the oracle's own deviation under 1e-6
    matmul noise) x max|logits| -- for short prompts the envelope is ~0 and
    the bar is 1e-2; a 300-token prompt moves the oracle itself by ~2 %.
    Greedy tokens: the oracle's wherever its top-2 margin exceeds the bar."""
    print_case("decoder", shape.hidden_dim, shape.n_layers, n_prompt, n_gen, preset)
    import oracle
    oracle.set_threads(min(16, os.cpu_count() or 1))
    model = decoder.synth_np(shape, seed, preset)
    prompt = synth.rng(seed + 100).integers(0, shape.vocab_size, n_prompt).astype(np.int32)
    max_seq = n_prompt + n_gen
    orc = decoder_oracle.OracleDecoder(shape, model, max_seq)
    want_tok, want_logits = [orc.prefill(list(prompt))], [orc.logits.copy()]
    for i in range(1, n_gen):
        want_tok.append(orc.step(want_tok[-1], n_prompt + i - 1))
        want_logits.append(orc.logits.copy())
    bar = max(TOL, 2.0 * _envelope(shape, model, prompt, want_tok, max_seq))
    dm = decoder.to_device(model, dev)
    gpu = decoder.Decoder(shape, dm, max_seq, max_batch=512)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    # teacher-forced: the oracle's token drives both
    tie = n_gen
    for i in range(n_gen):
        if i == 0:
            gpu.prefill(_tok(prompt, dev), 0, out)
        else:
            gpu.step(_tok([want_tok[i - 1]], dev), n_prompt + i - 1, out)
        lg, w = from_dev(gpu.logits()), want_logits[i]
        assert _rel(lg, w) <= bar, (i, _rel(lg, w), bar)
        top2 = np.sort(w)[-2:]
        if top2[1] - top2[0] > bar * np.abs(w).max():
            assert int(np.argmax(lg)) == want_tok[i], i
        else:
            tie = min(tie, i)
    # free-running greedy generation on the device: identical tokens up to a near-tie
    gpu2 = decoder.Decoder(shape, dm, max_seq, max_batch=512)
    gen = torch.zeros(n_gen, dtype=torch.int32, device=dev)
    gpu2.generate(_tok(prompt, dev), n_gen, gen)
    assert from_dev(gen).tolist()[:tie] == want_tok[:tie]
    gpu.close()
    gpu2.close()


def test_decoder_chunked_prefill_and_generate_bit_identical(dev):
    print_case("decoder chunking")
    shape = TINY
    model = decoder.to_device(decoder.synth_np(shape, 5), dev)
    prompt = _tok(synth.rng(6).integers(0, shape.vocab_size, 40), dev)
    n_gen = 5
    runs = []
    for max_batch in (64, 16, 7):
        d = decoder.Decoder(shape, model, 48, max_batch=max_batch)
        gen = torch.zeros(n_gen, dtype=torch.int32, device=dev)
        d.generate(prompt, n_gen, gen)
        runs.append((from_dev(gen).tolist(), from_dev(d.logits())))
        d.close()
    for toks, lg in runs[1:]:
        assert toks == runs[0][0] and np.array_equal(lg, runs[0][1])
    # generate() == prefill + explicit steps
    d = decoder.Decoder(shape, model, 48, max_batch=64)
    t = torch.zeros(n_gen, dtype=torch.int32, device=dev)
    d.prefill(prompt, 0, t[0:1])
    for i in range(1, n_gen):
        d.step(t[i - 1:i], 40 + i - 1, t[i:i + 1])
    assert from_dev(t).tolist() == runs[0][0]
    d.close()


def test_decoder_prefill_chunk_of_one_token(dev):
    """A prefill whose last chunk holds one token (40 = 3 x 13 + 1): that
    chunk's layers take the single-row forms (the products of one row are
    the reference's GEMVs, whose O / down activations are not q8_1-quantised)
    at start 39 against KV written by the batched chunks.  Its logits match
    the oracle prefilled in the same chunks within the decoder bar (the
    whole-prompt prefill differs by the GEMV-vs-MMQ activation rounding, ~2 %
    on this shape), and the KV rows of the batched chunks are the bytes of the
    whole-prompt prefill."""
    print_case("decoder chunk of one")
    import oracle
    oracle.set_threads(min(16, os.cpu_count() or 1))
    shape = TINY
    model_np = decoder.synth_np(shape, 7)
    model = decoder.to_device(model_np, dev)
    prompt = synth.rng(8).integers(0, shape.vocab_size, 40).astype(np.int32)
    res = []
    for max_batch in (64, 13):
        d = decoder.Decoder(shape, model, 48, max_batch=max_batch)
        t = torch.zeros(1, dtype=torch.int32, device=dev)
        d.prefill(_tok(prompt, dev), 0, t)
        res.append((int(from_dev(t)[0]), from_dev(d.logits()), d.kv(0, 39) + d.kv(1, 39)))
        d.close()
    (_, _, kv0), (t1, lg1, kv1) = res
    for a, b in zip(kv0, kv1):
        assert np.array_equal(a, b)
    orc = decoder_oracle.OracleDecoder(shape, model_np, 48)
    for c0 in range(0, 40, 13):
        want_tok = orc.prefill(list(prompt[c0:c0 + 13]), c0)
    want = orc.logits
    assert _rel(lg1, want) <= TOL, _rel(lg1, want)
    top2 = np.sort(want)[-2:]
    if top2[1] - top2[0] > TOL * np.abs(want).max():
        assert t1 == want_tok


def test_decoder_rejects_bad_config(dev):
    shape = TINY
    model = decoder.to_device(decoder.synth_np(shape, 9), dev)
    bad = dict(model)
    bad["layers"] = [dict(L) for L in model["layers"]]
    bad["layers"][1]["types"] = dict(bad["layers"][1]["types"], w_up=15)
    with pytest.raises(Exception):
        decoder.Decoder(shape, bad, 16)
    d = decoder.Decoder(shape, model, 16)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(Exception):
        d.prefill(_tok(np.zeros(17), dev), 0, out)           # past max_seq
    d.close()


@pytest.mark.parametrize("preset,N,tiny,start", [("q4km", 512, False, 0), ("q4km", 500, False, 0),
                                                 ("q4km", 300, False, 0), ("q4km", 64, False, 0),
                                                 ("q5km", 300, False, 0), ("q4km", 40, True, 0),
                                                 ("q4km", 512, False, 512), ("q4km", 64, False, 300),
                                                 ("q4km_mixed", 512, False, 0), ("q4km_mixed", 300, False, 0)])
def test_decoder_prefill_layer_equals_c_abi_composition(dev, preset, N, tiny, start):
    """One prefill layer of the decoder (whose residual adds, RMSNorms and
    activation quantisation run fused, one pass per norm) is bit-identical to
    the same layer composed from the separate C-ABI entry points in the
    reference engine's order (transformer_layer, decode.cu:1760-1884):
    RMSNorm, Q/K/V GEMM, q/k norm + RoPE + KV store, attention, O GEMM,
    residual add, RMSNorm, gate/up GEMM, SwiGLU, down GEMM, residual add.
    Cases: 512 and 500 tokens take every fused form (RMSNorm rows with the
    codes, the attention front in the Q/K/V GEMM, the O codes in the
    attention, the SwiGLU codes in the gate/up GEMM; 500 with a partial
    last token tile); 300 and 64 tokens the smaller grids without the GEMM
    epilogue forms; the Q5_K_M-style layer the fp16 GEMM; the tiny shape
    (hidden 512, head_dim 64) the one-wave RMSNorm rows; the mixed layers
    (Q6_K V / O) the fp16 codes of the RMSNorm rows and of the attention
    output next to the int8 ones.  With start > 0 a
    first chunk of `start` tokens fills the KV rows before the checked chunk
    of N tokens at positions start.. (RoPE positions and KV rows offset, the
    attention over the earlier rows)."""
    import ctypes
    import jllm
    print_case("prefill layer composition", preset, N, tiny, start)
    shape = TINY if tiny else WIDE
    H, QD, KVD, I = shape.hidden_dim, shape.n_heads * shape.head_dim, shape.n_kv_heads * shape.head_dim, \
        shape.intermediate_dim
    model = decoder.to_device(decoder.synth_np(shape, 21, preset), dev)
    T = start + N
    d = decoder.Decoder(shape, model, T, max_batch=512)
    g = synth.rng(22)
    xs = [torch.from_numpy(synth.x_f16(g, n * H).view(np.int16)).to(dev) for n in ((start, N) if start else (N,))]

    def e(n, dtype=torch.int16):
        return torch.empty(n, dtype=dtype, device=dev)
    for l in (0, 1):                                  # Q6_K and Q4_K down (q4km)
        L = model["layers"][l]
        t = L["types"]
        kc, vc = e(T * KVD, torch.int8), e(T * KVD, torch.int8)
        ks, vs = e(T * shape.n_kv_heads, torch.float32), e(T * shape.n_kv_heads, torch.float32)

        def multi(ys, names, x, n_tok, K):
            n = len(ys)
            yp = (ctypes.c_void_p * n)(*[a.data_ptr() for a in ys])
            wp = (ctypes.c_void_p * n)(*[L[m].data_ptr() for m in names])
            tp = (ctypes.c_int * n)(*[t[m] for m in names])
            mp = (ctypes.c_int * n)(*[shape.mat_shape(m)[0] for m in names])
            jllm.call("jllm_hip_gemm_quant_batched_multi", yp, wp, tp, mp, n, x, n_tok, K)

        def compose(x0, n, p0):
            normed, q, k, v, attn, x2, gate, up, act, y = (e(m) for m in (n * H, n * QD, n * KVD, n * KVD, n * QD,
                                                                          n * H, n * I, n * I, n * I, n * H))
            jllm.call("jllm_hip_fused_rmsnorm_residual", normed, x0, None, L["rms_attn"], n, H, shape.rms_eps, 1)
            multi([q, k, v], ["wq", "wk", "wv"], normed, n, H)
            kv_off, sc_off = p0 * KVD, p0 * shape.n_kv_heads
            jllm.call("jllm_hip_qk_norm_rope_store_kv", q, k, v, L["q_norm"], L["k_norm"], 1, shape.rms_eps,
                      kc.data_ptr() + kv_off, vc.data_ptr() + kv_off, ks.data_ptr() + 4 * sc_off,
                      vs.data_ptr() + 4 * sc_off, KVD, shape.n_heads, shape.n_kv_heads, shape.head_dim,
                      shape.head_dim, p0, n, shape.rope_theta, 1, 1)
            jllm.call("jllm_hip_flash_attention_prefill_batched", attn, q, kc, vc, shape.n_heads, shape.n_kv_heads,
                      shape.head_dim, shape.head_dim, n, p0, 1.0 / np.sqrt(shape.head_dim), 1, ks, vs, 0)
            jllm.call("jllm_hip_gemm_quant_batched", x2, L["wo"], t["wo"], attn, H, n, QD)
            jllm.call("jllm_hip_vec_add", x2, x2, x0, n * H)
            jllm.call("jllm_hip_fused_rmsnorm_residual", normed, x2, None, L["rms_ffn"], n, H, shape.rms_eps, 1)
            multi([gate, up], ["w_gate", "w_up"], normed, n, H)
            jllm.call("jllm_hip_fused_swiglu", act, gate, up, n, I)
            jllm.call("jllm_hip_gemm_quant_batched", y, L["w_down"], t["w_down"], act, H, n, I)
            jllm.call("jllm_hip_vec_add", y, y, x2, n * H)
            return x2, y

        p0 = 0
        for x0 in xs:
            n = x0.numel() // H
            xd = x0.clone()
            d.layer(l, xd, n, p0)
            x2, y = compose(x0, n, p0)
            p0 += n
        kd = d.kv(l, T)
        assert np.array_equal(from_dev(kc).reshape(kd[0].shape), kd[0]) and \
            np.array_equal(from_dev(vc).reshape(kd[1].shape), kd[1])
        assert np.array_equal(from_dev(ks).reshape(kd[2].shape), kd[2]) and \
            np.array_equal(from_dev(vs).reshape(kd[3].shape), kd[3])
        assert np.array_equal(from_dev(x2).view(np.uint16).reshape(N, H), d.act(2, N)), l
        assert np.array_equal(from_dev(y), from_dev(xd)), l
    d.close()
