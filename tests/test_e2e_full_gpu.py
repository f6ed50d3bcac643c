"""configs[4] at full size: the random-init Qwen3-4B-shaped Q4_K_M decoder
(36 layers, hidden 2560, 32/8 heads, head_dim 128, FFN 9728, vocab 151936,
INT8 KV), a 512-token prompt and 128 greedy tokens, through the decoder's C
ABI, against the CPU oracle's generation committed in
tests/golden/e2e_qwen3_4b.npz (tests/golden/make_e2e_golden.py: the same
seeded model and prompt, oracle/decoder_oracle.py -- the reference engine's
generate / prefill / decode loop, decode.cu:2779-3099, sample.cpp:160-184).

The generation is numerically chaotic: int8 KV codes and q8 activation
codes flip on ulp-level differences and 36 layers amplify the flips.  The
golden files e2e_qwen3_4b_env1/2.npz hold how far the ORACLE's own logits
move, position by position, when 1e-6 relative noise (the size of fp32
summation-order differences) is put on its matmul outputs: ~15 % of
max|logits| after the 512-token prefill, ~2-3 % per decode step.

Bars:
* teacher forcing (the oracle's tokens fed to the GPU decoder): at every one
  of the 128 positions the fp32 logits at 512 fixed vocabulary indices and
  the top-8 logits are within bar_i = max(1e-2 * max|logits|, 2 x the
  larger of the two envelopes at that position) of the oracle's, and the
  greedy token is the oracle's wherever the oracle's top-2 margin exceeds
  bar_i;
* free-running generation on the device: the tokens equal the oracle's up
  to the first position whose top-2 margin is within the larger envelope
  there (a tie at the precision any two correct implementations agree to;
  twice the envelope, the logit bar, already exceeds the margin at position
  0, where the prefill's envelope is ~15 % of max|logits|);
* drift ceilings on the same teacher-forced deviations: their median over
  the 128 positions at most MEDIAN_ENV_RATIO times the envelope, and at
  every decode position at most DECODE_ENV_RATIO times it (no 1e-2 floor);
* each of the 36 layers alone, at full size, on the GPU's own input: stage
  by stage and as a whole against the oracle's layer on the same input and
  KV cache (the tests at the end of this file) -- free of the 36-layer
  amplification.
"""
import os

import numpy as np
import pytest
import torch

import decoder
import decoder_oracle
import jllm
import oracle
from gpu_util import f16_to_f64, from_dev, print_case

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "e2e_qwen3_4b.npz")
TOL = 1e-2
MEDIAN_ENV_RATIO = 1.25
DECODE_ENV_RATIO = 2.0


def _golden():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_e2e_golden", os.path.join(HERE, "golden",
                                                                                   "make_e2e_golden.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    return mk, np.load(GOLDEN)


@pytest.fixture(scope="module")
def full_model(dev):
    mk, gold = _golden()
    shape = decoder.QWEN3_4B
    print_case("e2e full: synthesising the 36-layer model")
    model_np = decoder.synth_np(shape, int(gold["model_seed"]))
    model = decoder.to_device(model_np, dev)
    torch.cuda.synchronize()
    prompt = mk.prompt_ids(shape.vocab_size)
    assert np.array_equal(prompt, gold["prompt"])
    yield shape, model, prompt, gold, model_np
    del model, model_np
    torch.cuda.empty_cache()


def _envelope():
    return np.maximum(np.load(os.path.join(HERE, "golden", "e2e_qwen3_4b_env1.npz"))["deviation"],
                      np.load(os.path.join(HERE, "golden", "e2e_qwen3_4b_env2.npz"))["deviation"])


def _bars(gold):
    return np.maximum(TOL * gold["absmax"], 2.0 * _envelope())


@pytest.fixture(scope="module")
def teacher_forced(dev, full_model):
    """Per position: the GPU logits' largest deviation from the oracle's (512
    sampled + top-8 indices) and the GPU argmax, the oracle's tokens fed."""
    shape, model, prompt, gold, _ = full_model
    n_prompt, n_gen = prompt.size, gold["tokens"].size
    d = decoder.Decoder(shape, model, n_prompt + n_gen, max_batch=n_prompt)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    toks = torch.tensor(gold["tokens"], dtype=torch.int32, device=dev)
    print_case("e2e full: prefill + 127 teacher-forced steps")
    devs, amax = [], []
    d.prefill(torch.from_numpy(prompt).to(dev), 0, out)
    for i in range(n_gen):
        if i > 0:
            d.step(toks[i - 1:i], n_prompt + i - 1, out)
        lg = from_dev(d.logits())
        devs.append(max(float(np.abs(lg[gold["sample_idx"]] - gold["sample"][i]).max()),
                        float(np.abs(lg[gold["top_idx"][i]] - gold["top_val"][i]).max())))
        amax.append(int(np.argmax(lg)))
    d.close()
    return np.array(devs), np.array(amax)


def test_e2e_teacher_forced_logits(full_model, teacher_forced):
    _, _, _, gold, _ = full_model
    devs, amax = teacher_forced
    bars = _bars(gold)
    bad = np.nonzero(devs > bars)[0]
    assert bad.size == 0, [(int(i), float(devs[i]), float(bars[i])) for i in bad[:8]]
    clear = gold["margin"] > bars
    wrong = np.nonzero(clear & (amax != gold["tokens"]))[0]
    assert wrong.size == 0, [(int(i), float(gold["margin"][i])) for i in wrong]
    env = _envelope()
    r = devs / env
    print_case("e2e full: deviation / envelope per position: median %.3f, decode positions p50 %.3f p90 %.3f max "
               "%.3f; deviation / max|logits| at decode positions p50 %.4f max %.4f"
               % (float(np.median(r)), float(np.median(r[1:])), float(np.percentile(r[1:], 90)), float(r[1:].max()),
                  float(np.median(devs[1:] / gold["absmax"][1:])), float((devs[1:] / gold["absmax"][1:]).max())))
    # drift ceilings (measured: median 0.89, decode positions at most 1.58):
    # the typical deviation stays at the size of the oracle's own envelope,
    # and at the decode positions every one stays within twice it, with no
    # 1e-2 floor
    assert float(np.median(r)) <= MEDIAN_ENV_RATIO, float(np.median(r))
    assert float(r[1:].max()) <= DECODE_ENV_RATIO, float(r[1:].max())
    print_case(f"e2e full: worst logit deviation {float((devs / gold['absmax']).max()):.3f} of max|logits|, "
               f"median ratio to the oracle's own envelope {float(np.median(devs / (bars / 2))):.2f}; "
               f"argmax equal at {int((amax == gold['tokens']).sum())} of {amax.size} positions")


def test_e2e_free_running_tokens(dev, full_model):
    shape, model, prompt, gold, _ = full_model
    n_prompt, n_gen = prompt.size, gold["tokens"].size
    d = decoder.Decoder(shape, model, n_prompt + n_gen, max_batch=n_prompt)
    gen = torch.zeros(n_gen, dtype=torch.int32, device=dev)
    print_case("e2e full: generate")
    d.generate(torch.from_numpy(prompt).to(dev), n_gen, gen)
    got = from_dev(gen)
    d.close()
    ties = np.nonzero(gold["margin"] <= _envelope())[0]
    t0 = int(ties[0]) if ties.size else n_gen             # up to the first near-tie, if any
    assert t0 > 0
    assert np.array_equal(got[:t0], gold["tokens"][:t0]), (t0, got[:16], gold["tokens"][:16])
    same = int(np.argmin(np.append(got == gold["tokens"], False)))
    print_case(f"e2e full: tokens equal to the oracle's for the first {same} positions "
               f"({t0} required: first near-tie at {t0})")


# ---- each layer at full size on its own input ------------------------------------------
#
# The 36 layers of the GPU decoder run one at a time (jllm_hip_decoder_layer)
# on the GPU's own hidden state, and each is compared with the oracle's layer
# on THE SAME input and KV cache, so no comparison goes through the 36-layer
# amplification.  Two kinds of check per layer:
#
# * stage by stage -- the oracle's attention front (q after norm + RoPE, the
#   KV row), attention, O + residual and FFN + residual, each fed the GPU's
#   output of the stage before it (jllm_hip_decoder_copy_act), within
#   STAGE_TOL of the stage output's max|.|: one matmul's arithmetic and at
#   most two fp16 / q8 rounding steps apart (measured worst: q 1.56e-3, FFN
#   1.26e-3 in the prefill; 9.1e-4 in the decode step);
# * the whole layer from its input, within WHOLE_ENV_X times the oracle's
#   own one-layer envelope -- the largest change of the oracle's output when
#   every matmul output carries 1e-6 relative noise (two seeds), measured on
#   the same input in the test -- and, for the decode step, within
#   DECODE_TOL = 1e-3 of max|out| as well (measured worst 8.6e-4).  The
#   prefill layer cannot be held to 1e-3: a 1e-6 change of q flips fp16
#   roundings and q8 codes downstream, and the oracle's own prefill layers
#   move by 0.4-3.0e-3 of max|out| under that noise (1-4 fp16 ulps of the
#   largest element); the GPU's errors are 1.0-2.2 times that envelope.
#
# The kernels are deterministic, so these numbers repeat run to run.

STAGE_TOL = 2e-3
WHOLE_ENV_X = 3.0
DECODE_TOL = 1e-3
KV_SCALE_TOL = 2e-3
KV_FLIP_FRAC = 0.05
# prompt positions whose whole layer is recomputed by the oracle (first,
# last, and spread between; the attention of each reads all earlier keys)
ROWS = [0, 1, 2, 31, 64, 127, 128, 200, 255, 256, 300, 383, 384, 449, 510, 511]


def _kv_close(gk, gv, gks, gvs, ok, ov, oks, ovs):
    dk = np.abs(gk.astype(np.int32) - ok.astype(np.int32))
    dv = np.abs(gv.astype(np.int32) - ov.astype(np.int32))
    sc = max(float(np.abs(g.astype(np.float64) - o).max() / np.abs(o).max()) for g, o in ((gks, oks), (gvs, ovs)))
    return max(int(dk.max()), int(dv.max())), max(float((dk > 0).mean()), float((dv > 0).mean())), sc


def _rel(got_bits, want_bits):
    g, w = f16_to_f64(got_bits), f16_to_f64(want_bits)
    return float(np.abs(g - w).max() / np.abs(w).max())


def _envelope_of(fn):
    """Largest relative (infinity-norm) change of fn()'s fp16 output when every
    matmul output of the oracle carries 1e-6 relative noise, two seeds."""
    ref = fn()
    env = 0.0
    for seed in (1, 2):
        with decoder_oracle.perturbed_matmuls(seed):
            env = max(env, _rel(fn(), ref))
    return ref, env


def _report(kind, stats, whole_cap=None):
    print_case(kind)
    for l, st in enumerate(stats):
        print("  layer %2d " % l + " ".join("%s=%.3g" % kv for kv in st.items()), flush=True)
    bad = [(l, k, v) for l, st in enumerate(stats) for k, v in st.items()
           if (k.startswith("st_") and v > STAGE_TOL)
           or (k == "whole" and (v > WHOLE_ENV_X * st["env"] or (whole_cap is not None and v > whole_cap)))
           or (k == "kv_code" and v > 1) or (k == "kv_flip" and v >= KV_FLIP_FRAC) or (k == "kv_scale" and v > KV_SCALE_TOL)]
    assert not bad, bad


@pytest.fixture(scope="module")
def layer_decoder(dev, full_model):
    shape, model, prompt, gold, _ = full_model
    oracle.set_threads(min(16, os.cpu_count() or 1))
    d = decoder.Decoder(shape, model, prompt.size + gold["tokens"].size, max_batch=prompt.size)
    yield d
    d.close()


def test_e2e_each_layer_prefill_full_size(dev, full_model, layer_decoder):
    """The 512-token prefill, one layer at a time, at the Qwen3-4B shape."""
    shape, model, prompt, gold, model_np = full_model
    d, H, n = layer_decoder, shape.hidden_dim, prompt.size
    x = torch.empty(n * H, dtype=torch.int16, device=dev)
    jllm.call("jllm_hip_dequant_embedding_rows", x, model["tok_embd"], model["embd_type"],
              torch.from_numpy(prompt).to(dev), n, H, shape.vocab_size)
    emb = from_dev(x).view(np.uint16).reshape(n, H)
    want = np.stack([oracle.embed_row(model_np["tok_embd"], model_np["embd_type"], int(t), H) for t in prompt])
    assert np.array_equal(emb, want)
    stats = []
    for l in range(shape.n_layers):
        print_case("e2e layer prefill", l)
        L = model_np["layers"][l]
        x_in = from_dev(x).view(np.uint16).reshape(n, H)[ROWS]
        d.layer(l, x, n, 0)
        x_out = from_dev(x).view(np.uint16).reshape(n, H)[ROWS]
        g_q, g_attn, g_x2 = (d.act(w, n)[ROWS] for w in range(3))
        kc, vc, ks, vs = d.kv(l, n)
        q, ok, ov, oks, ovs = decoder_oracle.prefill_front_rows(shape, L, x_in, ROWS)
        code, flip, scl = _kv_close(kc[ROWS], vc[ROWS], ks[ROWS], vs[ROWS], ok, ov, oks, ovs)
        whole, env = _envelope_of(lambda: decoder_oracle.prefill_layer_rows(shape, L, x_in, ROWS, kc, vc, ks, vs)[0])
        stats.append({
            "st_q": _rel(g_q, q),
            "st_attn": _rel(g_attn, decoder_oracle.prefill_attn_rows(shape, g_q, ROWS, kc, vc, ks, vs)),
            "st_o": _rel(g_x2, decoder_oracle.prefill_o_rows(shape, L, g_attn, x_in)),
            "st_ffn": _rel(x_out, decoder_oracle.prefill_ffn_rows(shape, L, g_x2)),
            "whole": _rel(x_out, whole), "env": env, "kv_code": code, "kv_flip": flip, "kv_scale": scl})
    _report("e2e layer prefill (rows %s)" % ROWS, stats)


def test_e2e_each_layer_decode_full_size(dev, full_model, layer_decoder):
    """One decode step at context 639 (the 128th generated token's step),
    one layer at a time; the KV cache holds the prefill and 126
    teacher-forced decode steps of the oracle's tokens."""
    shape, model, prompt, gold, model_np = full_model
    d, H, n = layer_decoder, shape.hidden_dim, prompt.size
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    toks = torch.tensor(gold["tokens"], dtype=torch.int32, device=dev)
    print_case("e2e layer decode: prefill + 126 teacher-forced steps")
    d.prefill(torch.from_numpy(prompt).to(dev), 0, out)
    n_gen = gold["tokens"].size
    for i in range(1, n_gen - 1):
        d.step(toks[i - 1:i], n + i - 1, out)
    pos = n + n_gen - 2                                   # 638: the step that produces the last token
    x = torch.empty(H, dtype=torch.int16, device=dev)
    jllm.call("jllm_hip_dequant_embedding_rows", x, model["tok_embd"], model["embd_type"], toks[n_gen - 2:n_gen - 1],
              1, H, shape.vocab_size)
    stats = []
    for l in range(shape.n_layers):
        print_case("e2e layer decode", l, "pos", pos)
        L = model_np["layers"][l]
        x_in = from_dev(x).view(np.uint16).copy()
        prev = [np.concatenate([a, np.zeros((1,) + a.shape[1:], a.dtype)]) for a in d.kv(l, pos)]
        d.layer(l, x, 1, pos)
        x_out = from_dev(x).view(np.uint16)
        g_q, g_attn, g_x2 = (d.act(w, 1)[0] for w in range(3))
        gkv = d.kv(l, pos + 1)                            # the GPU's cache, its own row pos included
        kc, vc, ks, vs = (a.copy() for a in prev)
        q = decoder_oracle.decode_front(shape, L, x_in, pos, kc, vc, ks, vs)
        code, flip, scl = _kv_close(*(a[pos:] for a in gkv), kc[pos:], vc[pos:], ks[pos:], vs[pos:])

        def whole_layer():
            c = [a.copy() for a in prev]
            return decoder_oracle.decode_layer(shape, L, x_in, pos, *c)
        whole, env = _envelope_of(whole_layer)
        stats.append({
            "st_q": _rel(g_q, q),
            "st_attn": _rel(g_attn, decoder_oracle.decode_attn(shape, g_q, pos, *gkv)),
            "st_o": _rel(g_x2, decoder_oracle.decode_o(shape, L, g_attn, x_in)),
            "st_ffn": _rel(x_out, decoder_oracle.decode_ffn(shape, L, g_x2)),
            "whole": _rel(x_out, whole), "env": env, "kv_code": code, "kv_flip": flip, "kv_scale": scl})
    _report("e2e layer decode (pos %d)" % pos, stats, whole_cap=DECODE_TOL)
