"""GPU parity of the decoder loop (jllm_hip_decoder_*): random Q4_K_M and
Q5_K_M-style models run through the C ABI against the CPU restatement of the reference
engine's layer order (oracle/decoder_oracle.py).

Bars: the greedy tokens of a free-running generation are identical to the
oracle's; with the oracle's tokens fed back (teacher forcing) every step's
fp32 logits are within 1e-2 * max|logits| of the oracle's -- the fp16
activations of ~15 rounded stages per layer may differ by an ulp here and
there, as each kernel's own parity test allows; the chunked prefill and
the one-call generate() are bit-identical to the plain prefill / steps.
"""
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


@pytest.mark.parametrize("shape,n_prompt,n_gen,seed,preset", [(TINY, 20, 8, 1, "q4km"), (TINY, 1, 4, 2, "q4km"),
                                                               (WIDE, 6, 3, 3, "q4km"), (TINY, 20, 6, 4, "q5km"),
                                                               (WIDE, 5, 3, 5, "q5km")])
def test_decoder_vs_oracle(dev, shape, n_prompt, n_gen, seed, preset):
    print_case("decoder", shape.hidden_dim, shape.n_layers, n_prompt, n_gen, preset)
    model = decoder.synth_np(shape, seed, preset)
    prompt = synth.rng(seed + 100).integers(0, shape.vocab_size, n_prompt).astype(np.int32)
    max_seq = n_prompt + n_gen
    orc = decoder_oracle.OracleDecoder(shape, model, max_seq)
    dm = decoder.to_device(model, dev)
    gpu = decoder.Decoder(shape, dm, max_seq, max_batch=64)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    # teacher-forced: the oracle's token drives both
    want_tok = [orc.prefill(list(prompt))]
    gpu.prefill(_tok(prompt, dev), 0, out)
    assert _rel(from_dev(gpu.logits()), orc.logits) <= TOL
    for i in range(1, n_gen):
        want_tok.append(orc.step(want_tok[-1], n_prompt + i - 1))
        gpu.step(_tok([want_tok[-2]], dev), n_prompt + i - 1, out)
        assert _rel(from_dev(gpu.logits()), orc.logits) <= TOL, i
    # free-running greedy generation on the device: identical tokens
    gpu2 = decoder.Decoder(shape, dm, max_seq, max_batch=64)
    gen = torch.zeros(n_gen, dtype=torch.int32, device=dev)
    gpu2.generate(_tok(prompt, dev), n_gen, gen)
    assert from_dev(gen).tolist() == want_tok
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
