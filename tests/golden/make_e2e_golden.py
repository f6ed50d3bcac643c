"""Writes tests/golden/e2e_qwen3_4b.npz: the CPU oracle's greedy generation
for the end-to-end configuration at FULL size -- a random-init
Qwen3-4B-shaped Q4_K_M decoder (36 layers, hidden 2560, 32/8 heads,
head_dim 128, FFN 9728, vocab 151936, INT8 KV), a 512-token random prompt,
128 greedy tokens.

The model is decoder.synth_np(QWEN3_4B, MODEL_SEED) and the prompt
prompt_ids() below, both seeded numpy generators, so the GPU test and
bench.py rebuild exactly these inputs on the GPU box.  The oracle is
oracle/decoder_oracle.OracleDecoder (the reference engine's layer order,
decode.cu:2779-3099, composed from the pinned kernel restatements).

Stored per generated position i (i = 0 is the token sampled from the
prefill's last row, decode.cu:2950-2990; i >= 1 the decode step fed token
i-1 at position 512+i-1, decode.cu:2101-2236):
  tokens[i]            greedy id (sample_greedy, sample.cpp:160-170)
  margin[i]            top-1 minus top-2 logit
  absmax[i]            max |logit|
  lsum[i]              float64 sum of the logits
  sample_idx, sample[i, :]  the logits at 512 fixed vocab indices
  top_idx[i, :], top_val[i, :]  the 8 largest logits

Run (8 threads, ~20-30 min on the build container's CPU):
    python tests/golden/make_e2e_golden.py [threads]

The decoder is numerically chaotic: int8 KV codes and q8 activation codes
flip on ulp-level differences, and 36 layers amplify them.  To measure how
much, `--perturb SEED` reruns the oracle, teacher-forced with the stored
tokens, with every matmul output (MMQ, MMVQ, float GEMV) multiplied by
(1 + 1e-6 * N(0, 1)) -- the size of the fp32 summation-order differences
between any two correct implementations -- and writes, per position, the
largest deviation of the 512 sampled and the 8 top logits from the
unperturbed run, to e2e_qwen3_4b_env<SEED>.npz.
    python tests/golden/make_e2e_golden.py [threads] --perturb SEED
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "genie-ai-runtime_amd")]

MODEL_SEED = 4242
PROMPT_SEED = 1
N_PROMPT = 512
N_GEN = 128
N_SAMPLE = 512
OUT = os.path.join(HERE, "e2e_qwen3_4b.npz")


def prompt_ids(vocab, n=N_PROMPT, seed=PROMPT_SEED):
    """The configs[4] prompt: n token ids uniform in [0, vocab)."""
    return np.random.Generator(np.random.MT19937(seed)).integers(0, vocab, n).astype(np.int32)


def sample_indices(vocab, n=N_SAMPLE):
    return np.sort(np.random.Generator(np.random.MT19937(99)).choice(vocab, n, replace=False)).astype(np.int64)


def record(logits):
    lg = np.asarray(logits, np.float32)
    order = np.argsort(-lg, kind="stable")[:8]
    return lg, order, lg[order]


def perturb_oracle(oracle, seed, rel=1e-6):
    """Multiply every matmul output of the oracle by (1 + rel * N(0, 1))."""
    rng = np.random.default_rng(seed)
    for name in ("mmq", "mmvq", "gemv_quant_cpu"):
        fn = getattr(oracle, name)

        def wrapped(*a, _fn=fn, **kw):
            y = _fn(*a, **kw)
            return (y * (1.0 + rel * rng.standard_normal(y.shape))).astype(np.float32)
        setattr(oracle, name, wrapped)


def envelope(threads, seed):
    import decoder
    import decoder_oracle
    import oracle
    gold = np.load(OUT)
    oracle.set_threads(threads)
    perturb_oracle(oracle, seed)
    shape = decoder.QWEN3_4B
    model = decoder.synth_np(shape, int(gold["model_seed"]))
    od = decoder_oracle.OracleDecoder(shape, model, N_PROMPT + N_GEN)
    toks = gold["tokens"]
    dev = []

    def keep(i):
        lg = np.asarray(od.logits, np.float32)
        d = max(float(np.abs(lg[gold["sample_idx"]] - gold["sample"][i]).max()),
                float(np.abs(lg[gold["top_idx"][i]] - gold["top_val"][i]).max()))
        dev.append(d)
        print(f"pos {i} deviation {d:.4f} ({d / gold['absmax'][i]:.4f} of max|logits|)", flush=True)

    od.prefill(list(gold["prompt"]))
    keep(0)
    for i in range(1, N_GEN):
        od.step(int(toks[i - 1]), N_PROMPT + i - 1)
        keep(i)
    path = OUT.replace(".npz", f"_env{seed}.npz")
    np.savez_compressed(path, deviation=np.array(dev, np.float32), seed=seed, rel=1e-6)
    print("wrote", path, flush=True)


def main():
    import decoder
    import decoder_oracle
    import oracle
    threads = int(sys.argv[1]) if len(sys.argv) > 1 else (os.cpu_count() or 1)
    if "--perturb" in sys.argv:
        envelope(threads, int(sys.argv[sys.argv.index("--perturb") + 1]))
        return
    oracle.set_threads(threads)
    shape = decoder.QWEN3_4B
    t0 = time.time()
    model = decoder.synth_np(shape, MODEL_SEED)
    prompt = prompt_ids(shape.vocab_size)
    sidx = sample_indices(shape.vocab_size)
    print(f"model + prompt in {time.time() - t0:.1f} s", flush=True)
    od = decoder_oracle.OracleDecoder(shape, model, N_PROMPT + N_GEN)
    toks, margin, absmax, lsum, samp, tidx, tval = [], [], [], [], [], [], []

    def keep(tok):
        lg, order, vals = record(od.logits)
        assert order[0] == tok
        toks.append(tok)
        margin.append(vals[0] - vals[1])
        absmax.append(np.abs(lg).max())
        lsum.append(lg.astype(np.float64).sum())
        samp.append(lg[sidx])
        tidx.append(order)
        tval.append(vals)

    t0 = time.time()
    keep(od.prefill(list(prompt)))
    print(f"prefill {time.time() - t0:.1f} s -> {toks[0]} margin {margin[0]:.4f}", flush=True)
    for i in range(1, N_GEN):
        t1 = time.time()
        keep(od.step(toks[-1], N_PROMPT + i - 1))
        print(f"step {i} {time.time() - t1:.1f} s -> {toks[-1]} margin {margin[-1]:.4f}", flush=True)
    np.savez_compressed(OUT, prompt=prompt, tokens=np.array(toks, np.int32), margin=np.array(margin, np.float32),
                        absmax=np.array(absmax, np.float32), lsum=np.array(lsum, np.float64),
                        sample_idx=sidx, sample=np.array(samp, np.float32), top_idx=np.array(tidx, np.int64),
                        top_val=np.array(tval, np.float32), model_seed=MODEL_SEED, prompt_seed=PROMPT_SEED)
    print("wrote", OUT, flush=True)


if __name__ == "__main__":
    main()
