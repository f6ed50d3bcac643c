"""Regenerates tests/golden/fixtures.npz: seeded slices of the BASELINE
configs and the CPU oracle's outputs for them, plus full-size checksums.

The reference (C++/CUDA for SM 8.7) cannot run here and holds no golden
vectors, so these fixtures come from this repository's CPU restatement
(oracle/, pinned by tests/test_oracle_pins.py): they freeze the oracle's
values so that a later change to it or to the seeded generators shows up,
and they let the GPU tests check full-size configs through checksums.

Run from the repository root: python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "genie-ai-runtime_amd")]
import oracle  # noqa: E402
import synth  # noqa: E402

# (seed, description) of every fixture; tests regenerate the inputs from these
SEED_GEMV, SEED_GEMV6, SEED_MMQ, SEED_ATTN = 101, 102, 103, 104


def config1_inputs():
    """Q4_K 9728 x 2560, x fp16 N(0, 1)."""
    g = synth.rng(SEED_GEMV)
    return synth.q4k(g, 9728, 2560), synth.x_f16(g, 2560)


def config2_down_inputs():
    """configs[1] Q6_K down: 2560 x 9728."""
    g = synth.rng(SEED_GEMV6)
    return synth.q6k(g, 2560, 9728), synth.x_f16(g, 9728)


def config3_inputs():
    """Q4_K 9728 x 2560 weights, 64 tokens."""
    g = synth.rng(SEED_MMQ)
    return synth.q4k(g, 9728, 2560), synth.x_f16(g, (64, 2560))


def config4_inputs(ctx=512):
    """32 q heads / 8 KV heads x 128, INT8 KV, ctx 512."""
    g = synth.rng(SEED_ATTN)
    q = synth.x_f16(g, 32 * 128)
    k, v = synth.kv_int8(g, ctx, 8, 128), synth.kv_int8(g, ctx, 8, 128)
    return q, k, v, synth.kv_scales(g, ctx, 8), synth.kv_scales(g, ctx, 8)


def build():
    out = {}
    W, x = config1_inputs()
    y = oracle.gemv_quant_cpu(W, 12, x, 9728, 2560, threads=8)
    ym = oracle.mmvq(W, 12, oracle.quantize_q8_1(x, 2560), 9728, 2560)
    out["c1_y_rows0_64"] = y[:64]
    out["c1_mmvq_rows0_64"] = ym[:64]
    out["c1_y_sum"] = np.float64(y.astype(np.float64).sum())
    out["c1_y_l2"] = np.float64(np.sqrt((y.astype(np.float64) ** 2).sum()))
    out["c1_mmvq_l2"] = np.float64(np.sqrt((ym.astype(np.float64) ** 2).sum()))
    out["c1_q8_1"] = oracle.quantize_q8_1(x, 2560)
    W6, x6 = config2_down_inputs()
    y6 = oracle.gemv_quant_cpu(W6, 14, x6, 2560, 9728, threads=8)
    out["c2_down_y_rows0_64"] = y6[:64]
    out["c2_down_y_l2"] = np.float64(np.sqrt((y6.astype(np.float64) ** 2).sum()))
    Wm, xm = config3_inputs()
    q8 = oracle.quantize_mmq(xm, 64, 2560, 64, True)
    out["c3_q8_ds4_crc"] = np.uint64(int.from_bytes(__import__("hashlib").sha256(q8.tobytes()).digest()[:8], "little"))
    ym3 = oracle.mmq(Wm[:64], 12, q8, 64, 64, 2560, 64)
    out["c3_y_rows0_64"] = ym3
    q, k, v, ks, vs = config4_inputs()
    out["c4_out"] = oracle.attn_decode_int8(q, k, v, 32, 8, 128, 128, 512, 1.0 / np.sqrt(128), ks, vs, 0,
                                            oracle.decode_attn_splits(512))
    return out


if __name__ == "__main__":
    oracle.build()
    np.savez_compressed(os.path.join(os.path.dirname(os.path.abspath(__file__)), "fixtures.npz"), **build())
    print("wrote tests/golden/fixtures.npz")
