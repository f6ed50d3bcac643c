"""Seeded synthetic inputs with the distributions of the BASELINE configs.

Weights are raw GGUF K-quant blocks (uint8 arrays, rows contiguous):
  Q4_K (144 B / 256 weights): d, dmin = fp16(|N(0, 0.02)|); 12 random scale
      bytes (all 16 six-bit scale/min fields uniform in [0, 63]); 128 random
      qs bytes (nibbles uniform in [0, 15]).
  Q5_K (176 B / 256 weights): Q4_K header (d, dmin, scales) as above, 32
      random qh bytes (fifth code bits) and 128 random qs bytes.
  Q6_K (210 B / 256 weights): random ql/qh bytes (codes uniform in [0, 63]);
      int8 sub-block scales uniform in [-32, 31]; d = fp16(|N(0, 0.01)|).
Activations: fp32 N(0, 1) rounded to fp16 (RNE), returned as uint16 bits.
"""
import numpy as np

QK_K = 256
BLOCK_BYTES = {12: 144, 13: 176, 14: 210}


def rng(seed):
    return np.random.Generator(np.random.MT19937(seed))


def _f16_bits(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def q4k(g, rows, K, d_sigma=0.02, dmin_sigma=0.02):
    nb = K // QK_K
    blk = np.frombuffer(g.bytes(rows * nb * 144), dtype=np.uint8).reshape(rows, nb, 144).copy()
    d = _f16_bits(np.abs(g.standard_normal((rows, nb), dtype=np.float32)) * d_sigma)
    dm = _f16_bits(np.abs(g.standard_normal((rows, nb), dtype=np.float32)) * dmin_sigma)
    blk[:, :, 0:2] = d.reshape(rows, nb, 1).view(np.uint8)
    blk[:, :, 2:4] = dm.reshape(rows, nb, 1).view(np.uint8)
    return blk.reshape(rows, nb * 144)


def q5k(g, rows, K, d_sigma=0.01, dmin_sigma=0.02):
    nb = K // QK_K
    blk = np.frombuffer(g.bytes(rows * nb * 176), dtype=np.uint8).reshape(rows, nb, 176).copy()
    d = _f16_bits(np.abs(g.standard_normal((rows, nb), dtype=np.float32)) * d_sigma)
    dm = _f16_bits(np.abs(g.standard_normal((rows, nb), dtype=np.float32)) * dmin_sigma)
    blk[:, :, 0:2] = d.reshape(rows, nb, 1).view(np.uint8)
    blk[:, :, 2:4] = dm.reshape(rows, nb, 1).view(np.uint8)
    return blk.reshape(rows, nb * 176)


def q6k(g, rows, K, d_sigma=0.01):
    nb = K // QK_K
    blk = np.frombuffer(g.bytes(rows * nb * 210), dtype=np.uint8).reshape(rows, nb, 210).copy()
    blk[:, :, 192:208] = g.integers(-32, 32, size=(rows, nb, 16), dtype=np.int8).view(np.uint8)
    d = _f16_bits(np.abs(g.standard_normal((rows, nb), dtype=np.float32)) * d_sigma)
    blk[:, :, 208:210] = d.reshape(rows, nb, 1).view(np.uint8)
    return blk.reshape(rows, nb * 210)


def weights(g, ggml_type, rows, K):
    return {12: q4k, 13: q5k, 14: q6k}[ggml_type](g, rows, K)


def x_f16(g, shape):
    return _f16_bits(g.standard_normal(shape, dtype=np.float32))


def kv_int8(g, ctx, n_kv, hd):
    return g.integers(-127, 128, size=(ctx, n_kv, hd), dtype=np.int8)


def kv_scales(g, ctx, n_kv, sigma=0.05):
    """|N(0, sigma)| rounded to fp16, stored as fp32 (the reference's KV scale buffers are fp32)."""
    s = np.abs(g.standard_normal((ctx, n_kv), dtype=np.float32)) * sigma
    return s.astype(np.float16).astype(np.float32)
