"""Independent numpy restatements used to PIN the C oracle (tests only).

Written from the GGUF K-quant block specification, vectorised over whole
tensors (a different code structure from the oracle's per-element loops),
and evaluated in float64 / int64 so that the oracle's fp32 results can be
checked against exact or near-exact values.
"""
import numpy as np


def f16(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def q4k_fields(W, rows, K):
    nb = K // 256
    b = np.asarray(W, dtype=np.uint8).reshape(rows, nb, 144)
    d = f16(b[:, :, 0:2].copy().view(np.uint16)[..., 0])
    dmin = f16(b[:, :, 2:4].copy().view(np.uint16)[..., 0])
    s = b[:, :, 4:16].astype(np.int64)
    sc = np.empty((rows, nb, 8), np.int64)
    mn = np.empty((rows, nb, 8), np.int64)
    # sub-blocks 0..3: low 6 bits of bytes 0..3 (scale) and 4..7 (min)
    sc[..., 0:4] = s[..., 0:4] & 63
    mn[..., 0:4] = s[..., 4:8] & 63
    # sub-blocks 4..7: low/high nibble of bytes 8..11 plus the top 2 bits of bytes 0..3 / 4..7
    sc[..., 4:8] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:8] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    qs = b[:, :, 16:144].reshape(rows, nb, 4, 32).astype(np.int64)
    q = np.empty((rows, nb, 8, 32), np.int64)
    q[:, :, 0::2, :] = qs & 15   # sub-block 2*il: low nibbles of the il-th 32 bytes
    q[:, :, 1::2, :] = qs >> 4   # sub-block 2*il+1: high nibbles
    return d, dmin, sc, mn, q


def q4k_dequant(W, rows, K):
    d, dmin, sc, mn, q = q4k_fields(W, rows, K)
    w = d[..., None, None] * sc[..., None] * q - dmin[..., None, None] * mn[..., None]
    return w.reshape(rows, K)


def q5k_fields(W, rows, K):
    """Q5_K: Q4_K header (d, dmin, 12 scale bytes), qh[32], qs[128]; code =
    nibble + 16 * bit (2*il for the low nibbles, 2*il+1 for the high) of qh."""
    nb = K // 256
    b = np.asarray(W, dtype=np.uint8).reshape(rows, nb, 176)
    hdr = np.concatenate([b[:, :, 0:16], np.zeros((rows, nb, 128), np.uint8)], axis=2)
    d, dmin, sc, mn, _ = q4k_fields(hdr.reshape(rows, -1), rows, K)
    qh = b[:, :, 16:48].astype(np.int64)
    qs = b[:, :, 48:176].reshape(rows, nb, 4, 32).astype(np.int64)
    q = np.empty((rows, nb, 8, 32), np.int64)
    for il in range(4):
        q[:, :, 2 * il, :] = (qs[:, :, il] & 15) + 16 * ((qh >> (2 * il)) & 1)
        q[:, :, 2 * il + 1, :] = (qs[:, :, il] >> 4) + 16 * ((qh >> (2 * il + 1)) & 1)
    return d, dmin, sc, mn, q


def q5k_dequant(W, rows, K):
    d, dmin, sc, mn, q = q5k_fields(W, rows, K)
    w = d[..., None, None] * sc[..., None] * q - dmin[..., None, None] * mn[..., None]
    return w.reshape(rows, K)


def q6k_fields(W, rows, K):
    nb = K // 256
    b = np.asarray(W, dtype=np.uint8).reshape(rows, nb, 210)
    ql = b[:, :, 0:128].reshape(rows, nb, 2, 64).astype(np.int64)
    qh = b[:, :, 128:192].reshape(rows, nb, 2, 32).astype(np.int64)
    sc = b[:, :, 192:208].copy().view(np.int8).astype(np.int64)
    d = f16(b[:, :, 208:210].copy().view(np.uint16)[..., 0])
    q = np.empty((rows, nb, 2, 4, 32), np.int64)
    q[..., 0, :] = (ql[..., 0:32] & 15) | (((qh >> 0) & 3) << 4)
    q[..., 1, :] = (ql[..., 32:64] & 15) | (((qh >> 2) & 3) << 4)
    q[..., 2, :] = (ql[..., 0:32] >> 4) | (((qh >> 4) & 3) << 4)
    q[..., 3, :] = (ql[..., 32:64] >> 4) | (((qh >> 6) & 3) << 4)
    return d, sc, (q - 32).reshape(rows, nb, 256)


def q6k_dequant(W, rows, K):
    d, sc, q = q6k_fields(W, rows, K)
    scale = np.repeat(sc, 16, axis=2)        # scales[k >> 4]
    return (d[..., None] * scale * q).reshape(rows, K)


def dequant(W, t, rows, K):
    return {12: q4k_dequant, 13: q5k_dequant, 14: q6k_dequant}[t](W, rows, K)


def codes(W, t, rows, K):
    """Integer weight codes per element: Q4_K nibble (0..15), Q6_K q-32."""
    if t == 12:
        return q4k_fields(W, rows, K)[4].reshape(rows, K)
    return q6k_fields(W, rows, K)[2].reshape(rows, K)


def q8_1_blocks(xbits, K):
    """q8_1 per 32 values (clamped), float64 arithmetic: returns q int, d fp64."""
    x = f16(xbits).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax / 127.0).astype(np.float32).astype(np.float64)
    with np.errstate(divide="ignore"):
        idv = np.where(d > 0, (1.0 / d.astype(np.float32)).astype(np.float32), 0).astype(np.float64)
    q = np.clip(np.rint((x * idv[:, None]).astype(np.float32)), -127, 127).astype(np.int64)
    return q, d


def attention_f64(q, k, v, ks, vs, n_heads, n_kv, hd, seq, scale, window):
    """Exact softmax attention in float64 over int8 K/V with per-(pos, head) scales."""
    qf = f16(q).reshape(n_heads, hd)
    out = np.zeros((n_heads, hd))
    lo = max(0, seq - window) if window > 0 else 0
    for h in range(n_heads):
        kvh = h // (n_heads // n_kv)
        kk = k[lo:seq, kvh, :hd].astype(np.float64) * ks[lo:seq, kvh, None]
        vv = v[lo:seq, kvh, :hd].astype(np.float64) * vs[lo:seq, kvh, None]
        s = kk @ qf[h] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vv
    return out
