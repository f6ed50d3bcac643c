"""Host-side binding of the decoder loop (jllm_hip_decoder_* in the C ABI)
and a seeded random Q4_K_M-layout model for it.

The model mirrors the reference's LayerWeights / ModelWeights
(include/jllm_engine.h:165-225): per layer rms_attn, rms_ffn, q_norm,
k_norm (fp32) and seven K-quant matrices; the token embedding, the output
norm and the lm_head (untied: a Q4_K embedding table and a Q6_K lm_head;
with a random model a tied table makes greedy decoding repeat its input
token).  Weights live in device memory as raw GGUF blocks
(torch uint8 tensors), either generated on the device (large models) or
uploaded from numpy (small models whose bytes a test also needs on the host).
"""
import ctypes
from dataclasses import dataclass

import numpy as np

import jllm

P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float


class Config(ctypes.Structure):
    _fields_ = [("n_layers", I), ("hidden_dim", I), ("n_heads", I), ("n_kv_heads", I), ("head_dim", I),
                ("intermediate_dim", I), ("vocab_size", I), ("max_seq", I), ("rms_eps", F), ("rope_theta", F),
                ("rope_neox", I), ("kv_int8", I), ("norm_fp32", I), ("qk_norm_fp32", I),
                ("output_norm_fp32", I)]


class LayerW(ctypes.Structure):
    _fields_ = [(n, P) for n in ("rms_attn", "rms_ffn", "q_norm", "k_norm", "wq", "wk", "wv", "wo", "w_gate",
                                 "w_up", "w_down")] + \
               [(n, I) for n in ("type_wq", "type_wk", "type_wv", "type_wo", "type_w_gate", "type_w_up",
                                 "type_w_down")]


class ModelW(ctypes.Structure):
    _fields_ = [("tok_embd", P), ("embd_type", I), ("output_norm", P), ("output", P), ("output_type", I)]


MATS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")


@dataclass
class Shape:
    n_layers: int = 36
    hidden_dim: int = 2560
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    intermediate_dim: int = 9728
    vocab_size: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 1e6

    def mat_shape(self, name):
        """(rows M, K) of a layer matrix: y[M] = W[M x K] . x[K]."""
        H, Q, KV, I = self.hidden_dim, self.n_heads * self.head_dim, self.n_kv_heads * self.head_dim, \
            self.intermediate_dim
        return {"wq": (Q, H), "wk": (KV, H), "wv": (KV, H), "wo": (H, Q), "w_gate": (I, H), "w_up": (I, H),
                "w_down": (H, I)}[name]


QWEN3_4B = Shape()


def q4km_types(shape, layer):
    """Q4_K_M layout of the E2E config: Q4_K everywhere in attention and
    gate/up, Q6_K for every other ffn_down (the other half Q4_K)."""
    t = {m: 12 for m in MATS}
    t["w_down"] = 14 if layer % 2 == 0 else 12
    return t


def q5km_types(shape, layer):
    """A Q5_K_M-style layout: Q5_K everywhere, Q6_K for attn_v and ffn_down
    on every other layer."""
    t = {m: 13 for m in MATS}
    if layer % 2 == 0:
        t["wv"] = t["w_down"] = 14
    return t


def q4km_mixed_types(shape, layer):
    """Q4_K_M with more Q6_K matrices: attn_v and ffn_down Q6_K on even
    layers (as llama.cpp's Q4_K_M assigns them on part of the layers), attn_output
    Q6_K on odd layers -- mixed Q4_K / Q6_K products of one activation."""
    t = {m: 12 for m in MATS}
    if layer % 2 == 0:
        t["wv"] = t["w_down"] = 14
    else:
        t["wo"] = 14
    return t


PRESETS = {"q4km": q4km_types, "q5km": q5km_types, "q4km_mixed": q4km_mixed_types}


# Block scales chosen so the dequantised weights have mean ~0 and a
# standard deviation of about 0.02 (a transformer's usual init): Q4_K
# w = d*sc*q - dmin*m with sc, m ~ U[0,63], q ~ U[0,15], so dmin = 7.5 d
# centres it; Q6_K w = d*sc*(q-32) with sc ~ U[-32,31] is centred already.
# Q5_K (q ~ U[0,31]) the same with dmin = 15.5 d.
Q4_D, Q4_DMIN, Q6_D = 1e-4, 7.5e-4, 6e-5
Q5_D, Q5_DMIN = 5e-5, 7.75e-4


def _synth_mat(synth, g, t, M, K):
    if t == 12:
        return synth.q4k(g, M, K, Q4_D, Q4_DMIN)
    if t == 13:
        return synth.q5k(g, M, K, Q5_D, Q5_DMIN)
    return synth.q6k(g, M, K, Q6_D)


def synth_np(shape, seed, preset="q4km"):
    """Numpy model (host bytes) for shapes small enough to keep on the host.
    preset q4km: Q4_K embedding; q5km: Q5_K embedding; Q6_K output in both."""
    import synth
    g = synth.rng(seed)
    layers = []
    for l in range(shape.n_layers):
        types = PRESETS[preset](shape, l)
        L = {"types": types}
        for m in MATS:
            M, K = shape.mat_shape(m)
            L[m] = _synth_mat(synth, g, types[m], M, K)
        for n, dim in (("rms_attn", shape.hidden_dim), ("rms_ffn", shape.hidden_dim),
                       ("q_norm", shape.head_dim), ("k_norm", shape.head_dim)):
            L[n] = (1.0 + 0.02 * g.standard_normal(dim)).astype(np.float32)
        layers.append(L)
    et = 13 if preset == "q5km" else 12
    emb = _synth_mat(synth, g, et, shape.vocab_size, shape.hidden_dim)
    out = synth.q6k(g, shape.vocab_size, shape.hidden_dim, Q6_D)
    return {"layers": layers, "tok_embd": emb, "embd_type": et, "output": out, "output_type": 14,
            "output_norm": (1.0 + 0.02 * g.standard_normal(shape.hidden_dim)).astype(np.float32)}


def _dev_q4k(torch, gen, M, K, dev):
    nb = K // 256
    b = torch.randint(0, 256, (M, nb, 144), dtype=torch.uint8, device=dev, generator=gen)
    d = (torch.randn((M, nb, 2), device=dev, generator=gen).abs() * torch.tensor([Q4_D, Q4_DMIN], device=dev))
    b[:, :, 0:4] = d.to(torch.float16).view(torch.uint8)
    return b.reshape(-1)


def _dev_q6k(torch, gen, M, K, dev):
    nb = K // 256
    b = torch.randint(0, 256, (M, nb, 210), dtype=torch.uint8, device=dev, generator=gen)
    b[:, :, 192:208] = torch.randint(-32, 32, (M, nb, 16), dtype=torch.int8, device=dev, generator=gen).view(
        torch.uint8)
    d = torch.randn((M, nb, 1), device=dev, generator=gen).abs() * Q6_D
    b[:, :, 208:210] = d.to(torch.float16).view(torch.uint8)
    return b.reshape(-1)


def synth_device(shape, seed, dev="cuda:0"):
    """The same kind of model generated directly in device memory (for the
    Qwen3-4B-sized configuration, ~2.4 GB of blocks)."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    layers = []
    for l in range(shape.n_layers):
        types = q4km_types(shape, l)
        L = {"types": types}
        for m in MATS:
            M, K = shape.mat_shape(m)
            L[m] = (_dev_q4k if types[m] == 12 else _dev_q6k)(torch, gen, M, K, dev)
        for n, dim in (("rms_attn", shape.hidden_dim), ("rms_ffn", shape.hidden_dim),
                       ("q_norm", shape.head_dim), ("k_norm", shape.head_dim)):
            L[n] = 1.0 + 0.02 * torch.randn(dim, device=dev, generator=gen)
        layers.append(L)
    emb = _dev_q4k(torch, gen, shape.vocab_size, shape.hidden_dim, dev)
    out = _dev_q6k(torch, gen, shape.vocab_size, shape.hidden_dim, dev)
    return {"layers": layers, "tok_embd": emb, "embd_type": 12, "output": out, "output_type": 14,
            "output_norm": 1.0 + 0.02 * torch.randn(shape.hidden_dim, device=dev, generator=gen)}


def to_device(model_np, dev="cuda:0"):
    import torch

    def up(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    layers = []
    for L in model_np["layers"]:
        layers.append({k: (v if k == "types" else up(v)) for k, v in L.items()})
    out = up(model_np["output"])
    emb = out if model_np["tok_embd"] is model_np["output"] else up(model_np["tok_embd"])
    return {"layers": layers, "tok_embd": emb, "embd_type": model_np["embd_type"], "output": out,
            "output_type": model_np["output_type"], "output_norm": up(model_np["output_norm"])}


class Decoder:
    """Owns a jllm_hip_decoder over a device model (dict from synth_device /
    to_device).  Token buffers passed to the methods are device int32
    tensors; nothing here synchronises the stream."""

    def __init__(self, shape, model, max_seq, max_batch=512, kv_int8=True):
        self.shape, self.model = shape, model
        self.cfg = Config(shape.n_layers, shape.hidden_dim, shape.n_heads, shape.n_kv_heads, shape.head_dim,
                          shape.intermediate_dim, shape.vocab_size, max_seq, shape.rms_eps, shape.rope_theta,
                          1, 1 if kv_int8 else 0, 1, 1, 1)
        arr = (LayerW * shape.n_layers)()
        for l, L in enumerate(model["layers"]):
            w = arr[l]
            for n in ("rms_attn", "rms_ffn", "q_norm", "k_norm") + MATS:
                setattr(w, n, L[n].data_ptr())
            for m in MATS:
                setattr(w, "type_" + m, L["types"][m])
        self._layers = arr
        self.mw = ModelW(model["tok_embd"].data_ptr(), model["embd_type"], model["output_norm"].data_ptr(),
                         model["output"].data_ptr(), model["output_type"])
        self.h = jllm.lib().jllm_hip_decoder_create(ctypes.addressof(self.cfg), ctypes.addressof(self.mw),
                                                    ctypes.addressof(arr), max_batch)
        if not self.h:
            raise jllm.JllmError("jllm_hip_decoder_create failed")

    def prefill(self, tokens, start, next_tok, n=None):
        jllm.call("jllm_hip_decoder_prefill", self.h, tokens, n if n is not None else tokens.numel(), start,
                  next_tok)

    def step(self, token, pos, next_tok):
        jllm.call("jllm_hip_decoder_step", self.h, token, pos, next_tok)

    def generate(self, prompt, n_gen, out):
        jllm.call("jllm_hip_decoder_generate", self.h, prompt, prompt.numel(), n_gen, out)

    def layer(self, l, x, N, start):
        """Run layer l alone on the device rows x [N][hidden] (fp16 as int16),
        in place, at positions start..start+N-1 (decode path for N == 1)."""
        jllm.call("jllm_hip_decoder_layer", self.h, l, x, N, start)

    def kv(self, l, n_pos):
        """Layer l's KV cache, positions 0..n_pos-1, copied to the host:
        (k, v) int8 [n_pos][n_kv][head_dim], (k_scales, v_scales) fp32
        [n_pos][n_kv]."""
        import torch
        s = self.shape
        shp = (n_pos, s.n_kv_heads, s.head_dim)
        k, v = (torch.empty(shp, dtype=torch.int8, device="cuda:0") for _ in range(2))
        ks, vs = (torch.empty((n_pos, s.n_kv_heads), dtype=torch.float32, device="cuda:0") for _ in range(2))
        jllm.call("jllm_hip_decoder_copy_kv", self.h, l, n_pos, k, v, ks, vs)
        torch.cuda.synchronize()
        return k.cpu().numpy(), v.cpu().numpy(), ks.cpu().numpy(), vs.cpu().numpy()

    def act(self, which, rows):
        """Intermediate of the last layer run, first `rows` rows, as host fp16
        bits: which 0 = rotated q, 1 = attention output, 2 = hidden state
        after the attention residual."""
        import torch
        s = self.shape
        width = s.hidden_dim if which == 2 else s.n_heads * s.head_dim
        out = torch.empty(rows * width, dtype=torch.int16, device="cuda:0")
        jllm.call("jllm_hip_decoder_copy_act", self.h, which, rows, out)
        torch.cuda.synchronize()
        return out.cpu().numpy().view(np.uint16).reshape(rows, width)

    def logits(self):
        """fp32 logits [vocab] of the last prefill/step, as a new device tensor."""
        import torch
        out = torch.empty(self.shape.vocab_size, dtype=torch.float32, device="cuda:0")
        jllm.call("jllm_hip_decoder_copy_logits", self.h, out)
        return out

    def close(self):
        if self.h:
            jllm.lib().jllm_hip_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- GGUF ------------------------------------------------------------------------

def write_gguf(path, shape, model_np, arch="qwen3", max_seq=40960, hook=None):
    """Store a synth_np model as a GGUF v3 file with llama.cpp's tensor names
    (the names the reference loader maps, model.cpp:675-810).  hook(name,
    ggml_type, dims, array) -> (ggml_type, dims, array), when given, may
    change a tensor before it is written (tests write malformed models)."""
    lib = jllm.lib()
    w = lib.jllm_hip_gguf_writer_create()
    if not w:
        raise jllm.JllmError("gguf writer")
    try:
        def u32(k, v):
            jllm.check(lib.jllm_hip_gguf_writer_set_u32(w, k.encode(), int(v)), k)

        def f32(k, v):
            jllm.check(lib.jllm_hip_gguf_writer_set_f32(w, k.encode(), float(v)), k)
        jllm.check(lib.jllm_hip_gguf_writer_set_str(w, b"general.architecture", arch.encode()), "arch")
        jllm.check(lib.jllm_hip_gguf_writer_set_str(w, b"general.name", b"random Q4_K_M decoder"), "name")
        u32(f"{arch}.block_count", shape.n_layers)
        u32(f"{arch}.context_length", max_seq)
        u32(f"{arch}.embedding_length", shape.hidden_dim)
        u32(f"{arch}.feed_forward_length", shape.intermediate_dim)
        u32(f"{arch}.attention.head_count", shape.n_heads)
        u32(f"{arch}.attention.head_count_kv", shape.n_kv_heads)
        u32(f"{arch}.attention.key_length", shape.head_dim)
        u32(f"{arch}.attention.value_length", shape.head_dim)
        f32(f"{arch}.rope.freq_base", shape.rope_theta)
        f32(f"{arch}.attention.layer_norm_rms_epsilon", shape.rms_eps)
        keep = []

        def tensor(name, t, dims, arr):
            if hook:
                t, dims, arr = hook(name, t, dims, arr)
            a = np.ascontiguousarray(arr)
            keep.append(a)
            d = (ctypes.c_int64 * len(dims))(*dims)
            jllm.check(lib.jllm_hip_gguf_writer_add_tensor(w, name.encode(), t, len(dims), d,
                                                           a.ctypes.data_as(ctypes.c_void_p), a.nbytes), name)
        H, V = shape.hidden_dim, shape.vocab_size
        tensor("token_embd.weight", model_np["embd_type"], [H, V], model_np["tok_embd"])
        tensor("output_norm.weight", 0, [H], model_np["output_norm"])
        if model_np["output"] is not model_np["tok_embd"]:
            tensor("output.weight", model_np["output_type"], [H, V], model_np["output"])
        names = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "w_gate": "ffn_gate",
                 "w_up": "ffn_up", "w_down": "ffn_down"}
        for l, L in enumerate(model_np["layers"]):
            for m in MATS:
                M, K = shape.mat_shape(m)
                tensor(f"blk.{l}.{names[m]}.weight", L["types"][m], [K, M], L[m])
            tensor(f"blk.{l}.attn_norm.weight", 0, [H], L["rms_attn"])
            tensor(f"blk.{l}.ffn_norm.weight", 0, [H], L["rms_ffn"])
            tensor(f"blk.{l}.attn_q_norm.weight", 0, [shape.head_dim], L["q_norm"])
            tensor(f"blk.{l}.attn_k_norm.weight", 0, [shape.head_dim], L["k_norm"])
        jllm.check(lib.jllm_hip_gguf_writer_write(w, str(path).encode()), "gguf write")
    finally:
        lib.jllm_hip_gguf_writer_free(w)


def gguf_config(path):
    """(Config, raw handle) of a GGUF file; the caller closes the handle."""
    lib = jllm.lib()
    g = lib.jllm_hip_gguf_open(str(path).encode())
    if not g:
        raise jllm.JllmError(f"cannot read GGUF {path}")
    cfg = Config()
    st = lib.jllm_hip_gguf_config(g, ctypes.addressof(cfg))
    if st:
        lib.jllm_hip_gguf_close(g)
        jllm.check(st, "gguf config")
    return cfg, g


class GGUFDecoder:
    """A decoder over a GGUF file: tensors uploaded by the library's loader."""

    def __init__(self, path, max_seq=None, max_batch=512):
        lib = jllm.lib()
        self.cfg, self.g = gguf_config(path)
        if max_seq:
            self.cfg.max_seq = max_seq
        self.model = lib.jllm_hip_gguf_model_load(self.g, ctypes.addressof(self.cfg))
        if not self.model:
            lib.jllm_hip_gguf_close(self.g)
            raise jllm.JllmError("gguf model load")
        self.h = lib.jllm_hip_decoder_create(ctypes.addressof(self.cfg), lib.jllm_hip_gguf_model_weights(self.model),
                                             lib.jllm_hip_gguf_layer_weights(self.model), max_batch)
        if not self.h:
            self.close()
            raise jllm.JllmError("jllm_hip_decoder_create failed")

    def generate(self, prompt, n_gen, out):
        jllm.call("jllm_hip_decoder_generate", self.h, prompt, prompt.numel(), n_gen, out)

    def close(self):
        lib = jllm.lib()
        if getattr(self, "h", None):
            lib.jllm_hip_decoder_destroy(self.h)
            self.h = None
        if getattr(self, "model", None):
            lib.jllm_hip_gguf_model_free(self.model)
            self.model = None
        if getattr(self, "g", None):
            lib.jllm_hip_gguf_close(self.g)
            self.g = None
