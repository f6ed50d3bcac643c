"""GGUF reader / writer of the library (CPU), checked against an independent
restatement of the file format (struct-based, written from the GGUF spec:
header, typed metadata, tensor infos, 32-byte alignment) and against the
reference loader's config / name rules (model.cpp:150-345, :675-810); plus
the decoder built from a GGUF file on the GPU, which must generate the same
tokens as the same model handed over in memory."""
import ctypes
import struct

import numpy as np
import pytest

import decoder
import jllm
import synth

TINY = decoder.Shape(n_layers=2, hidden_dim=512, n_heads=8, n_kv_heads=2, head_dim=64, intermediate_dim=1024,
                     vocab_size=1000)


def parse_spec(buf):
    """Independent GGUF v3 parser (python struct)."""
    off = 0

    def take(fmt):
        nonlocal off
        v = struct.unpack_from("<" + fmt, buf, off)
        off += struct.calcsize("<" + fmt)
        return v[0] if len(v) == 1 else v

    def string():
        nonlocal off
        n = take("Q")
        s = bytes(buf[off:off + n]).decode()
        off += n
        return s
    magic, version, n_t, n_kv = take("I"), take("I"), take("Q"), take("Q")
    kv = {}
    scal = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
    for _ in range(n_kv):
        k = string()
        t = take("I")
        kv[k] = string() if t == 8 else take(scal[t])
    tensors = []
    for _ in range(n_t):
        name = string()
        nd = take("I")
        dims = [take("Q") for _ in range(nd)]
        tensors.append((name, dims, take("I"), take("Q")))
    data = (off + 31) // 32 * 32
    return magic, version, kv, tensors, data


@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    model = decoder.synth_np(TINY, 31)
    path = tmp_path_factory.mktemp("gguf") / "tiny.gguf"
    decoder.write_gguf(path, TINY, model)
    return path, model


def test_writer_matches_the_spec(tiny_file):
    path, model = tiny_file
    buf = open(path, "rb").read()
    magic, version, kv, tensors, data = parse_spec(buf)
    assert magic == 0x46554747 and version == 3
    assert kv["general.architecture"] == "qwen3" and kv["qwen3.block_count"] == 2
    assert kv["qwen3.embedding_length"] == 512 and kv["qwen3.attention.head_count_kv"] == 2
    assert abs(kv["qwen3.rope.freq_base"] - 1e6) < 1 and kv["qwen3.attention.layer_norm_rms_epsilon"] == np.float32(1e-6)
    names = [t[0] for t in tensors]
    assert names[:3] == ["token_embd.weight", "output_norm.weight", "output.weight"]
    assert len(names) == 3 + 2 * 11
    by = {t[0]: t for t in tensors}
    assert by["blk.1.ffn_down.weight"][1] == [1024, 512] and by["blk.1.ffn_down.weight"][2] == 12
    assert by["blk.0.ffn_down.weight"][2] == 14 and by["token_embd.weight"][1] == [512, 1000]
    for name, dims, t, o in tensors:
        assert o % 32 == 0
    # the bytes of a few tensors at data + offset
    q = by["blk.1.attn_q.weight"]
    nbytes = model["layers"][1]["wq"].nbytes
    assert bytes(buf[data + q[3]:data + q[3] + nbytes]) == model["layers"][1]["wq"].tobytes()
    on = by["output_norm.weight"]
    assert np.array_equal(np.frombuffer(buf, np.float32, 512, data + on[3]), model["output_norm"])


def test_reader_tensor_table_and_metadata(tiny_file):
    path, model = tiny_file
    lib = jllm.lib()
    g = lib.jllm_hip_gguf_open(str(path).encode())
    assert g
    try:
        assert lib.jllm_hip_gguf_n_tensors(g) == 25
        i = lib.jllm_hip_gguf_find_tensor(g, b"blk.0.ffn_down.weight")
        assert i >= 0 and lib.jllm_hip_gguf_find_tensor(g, b"nope") == -1
        name, t, nd = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
        dims = (ctypes.c_int64 * 4)()
        data, nb = ctypes.c_void_p(), ctypes.c_int64()
        assert lib.jllm_hip_gguf_tensor(g, i, ctypes.byref(name), ctypes.byref(t), ctypes.byref(nd), dims,
                                        ctypes.byref(data), ctypes.byref(nb)) == 0
        assert name.value == b"blk.0.ffn_down.weight" and t.value == 14 and nd.value == 2
        assert list(dims) == [1024, 512, 1, 1]
        w = model["layers"][0]["w_down"]
        assert nb.value == w.nbytes and ctypes.string_at(data.value, nb.value) == w.tobytes()
        u, f = ctypes.c_uint64(), ctypes.c_double()
        assert lib.jllm_hip_gguf_get_u64(g, b"qwen3.feed_forward_length", ctypes.byref(u)) == 0 and u.value == 1024
        assert lib.jllm_hip_gguf_get_f64(g, b"qwen3.rope.freq_base", ctypes.byref(f)) == 0 and f.value == 1e6
        assert lib.jllm_hip_gguf_get_str(g, b"general.architecture") == b"qwen3"
        assert lib.jllm_hip_gguf_get_u64(g, b"general.architecture", ctypes.byref(u)) != 0
    finally:
        lib.jllm_hip_gguf_close(g)


def test_config_from_metadata(tiny_file):
    path, _ = tiny_file
    cfg, g = decoder.gguf_config(path)
    jllm.lib().jllm_hip_gguf_close(g)
    assert (cfg.n_layers, cfg.hidden_dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.intermediate_dim,
            cfg.vocab_size) == (2, 512, 8, 2, 64, 1024, 1000)
    assert cfg.rope_neox == 1 and cfg.norm_fp32 == 1 and cfg.qk_norm_fp32 == 1 and cfg.output_norm_fp32 == 1
    assert abs(cfg.rope_theta - 1e6) < 1 and cfg.max_seq == 40960 and cfg.kv_int8 == 1


def test_config_vocab_from_embedding_and_llama_rope(tmp_path):
    """Without `.vocab_size` the vocabulary comes from token_embd.weight's
    second dimension; a llama architecture uses interleaved RoPE."""
    model = decoder.synth_np(TINY, 32)
    path = tmp_path / "llama.gguf"
    decoder.write_gguf(path, TINY, model, arch="llama")
    cfg, g = decoder.gguf_config(path)
    jllm.lib().jllm_hip_gguf_close(g)
    assert cfg.vocab_size == 1000 and cfg.rope_neox == 0


@pytest.mark.parametrize("damage", ["magic", "truncate_header", "truncate_data", "huge_len"])
def test_malformed_files_are_rejected(tiny_file, tmp_path, damage):
    path, _ = tiny_file
    buf = bytearray(open(path, "rb").read())
    if damage == "magic":
        buf[0] = ord("X")
    elif damage == "truncate_header":
        buf = buf[:200]
    elif damage == "truncate_data":
        buf = buf[:len(buf) - 1000]
    else:
        struct.pack_into("<Q", buf, 24, 1 << 60)          # the first key's length
    bad = tmp_path / f"{damage}.gguf"
    open(bad, "wb").write(bytes(buf))
    assert not jllm.lib().jllm_hip_gguf_open(str(bad).encode())


def _write_one_tensor(path, align=None):
    lib = jllm.lib()
    w = lib.jllm_hip_gguf_writer_create()
    try:
        jllm.check(lib.jllm_hip_gguf_writer_set_str(w, b"general.architecture", b"qwen3"), "arch")
        if align is not None:
            jllm.check(lib.jllm_hip_gguf_writer_set_u32(w, b"general.alignment", align), "alignment")
        a = np.arange(3 * 256, dtype=np.float32)
        d = (ctypes.c_int64 * 2)(256, 3)
        jllm.check(lib.jllm_hip_gguf_writer_add_tensor(w, b"t.weight", 0, 2, d, a.ctypes.data_as(ctypes.c_void_p),
                                                       a.nbytes), "tensor")
        return lib.jllm_hip_gguf_writer_write(w, str(path).encode()), a
    finally:
        lib.jllm_hip_gguf_writer_free(w)


def test_alignment_is_honoured_and_validated(tmp_path):
    """general.alignment (a power of two, per the GGUF spec) places the
    tensor data; the writer pads to the declared alignment, and a file
    declaring a non-power-of-two alignment is rejected (it would misplace
    every tensor)."""
    lib = jllm.lib()
    p64 = tmp_path / "a64.gguf"
    st, a = _write_one_tensor(p64, 64)
    assert st == 0
    g = lib.jllm_hip_gguf_open(str(p64).encode())
    assert g
    try:
        data, nbytes = ctypes.c_void_p(), ctypes.c_int64()
        jllm.check(lib.jllm_hip_gguf_tensor(g, 0, None, None, None, None, ctypes.byref(data), ctypes.byref(nbytes)),
                   "tensor")
        got = np.ctypeslib.as_array((ctypes.c_float * (nbytes.value // 4)).from_address(data.value))
        assert np.array_equal(got, a)
    finally:
        lib.jllm_hip_gguf_close(g)
    buf = bytearray(open(p64, "rb").read())
    assert (len(buf) - 3 * 256 * 4) % 64 == 0
    key = b"general.alignment"
    at = buf.index(key) + len(key) + 4                 # after the key string and the u32 value type
    assert struct.unpack_from("<I", buf, at)[0] == 64
    for bad in (48, 0):
        struct.pack_into("<I", buf, at, bad)
        path = tmp_path / f"a{bad}.gguf"
        open(path, "wb").write(bytes(buf))
        assert not lib.jllm_hip_gguf_open(str(path).encode()), bad
    assert _write_one_tensor(tmp_path / "w48.gguf", 48)[0] != 0


@pytest.mark.gpu
def test_decoder_from_gguf_matches_in_memory_model(dev, tiny_file):
    import torch
    path, model = tiny_file
    prompt = torch.tensor(synth.rng(33).integers(0, 1000, 16).astype(np.int32), device=dev)
    ref = decoder.Decoder(TINY, decoder.to_device(model, dev), 32, max_batch=64)
    a = torch.zeros(6, dtype=torch.int32, device=dev)
    ref.generate(prompt, 6, a)
    gg = decoder.GGUFDecoder(path, max_seq=32, max_batch=64)
    b = torch.zeros(6, dtype=torch.int32, device=dev)
    gg.generate(prompt, 6, b)
    torch.cuda.synchronize()
    assert a.cpu().tolist() == b.cpu().tolist()
    ref.close()
    gg.close()


def _load_fails(path, capfd, needle):
    """The loader refuses the file before any device allocation (the message
    names the offending tensor)."""
    lib = jllm.lib()
    cfg, g = decoder.gguf_config(path)
    try:
        m = lib.jllm_hip_gguf_model_load(g, ctypes.addressof(cfg))
        assert not m
    finally:
        lib.jllm_hip_gguf_close(g)
    err = capfd.readouterr().err
    assert needle in err, err


def test_model_load_rejects_wrong_shaped_matrix(tmp_path, capfd):
    """attn_k stored as [1024, 64] instead of [512, 128]: the same byte count,
    but the GEMV would read rows of the wrong length."""
    model = decoder.synth_np(TINY, 34)

    def hook(name, t, dims, arr):
        return (t, [1024, 64], arr) if name == "blk.1.attn_k.weight" else (t, dims, arr)
    path = tmp_path / "bad_k.gguf"
    decoder.write_gguf(path, TINY, model, hook=hook)
    _load_fails(path, capfd, "blk.1.attn_k.weight")


def test_model_load_rejects_mixed_norm_types(tmp_path, capfd):
    """blk.0 norms are F32 (so the config says fp32), blk.1's attn_norm is F16:
    the decoder would read it as fp32."""
    model = decoder.synth_np(TINY, 35)

    def hook(name, t, dims, arr):
        if name == "blk.1.attn_norm.weight":
            return 1, dims, np.asarray(arr, np.float32).astype(np.float16).view(np.uint16)
        return t, dims, arr
    path = tmp_path / "bad_norm.gguf"
    decoder.write_gguf(path, TINY, model, hook=hook)
    _load_fails(path, capfd, "blk.1.attn_norm.weight")


def test_model_load_rejects_unsupported_matrix_type(tmp_path, capfd):
    model = decoder.synth_np(TINY, 36)

    def hook(name, t, dims, arr):
        if name == "blk.0.ffn_up.weight":      # the same bytes declared as F16 [4096, 9*...] -> not a K-quant
            n = np.asarray(arr).nbytes // 2
            return 1, [n], arr
        return t, dims, arr
    path = tmp_path / "bad_type.gguf"
    decoder.write_gguf(path, TINY, model, hook=hook)
    _load_fails(path, capfd, "blk.0.ffn_up.weight")


@pytest.mark.parametrize("field,value,needle", [("hidden_dim", 5120, "hidden_dim must be <= 4096"),
                                                ("head_dim", 80, "head_dim must be a multiple of 32"),
                                                ("n_kv_heads", 3, "n_heads must be a multiple"),
                                                ("intermediate_dim", 1000, "multiples of 256")])
def test_decoder_create_rejects_unsupported_shapes(capfd, field, value, needle):
    """Refused at creation (before any allocation), with the reason."""
    cfg = decoder.Config(2, 2560, 32, 8, 128, 9728, 1000, 64, 1e-6, 1e6, 1, 1, 1, 1, 1)
    setattr(cfg, field, value)
    arr = (decoder.LayerW * 2)()
    mw = decoder.ModelW()
    h = jllm.lib().jllm_hip_decoder_create(ctypes.addressof(cfg), ctypes.addressof(mw), ctypes.addressof(arr), 16)
    assert not h
    err = capfd.readouterr().err
    assert needle in err, err


def test_gguf_config_rejects_unsupported_shapes(tmp_path, capfd):
    shape = decoder.Shape(n_layers=1, hidden_dim=512, n_heads=8, n_kv_heads=2, head_dim=64, intermediate_dim=1024,
                          vocab_size=1000)
    model = decoder.synth_np(shape, 37)
    path = tmp_path / "hd64.gguf"
    decoder.write_gguf(path, shape, model)

    lib = jllm.lib()
    g = lib.jllm_hip_gguf_open(str(path).encode())
    cfg = decoder.Config()
    assert lib.jllm_hip_gguf_config(g, ctypes.addressof(cfg)) == 0     # head_dim 64 is supported
    lib.jllm_hip_gguf_close(g)
    bad = decoder.Shape(n_layers=1, hidden_dim=512, n_heads=8, n_kv_heads=3, head_dim=64, intermediate_dim=1024,
                        vocab_size=1000)
    path = tmp_path / "kv3.gguf"
    decoder.write_gguf(path, bad, decoder.synth_np(bad, 38))
    g = lib.jllm_hip_gguf_open(str(path).encode())
    assert lib.jllm_hip_gguf_config(g, ctypes.addressof(cfg)) == -2
    lib.jllm_hip_gguf_close(g)
    assert "n_heads must be a multiple" in capfd.readouterr().err
