"""CPU checks of the boundary: the C-ABI library loads without a GPU and
exports every entry point that include/*.h declares (C symbols of
jllm_hip.h and the namespace jllm C++ functions of jllm_kernels.h); plus the
host-side pieces that need no device (status strings, mapped-weight
registry, split policy)."""
import ctypes
import os
import re
import subprocess

import pytest

import jllm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _exports():
    out = subprocess.run(["nm", "-DC", "--defined-only", jllm.LIB_PATH], capture_output=True, text=True, check=True)
    return out.stdout


def test_library_loads():
    assert jllm.lib() is not None


def test_every_c_declaration_exported():
    hdr = open(os.path.join(ROOT, "include", "jllm_hip.h")).read()
    names = set(re.findall(r"\b(jllm_hip_\w+)\s*\(", hdr))
    assert len(names) >= 20
    exp = _exports()
    missing = [n for n in sorted(names) if not re.search(rf"\bT {n}\b", exp)]
    assert not missing, missing
    for n in names:                       # and the ctypes binding knows every one
        assert n in jllm.SIGNATURES, n


# the engine's mapped-weight registry: declared in jllm_kernels.h, defined by
# the engine's src/engine/model.cpp:39-66 (which stays compiled), never by the library
REGISTRY = {"register_mapped_weight_region", "clear_mapped_weight_region", "resolve_mapped_weight_device_ptr"}


def _cpp_declared():
    hdr = open(os.path.join(ROOT, "include", "jllm_kernels.h")).read()
    body = hdr[hdr.index("namespace jllm {"):]
    return set(re.findall(r"^\s*(?:const\s+)?[\w\*]+\*?\s+\**(\w+)\s*\(", body, re.M))


def test_every_cpp_declaration_exported():
    names = _cpp_declared()
    assert {"gemv_quant", "gemm_quant_batched", "flash_attention_decode", "fp16_to_int8"} <= names
    assert REGISTRY <= names
    exp = _exports()
    missing = [n for n in sorted(names - REGISTRY) if f"jllm::{n}(" not in exp]
    assert not missing, missing
    defined_registry = [n for n in REGISTRY if f"jllm::{n}(" in exp]
    assert not defined_registry, defined_registry


# Every function of the reference's include/jllm_kernels.h (namespace jllm):
# the engine's kernel translation units (gemv_q4.cu, mmq_q4k_llama.cu,
# mmq_q6k_llama.cu, attention.cu, rope.cu, fused_norm.cu, convert.cu,
# softmax.cu, dense_tc.cu) can all be dropped only if the library defines
# each of them except the registry, which model.cpp defines.
REFERENCE_HEADER_FUNCTIONS = {
    "resolve_mapped_weight_device_ptr", "register_mapped_weight_region", "clear_mapped_weight_region",
    "gemv_q4", "gemv_quant", "gemv_quant_add", "gemv_quant_pair", "gemv_quant_triple", "gemm_quant_batched",
    "gemv_quant_f32", "dequant_embedding_row", "fused_rmsnorm_residual", "fused_swiglu", "fused_geglu",
    "vec_scale", "logit_softcap", "gemv_dense", "gemm_dense_batched", "rope_precompute_table",
    "rope_clear_tables", "rope_inplace", "rope_inplace_store_kv_fp16", "rope_inplace_batched",
    "rope_inplace_store_kv_fp16_batched", "rope_inplace_store_kv_fp16_dyn", "rope_inplace_dyn",
    "flash_attention_decode", "flash_attention_prefill_batched", "flash_attention_decode_dyn",
    "decode_attn_splits", "get_splitk_partials", "softmax_inplace", "fp16_to_int8",
}


def test_reference_header_fully_declared():
    assert REFERENCE_HEADER_FUNCTIONS <= _cpp_declared()


def test_engine_links_against_library_alone(tmp_path):
    """A C++ translation unit calling every function the engine calls through
    jllm_kernels.h links against libjllm_hip.so plus a stand-in of
    model.cpp's registry and nothing else (-Wl,--no-undefined); no jllm::
    symbol is defined both by the library and by the stand-in; and the
    library's weak reference finds the engine's registry at run time."""
    cxx = os.path.join(ROOT, "tests", "cxx")
    exe = str(tmp_path / "engine_link")
    libdir = os.path.dirname(jllm.LIB_PATH)
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-O1", "-I" + os.path.join(ROOT, "include"),
           os.path.join(cxx, "engine_link.cpp"), os.path.join(cxx, "model_registry_stub.cpp"),
           "-L" + libdir, "-ljllm_hip", "-Wl,-rpath," + libdir, "-Wl,--no-undefined", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    stub_obj = str(tmp_path / "stub.o")
    r = subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++17", "-c", "-I" + os.path.join(ROOT, "include"),
                        os.path.join(cxx, "model_registry_stub.cpp"), "-o", stub_obj], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    stub = subprocess.run(["nm", "-C", "--defined-only", stub_obj], capture_output=True, text=True, check=True).stdout
    stub_defs = set(re.findall(r" T (jllm::\w+)\(", stub))
    lib_defs = set(re.findall(r" T (jllm::\w+)\(", _exports()))
    assert stub_defs == {"jllm::" + n for n in REGISTRY}
    assert not (stub_defs & lib_defs)
    called = subprocess.run(["nm", "-DC", exe], capture_output=True, text=True, check=True).stdout
    undefined = set(re.findall(r" U (jllm::\w+)\(", called))
    internal = {"quantize_q8_1", "gemm_q4k_mmq_llama", "gemm_q6k_mmq_llama"}   # gemv_q4.cu:468, :2462, :2470
    assert undefined == {"jllm::" + n for n in (REFERENCE_HEADER_FUNCTIONS - REGISTRY) | internal}
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "engine link ok" in r.stdout, r.stdout + r.stderr


def test_status_strings():
    l = jllm.lib()
    assert l.jllm_hip_status_string(0) == b"ok"
    assert b"unsupported" in l.jllm_hip_status_string(-2)
    assert l.jllm_hip_status_string(-99) == b"unknown status"


def test_mapped_weight_registry():
    # model.cpp:24-66 semantics: a pointer inside a registered host range maps
    # to the device alias at the same offset; outside -> NULL; clear removes.
    l = jllm.lib()
    host = ctypes.create_string_buffer(4096)
    hb = ctypes.addressof(host)
    dev = 0x7F0000000000
    assert l.jllm_hip_register_mapped_weight_region(hb, dev, 4096) == 0
    assert l.jllm_hip_resolve_mapped_weight_device_ptr(hb + 100) == dev + 100
    assert l.jllm_hip_resolve_mapped_weight_device_ptr(hb + 4096) is None
    assert l.jllm_hip_register_mapped_weight_region(None, dev, 10) == -1
    l.jllm_hip_clear_mapped_weight_region(hb)
    assert l.jllm_hip_resolve_mapped_weight_device_ptr(hb + 100) is None


def test_split_policy_host_only():
    l = jllm.lib()
    assert [l.jllm_hip_decode_attn_splits(s) for s in (0, 1, 32, 33, 512, 8192, 20000)] == [1, 1, 1, 2, 16, 128, 128]


def test_argument_validation_without_gpu():
    # shape / type checks happen before any HIP call
    l = jllm.lib()
    assert l.jllm_hip_gemv_quant(None, None, 13, None, 4, 256, None) != 0
    assert l.jllm_hip_gemm_quant_batched(None, None, 12, None, 4, 4, 300, None) == -1
    assert l.jllm_hip_quantize_mmq_q8_1(None, None, 1, 128, 64, 1, None) == -1
    import ctypes
    ys, ws = (ctypes.c_void_p * 4)(), (ctypes.c_void_p * 4)()
    ts, ms = (ctypes.c_int * 4)(12, 12, 12, 12), (ctypes.c_int * 4)(256, 256, 256, 256)
    args = [ctypes.cast(a, ctypes.c_void_p) for a in (ys, ws, ts, ms)]
    assert l.jllm_hip_gemm_quant_batched_multi(*args, 4, None, 8, 256, None) == -1      # more than 3 products
    assert l.jllm_hip_gemm_quant_batched_multi(*args, 0, None, 8, 256, None) == -1      # none
    assert l.jllm_hip_gemm_quant_batched_multi(*args, 2, None, 8, 300, None) == -1      # K % 256
    assert l.jllm_hip_gemm_quant_batched_multi(None, None, None, None, 2, None, 8, 256, None) == -1


def test_layer_op_argument_validation_without_gpu():
    l = jllm.lib()
    assert l.jllm_hip_fused_rmsnorm_residual(None, None, None, None, 1, 255, 1e-6, 1, None) == -1   # odd dim
    assert l.jllm_hip_fused_rmsnorm_residual(None, None, None, None, 0, 256, 1e-6, 1, None) == 0    # no rows
    assert l.jllm_hip_rope_inplace(None, None, 4, 2, 130, 0, 1e6, 1, None) == -1                   # hd > 128
    assert l.jllm_hip_rope_precompute_table(4096, 128, 1e6) == 0
    assert l.jllm_hip_qk_norm_rope_store_kv(None, None, None, None, None, 1, 1e-6, None, None, None, None,
                                            1024, 32, 8, 128, 64, 0, 1, 1e6, 1, 1, None) == -1    # chd < hd
    assert l.jllm_hip_dequant_embedding_row(None, None, 13, 0, 2560, None) == -2
    assert l.jllm_hip_dequant_embedding_rows(None, None, 12, None, 4, 2560, 0, None) == -1          # vocab 0
    assert l.jllm_hip_argmax_f32(None, None, 10, None) == -1
    assert l.jllm_hip_flash_attention_prefill_batched(None, None, None, None, 32, 8, 128, 128, 0, 0, 1.0, 1,
                                                      None, None, 0, None) == 0                     # N = 0


def test_pointer_returning_entry_points_keep_64_bit_results():
    """Every declaration of jllm_hip.h that returns a pointer is bound with a
    pointer restype in jllm.SIGNATURES itself (the ctypes default, int,
    would truncate the handle to 32 bits), whatever was imported first."""
    hdr = open(os.path.join(ROOT, "include", "jllm_hip.h")).read()
    ptr_fns = re.findall(r"^[\w ]*\*\s*(jllm_hip_\w+)\s*\(", hdr, re.M)
    assert "jllm_hip_decoder_create" in ptr_fns and "jllm_hip_get_splitk_partials" in ptr_fns
    for n in ptr_fns:
        assert jllm.SIGNATURES[n][0] in (ctypes.c_void_p, ctypes.c_char_p), n
        assert getattr(jllm.lib(), n).restype in (ctypes.c_void_p, ctypes.c_char_p), n


def test_zero_fill_size_helper(tmp_path):
    """The C++ layer's zero fill on an error path is sized by fill_bytes:
    0 for a negative dimension or a product over 2^40 bytes, the exact byte
    count otherwise (the reference's invalid sizes write nothing,
    gemv_q4.cu:2633-2775)."""
    exe = tmp_path / "fill_size_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "genie-ai-runtime_amd", "csrc"),
                    os.path.join(ROOT, "tests", "cxx", "fill_size_test.cpp"), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == [19456, 0, 0, 0, 0, 0, 1 << 40, 0, 0, 4194304, 1016]
