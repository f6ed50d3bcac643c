"""ctypes binding of libjllm_hip.so (the C ABI declared in include/jllm_hip.h).

Python is only the test/bench harness here: device buffers are torch
tensors on the GPU, passed by data_ptr(); every call goes through the C ABI
into the HIP kernels.  There is no fallback: if the library is missing,
loading raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("JLLM_HIP_LIB") or os.path.join(HERE, "libjllm_hip.so")

_lib = None
P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "jllm_hip_status_string": (ctypes.c_char_p, [I]),
    "jllm_hip_register_mapped_weight_region": (I, [P, P, I64]),
    "jllm_hip_clear_mapped_weight_region": (None, [P]),
    "jllm_hip_resolve_mapped_weight_device_ptr": (P, [P]),
    "jllm_hip_gemv_quant": (I, [P, P, I, P, I, I, P]),
    "jllm_hip_gemv_quant_add": (I, [P, P, I, P, P, I, I, P]),
    "jllm_hip_gemv_quant_pair": (I, [P, P, I, I, P, P, I, I, P, I, P]),
    "jllm_hip_gemv_quant_triple": (I, [P, P, I, I, P, P, I, I, P, P, I, I, P, I, P]),
    "jllm_hip_gemv_quant_f32": (I, [P, P, I, P, I, I, P]),
    "jllm_hip_gemv_quant_dequant_f32": (I, [P, P, I, P, I, I, P]),
    "jllm_hip_quantize_q8_1": (I, [P, P, I, P]),
    "jllm_hip_gemv_quant_triple_rmsnorm": (I, [P, P, I, I, P, P, I, I, P, P, I, I, P, P, I, F, I, P]),
    "jllm_hip_gemv_quant_pair_rmsnorm": (I, [P, P, I, I, P, P, I, I, P, P, I, F, I, P]),
    "jllm_hip_quantize_mmq_f16": (I, [P, P, P, I, I, I, I, P]),
    "jllm_hip_quantize_mmq_i8": (I, [P, P, P, I, I, I, I, P]),
    "jllm_hip_gemv_quant_pair_swiglu": (I, [P, P, I, P, I, I, P, I, P]),
    "jllm_hip_gemv_quant_pair_rmsnorm_swiglu": (I, [P, P, I, P, I, I, P, P, I, F, I, P]),
    "jllm_hip_gemv_quant_f32_rmsnorm": (I, [P, P, I, P, P, I, F, I, I, P]),
    "jllm_hip_gemm_quant_batched": (I, [P, P, I, P, I, I, I, P]),
    "jllm_hip_gemm_quant_batched_f32": (I, [P, P, I, P, I, I, I, P]),
    "jllm_hip_gemm_quant_batched_multi": (I, [P, P, P, P, I, P, I, I, P]),
    "jllm_hip_quantize_mmq_q8_1": (I, [P, P, I, I, I, I, P]),
    "jllm_hip_mmq_subdots": (I, [P, P, I, P, I, I, I, P]),
    "jllm_hip_flash_attention_decode": (I, [P, P, P, P, I, I, I, I, I, F, I, P, P, I, P]),
    "jllm_hip_flash_attention_decode_splits": (I, [P, P, P, P, I, I, I, I, I, F, I, P, P, I, I, P]),
    "jllm_hip_flash_attention_decode_dyn": (I, [P, P, P, P, I, I, I, I, P, F, I, P, P, I, I, P]),
    "jllm_hip_flash_attention_decode_noalloc": (I, [P, P, P, P, I, I, I, I, I, F, I, P, P, I, P]),
    "jllm_hip_decode_attn_splits": (I, [I]),
    "jllm_hip_get_splitk_partials": (P, [I, I, I]),
    "jllm_hip_fp16_to_int8": (I, [P, P, P, I, I, P]),
    "jllm_hip_flash_attention_prefill_batched": (I, [P, P, P, P, I, I, I, I, I, I, F, I, P, P, I, P]),
    "jllm_hip_fused_rmsnorm_residual": (I, [P, P, P, P, I, I, F, I, P]),
    "jllm_hip_fused_swiglu": (I, [P, P, P, I, I, P]),
    "jllm_hip_vec_add": (I, [P, P, P, I64, P]),
    "jllm_hip_rope_inplace": (I, [P, P, I, I, I, I, F, I, P]),
    "jllm_hip_rope_inplace_batched": (I, [P, P, I, I, I, I, I, I, I, F, I, P]),
    "jllm_hip_rope_inplace_dyn": (I, [P, P, I, I, I, P, F, I, P]),
    "jllm_hip_rope_inplace_store_kv_fp16_dyn": (I, [P, P, P, P, P, I, I, I, I, P, F, I, P]),
    "jllm_hip_rope_inplace_store_kv_fp16_batched": (I, [P, P, P, P, P, I, I, I, I, I, I, I, I, F, I, P]),
    "jllm_hip_rope_precompute_table": (I, [I, I, F]),
    "jllm_hip_rope_clear_tables": (None, []),
    "jllm_hip_qk_norm_rope_store_kv": (I, [P, P, P, P, P, I, F, P, P, P, P, I64, I, I, I, I, I, I, F, I, I, P]),
    "jllm_hip_dequant_embedding_row": (I, [P, P, I, I, I, P]),
    "jllm_hip_dequant_embedding_rows": (I, [P, P, I, P, I, I, I, P]),
    "jllm_hip_argmax_f32": (I, [P, P, I, P]),
    # outside the Llama/Qwen decode path (Gemma family, logits)
    "jllm_hip_fused_geglu": (I, [P, P, P, I, I, P]),
    "jllm_hip_vec_scale": (I, [P, I64, F, P]),
    "jllm_hip_logit_softcap": (I, [P, I64, F, P]),
    "jllm_hip_softmax_inplace": (I, [P, I, P]),
    "jllm_hip_gemv_dense": (I, [P, P, I, P, I, I, P]),
    "jllm_hip_gemm_dense_batched": (I, [P, P, I, P, I, I, I, P]),
    # GGUF reader / loader / writer
    "jllm_hip_gguf_open": (P, [ctypes.c_char_p]),
    "jllm_hip_gguf_close": (None, [P]),
    "jllm_hip_gguf_n_tensors": (I64, [P]),
    "jllm_hip_gguf_find_tensor": (I64, [P, ctypes.c_char_p]),
    "jllm_hip_gguf_tensor": (I, [P, I64, P, P, P, P, P, P]),
    "jllm_hip_gguf_get_u64": (I, [P, ctypes.c_char_p, P]),
    "jllm_hip_gguf_get_f64": (I, [P, ctypes.c_char_p, P]),
    "jllm_hip_gguf_get_str": (ctypes.c_char_p, [P, ctypes.c_char_p]),
    "jllm_hip_gguf_config": (I, [P, P]),
    "jllm_hip_gguf_model_load": (P, [P, P]),
    "jllm_hip_gguf_model_weights": (P, [P]),
    "jllm_hip_gguf_layer_weights": (P, [P]),
    "jllm_hip_gguf_model_free": (None, [P]),
    "jllm_hip_gguf_writer_create": (P, []),
    "jllm_hip_gguf_writer_free": (None, [P]),
    "jllm_hip_gguf_writer_set_u32": (I, [P, ctypes.c_char_p, ctypes.c_uint32]),
    "jllm_hip_gguf_writer_set_f32": (I, [P, ctypes.c_char_p, F]),
    "jllm_hip_gguf_writer_set_str": (I, [P, ctypes.c_char_p, ctypes.c_char_p]),
    "jllm_hip_gguf_writer_add_tensor": (I, [P, ctypes.c_char_p, I, I, P, P, I64]),
    "jllm_hip_gguf_writer_write": (I, [P, ctypes.c_char_p]),
    # decoder loop; the struct arguments are passed by address
    "jllm_hip_decoder_create": (P, [P, P, P, I]),
    "jllm_hip_decoder_destroy": (None, [P]),
    "jllm_hip_decoder_prefill": (I, [P, P, I, I, P, P]),
    "jllm_hip_decoder_step": (I, [P, P, I, P, P]),
    "jllm_hip_decoder_generate": (I, [P, P, I, I, P, P]),
    "jllm_hip_decoder_copy_logits": (I, [P, P, P]),
    "jllm_hip_decoder_layer": (I, [P, I, P, I, I, P]),
    "jllm_hip_decoder_copy_kv": (I, [P, I, I, P, P, P, P, P]),
    "jllm_hip_decoder_copy_act": (I, [P, I, I, P, P]),
}


class JllmError(RuntimeError):
    pass


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise JllmError(f"{LIB_PATH} is not built; run genie-ai-runtime_amd/build.py")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            if hasattr(l, name):
                fn = getattr(l, name)
                fn.restype = res
                fn.argtypes = args
        _lib = l
    return _lib


def _ptr(t):
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return ctypes.c_void_p(stream)


def check(status, what):
    if status != 0:
        msg = lib().jllm_hip_status_string(status).decode()
        raise JllmError(f"{what}: {msg} ({status})")


def call(name, *args, stream=None):
    conv = []
    for a in args:
        if hasattr(a, "data_ptr"):
            conv.append(_ptr(a))
        else:
            conv.append(a)
    st = getattr(lib(), name)(*conv, _stream(stream))
    check(st, name)


# convenience wrappers (tensor arguments)
def gemv_quant(y, W, t, x, M, K, stream=None):
    call("jllm_hip_gemv_quant", y, W, t, x, M, K, stream=stream)


def gemv_quant_f32(y, W, t, x, M, K, stream=None):
    call("jllm_hip_gemv_quant_f32", y, W, t, x, M, K, stream=stream)


def gemv_quant_dequant_f32(y, W, t, x, M, K, stream=None):
    call("jllm_hip_gemv_quant_dequant_f32", y, W, t, x, M, K, stream=stream)


def gemv_quant_add(y, W, t, x, res, M, K, stream=None):
    call("jllm_hip_gemv_quant_add", y, W, t, x, res, M, K, stream=stream)


def gemv_quant_pair(y0, W0, t0, M0, y1, W1, t1, M1, x, K, stream=None):
    call("jllm_hip_gemv_quant_pair", y0, W0, t0, M0, y1, W1, t1, M1, x, K, stream=stream)


def gemv_quant_triple(y0, W0, t0, M0, y1, W1, t1, M1, y2, W2, t2, M2, x, K, stream=None):
    call("jllm_hip_gemv_quant_triple", y0, W0, t0, M0, y1, W1, t1, M1, y2, W2, t2, M2, x, K, stream=stream)


def quantize_q8_1(x, y, K, stream=None):
    call("jllm_hip_quantize_q8_1", x, y, K, stream=stream)
