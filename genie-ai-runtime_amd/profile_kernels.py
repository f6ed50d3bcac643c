"""Workloads for rocprofv3 counter runs (run under `rocprofv3 --pmc ... -- python3 ...`).

  pair  : the decode gate/up pair GEMV (Q4_K 2 x 9728 x 2560) over 36 distinct
          layers' weights, 3 passes -- the dominant kernel of bench.py
  lmhead: the Q6_K lm_head GEMV (151936 x 2560, fp32 out), 4 distinct copies
  e2e   : the Qwen3-4B-shaped Q4_K_M decoder (36 layers, INT8 KV): prefill
          of a 512-token prompt, then 32 greedy decode steps
  attnp : INT8-KV prefill attention of 512 tokens at position 0 (32 q / 8 KV
          heads, head_dim 128), 5 calls
  copy  : a plain device-to-device copy of 256 MiB (calibrates FETCH_SIZE /
          WRITE_SIZE against a known byte count)
  mmq   : the Q4_K prefill GEMM 9728 x 2560 at N = 512 tokens (fp16 out), 5 calls
  mmq6  : the Q6_K prefill GEMM 2560 x 9728 at N = 512 tokens (fp16 out), 5 calls
  attn  : INT8-KV split-K decode attention (32 q / 8 KV heads, head_dim 128) at
          ctx 8192 over 16 distinct caches (277 MB), 2 passes; then ctx 512
          over 240 caches (263 MB), 2 passes
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def main(mode):
    import numpy as np
    import torch
    import jllm
    import synth
    dev = torch.device("cuda:0")
    g = synth.rng(99)

    def up(a):
        a = np.ascontiguousarray(a)
        return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)

    if mode == "pair":
        gate, upw = up(synth.q4k(g, 9728, 2560)), up(synth.q4k(g, 9728, 2560))
        layers = [(gate.clone(), upw.clone()) for _ in range(36)]
        x = up(synth.x_f16(g, 2560))
        y0 = torch.empty(9728, dtype=torch.int16, device=dev)
        y1 = torch.empty(9728, dtype=torch.int16, device=dev)
        for _ in range(3):
            for gw, uw in layers:
                jllm.gemv_quant_pair(y0, gw, 12, 9728, y1, uw, 12, 9728, x, 2560)
    elif mode == "lmhead":
        w = up(synth.q6k(g, 151936, 2560))
        ws = [w] + [w.clone() for _ in range(3)]
        x = up(synth.x_f16(g, 2560))
        y = torch.empty(151936, dtype=torch.float32, device=dev)
        for _ in range(3):
            for wi in ws:
                jllm.gemv_quant_f32(y, wi, 14, x, 151936, 2560)
    elif mode == "e2e":
        import decoder
        shape = decoder.QWEN3_4B
        model = decoder.synth_device(shape, 4242, dev)
        d = decoder.Decoder(shape, model, 640, max_batch=512)
        prompt = torch.randint(0, shape.vocab_size, (512,), dtype=torch.int32, device=dev,
                               generator=torch.Generator(device=dev).manual_seed(1))
        toks = torch.zeros(33, dtype=torch.int32, device=dev)
        d.generate(prompt, 33, toks)
        torch.cuda.synchronize()
        d.close()
    elif mode == "mmq":
        W = up(synth.q4k(g, 9728, 2560))
        x = up(synth.x_f16(g, (512, 2560)))
        y = torch.empty(512 * 9728, dtype=torch.int16, device=dev)
        for _ in range(5):
            jllm.call("jllm_hip_gemm_quant_batched", y, W, 12, x, 9728, 512, 2560)
    elif mode == "mmq6":
        W = up(synth.q6k(g, 2560, 9728))
        x = up(synth.x_f16(g, (512, 9728)))
        y = torch.empty(512 * 2560, dtype=torch.int16, device=dev)
        for _ in range(5):
            jllm.call("jllm_hip_gemm_quant_batched", y, W, 14, x, 2560, 512, 9728)
    elif mode == "attn":
        H, KV, HD = 32, 8, 128
        q = up(synth.x_f16(g, H * HD))
        out = torch.empty(H * HD, dtype=torch.int16, device=dev)
        for ctx, n in ((8192, 16), (512, 240)):
            k0, v0 = up(synth.kv_int8(g, ctx, KV, HD)), up(synth.kv_int8(g, ctx, KV, HD))
            s0 = up(synth.kv_scales(g, ctx, KV))
            caches = [(k0.clone(), v0.clone(), s0.clone()) for _ in range(n)]
            for _ in range(2):
                for k, v, s in caches:
                    jllm.call("jllm_hip_flash_attention_decode", out, q, k, v, H, KV, HD, HD, ctx, 0.0884, 1,
                              s, s, 0)
            torch.cuda.synchronize()
            del caches
    elif mode == "attnp":
        H, KV, HD, N = 32, 8, 128, 512
        q = up(synth.x_f16(g, N * H * HD))
        out = torch.empty(N * H * HD, dtype=torch.int16, device=dev)
        k, v, s = up(synth.kv_int8(g, N, KV, HD)), up(synth.kv_int8(g, N, KV, HD)), up(synth.kv_scales(g, N, KV))
        for _ in range(5):
            jllm.call("jllm_hip_flash_attention_prefill_batched", out, q, k, v, H, KV, HD, HD, N, 0, 0.0884, 1,
                      s, s, 0)
    elif mode == "copy":
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
    torch.cuda.synchronize()
    print("done", mode)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "pair")
