"""Benchmark of the MI355X quantized-matmul hot path (one GPU).

Headline (BASELINE.json metric, configs[1]): Q4_K/Q6_K decode GEMV HBM
bandwidth.  One step = the GEMV set of one decode token of a Qwen3-4B-shaped
model: for each of 36 layers (distinct weights, so the 2.6 GB working set
streams from HBM, not the 256 MB Infinity Cache) QKV triple (Q4_K
4096/1024/1024 x 2560), O + residual (Q4_K 2560 x 4096), gate/up pair (Q4_K
2 x 9728 x 2560), down + residual (Q6_K 2560 x 9728); then the Q6_K lm_head
(151936 x 2560, fp32 logits).  Inputs are resident in HBM before timing;
steps are replayed from a HIP graph.  value = algorithmic bytes / time.

Also reported in the same JSON line: the roofline of the dominant kernel
(gate/up pair GEMV, timed on its stream with HIP events), the int8 MMQ
prefill GEMM, INT8-KV split-K decode attention,
the end-to-end greedy decoder (configs[4]: TTFT, prefill and decode tok/s),
and the CPU baseline (the oracle's restatement of the reference's host
scalar GEMV, configs[0] shape, bounded sample).
"""
import argparse
import faulthandler
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "genie-ai-runtime_amd"), os.path.join(ROOT, "oracle")]

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
L, HID, QD, KVD, FFN, VOCAB = 36, 2560, 4096, 1024, 9728, 151936
Q4, Q6 = 12, 14
BB = {Q4: 144, Q6: 210}


def mat_bytes(t, rows, K):
    return rows * (K // 256) * BB[t]


def stage(msg):
    """Progress marker on stderr (the JSON result is the only stdout line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    faulthandler.enable()
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--skip-extras", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the hot path would shard by weight rows / KV heads, see DESIGN.md); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import jllm
    import synth

    dev = torch.device("cuda:0")
    stage("init cuda:0")
    torch.cuda.set_device(dev)
    g = synth.rng(20260101)

    def up(a):
        a = np.ascontiguousarray(a)
        return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)

    # ---- weights: one random layer, replicated to 36 distinct device copies
    base = {
        "q": up(synth.q4k(g, QD, HID)), "k": up(synth.q4k(g, KVD, HID)), "v": up(synth.q4k(g, KVD, HID)),
        "o": up(synth.q4k(g, HID, QD)), "gate": up(synth.q4k(g, FFN, HID)), "up": up(synth.q4k(g, FFN, HID)),
        "down": up(synth.q6k(g, HID, FFN)),
    }
    layers = [{k: v.clone() for k, v in base.items()} for _ in range(L)]
    del base
    lm_head = up(synth.q6k(g, VOCAB, HID))
    x_h, x_o, x_f = up(synth.x_f16(g, HID)), up(synth.x_f16(g, QD)), up(synth.x_f16(g, FFN))
    res = up(synth.x_f16(g, HID))
    yq, yk, yv = (torch.empty(n, dtype=torch.int16, device=dev) for n in (QD, KVD, KVD))
    yo, yd = torch.empty(HID, dtype=torch.int16, device=dev), torch.empty(HID, dtype=torch.int16, device=dev)
    yg, yu = torch.empty(FFN, dtype=torch.int16, device=dev), torch.empty(FFN, dtype=torch.int16, device=dev)
    logits = torch.empty(VOCAB, dtype=torch.float32, device=dev)

    layer_bytes = (mat_bytes(Q4, QD, HID) + 2 * mat_bytes(Q4, KVD, HID) + mat_bytes(Q4, HID, QD)
                   + 2 * mat_bytes(Q4, FFN, HID) + mat_bytes(Q6, HID, FFN))
    vec_bytes_layer = 2 * (HID * 3 + QD + KVD * 2 + QD + HID * 2 + HID * 3 + FFN * 2 + FFN + HID * 2)
    step_bytes = L * (layer_bytes + vec_bytes_layer) + mat_bytes(Q6, VOCAB, HID) + 2 * HID + 4 * VOCAB

    stage("weights resident; eager GEMV step")

    def step():
        for Lw in layers:
            jllm.gemv_quant_triple(yq, Lw["q"], Q4, QD, yk, Lw["k"], Q4, KVD, yv, Lw["v"], Q4, KVD, x_h, HID)
            jllm.gemv_quant_add(yo, Lw["o"], Q4, x_o, res, HID, QD)
            jllm.gemv_quant_pair(yg, Lw["gate"], Q4, FFN, yu, Lw["up"], Q4, FFN, x_h, HID)
            jllm.gemv_quant_add(yd, Lw["down"], Q6, x_f, res, HID, FFN)
        jllm.gemv_quant_f32(logits, lm_head, Q6, x_h, VOCAB, HID)

    step()
    torch.cuda.synchronize()
    stage("graph capture of the GEMV step")
    eager_logits = logits.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    # graph replays must reproduce the eager result exactly, replay after replay
    for _ in range(3):
        logits.zero_()
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(logits, eager_logits):
            print("graph replay differs from eager execution", file=sys.stderr)
            sys.exit(1)

    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    value = step_bytes / (ms_step * 1e-3) / 1e9

    out = {
        "metric": "Q4_K/Q6_K decode GEMV HBM bandwidth (Qwen3-4B decode-step GEMV set, 36 layers + lm_head)",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k/q6_k weights; int8 dot (MMVQ) + fp32",
        "data": "synthetic (seeded; BASELINE distributions)",
        "config": {"workload": "configs[1]: decode-step GEMV set, Qwen3-4B shape, batch 1",
                   "layers": L, "hidden": HID, "ffn": FFN, "vocab": VOCAB, "bytes_per_step": step_bytes,
                   "parallelism": "single GPU", "hbm_frac": round(value / HBM_PEAK_GBS, 4),
                   "wall_s_timed": round(wall, 3)},
    }

    stage("timed; pair-kernel roofline")
    # ---- dominant kernel: the gate/up pair GEMV (36 launches on distinct weights)
    pair_bytes = 2 * mat_bytes(Q4, FFN, HID) + 2 * HID + 4 * FFN
    gp = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gp):
        for Lw in layers:
            jllm.gemv_quant_pair(yg, Lw["gate"], Q4, FFN, yu, Lw["up"], Q4, FFN, x_h, HID)
    gp.replay()
    torch.cuda.synchronize()
    e0.record()
    reps = 10
    for _ in range(reps):
        gp.replay()
    e1.record()
    torch.cuda.synchronize()
    us_launch = e0.elapsed_time(e1) * 1e3 / (reps * L)
    achieved = pair_bytes / (us_launch * 1e-6) / 1e9
    out["roofline"] = {"kernel": "gemv_stream_kernel<MMVQ, half out> (gate/up pair, Q4_K 2x9728x2560)",
                       "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                       "bytes_per_launch": pair_bytes, "us_per_launch": round(us_launch, 3)}

    if not args.skip_extras:
        stage("MMQ prefill GEMM")
        out["mmq"] = bench_mmq(np, torch, jllm, synth, up, dev, g)
        stage("decode attention")
        out["attention"] = bench_attention(np, torch, jllm, synth, up, dev, g)
        del layers, lm_head, graph, gp
        torch.cuda.empty_cache()
        stage("end-to-end decoder")
        out["e2e"] = bench_e2e(np, torch, dev)
    stage("CPU baseline")
    out["cpu_baseline"] = cpu_baseline(np, synth, args.cpu_seconds)
    print(json.dumps(out), flush=True)


def measured_traffic():
    """HBM bytes per pair launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (profiles/gemv_pair_traffic.md), or None if it is absent."""
    try:
        for line in open(os.path.join(ROOT, "profiles", "gemv_pair_traffic.md")):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def bench_mmq(np, torch, jllm, synth, up, dev, g):
    """int8 MMQ, Q4_K 9728 x 2560 (and Q6_K 2560 x 9728) at N tokens; fp16 y
    (the reference's gemm_quant_batched).  Ops = 2*N*M*K; timed calls include the
    activation quantiser launch."""
    res = {}
    for t, M, K in ((12, 9728, 2560), (14, 2560, 9728)):
        W = up(synth.weights(g, t, M, K))
        for N in (64, 512, 1261):
            x = up(synth.x_f16(g, (N, K)))
            y = torch.empty(N * M, dtype=torch.int16, device=dev)
            jllm.call("jllm_hip_gemm_quant_batched", y, W, t, x, M, N, K)
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for _ in range(10):
                    jllm.call("jllm_hip_gemm_quant_batched", y, W, t, x, M, N, K)
            gr.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            gr.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / 10
            tops = 2.0 * N * M * K / (us * 1e-6) / 1e12
            # algorithmic bytes: weights + the activation as q8_1 (36 B per 32) + fp16 y
            nbytes = mat_bytes(t, M, K) + N * K * 36 // 32 + N * M * 2
            gbs = nbytes / (us * 1e-6) / 1e9
            res[f"{'q4k' if t == 12 else 'q6k'}_M{M}_K{K}_N{N}"] = {
                "us": round(us, 2), "TOPS": round(tops, 2), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    return res


def bench_attention(np, torch, jllm, synth, up, dev, g):
    """32 q heads / 8 KV heads, head_dim 128, INT8 KV with fp32 per-token
    scales; 36 distinct layer caches per context so the KV streams from HBM.
    Algorithmic bytes = ctx_eff * (2*8*128 + 2*8*4) + 16 KiB (q and out)."""
    H, KV, HD = 32, 8, 128
    res = {}
    q = up(synth.x_f16(g, H * HD))
    out = torch.empty(H * HD, dtype=torch.int16, device=dev)
    for ctx, window in ((512, 0), (4096, 0), (8192, 0), (8192, 512)):
        k0 = up(synth.kv_int8(g, ctx, KV, HD))
        v0 = up(synth.kv_int8(g, ctx, KV, HD))
        s0 = up(synth.kv_scales(g, ctx, KV))
        caches = [(k0.clone(), v0.clone(), s0.clone(), s0.clone()) for _ in range(L)]
        jllm.call("jllm_hip_flash_attention_decode", out, q, *caches[0][:2], H, KV, HD, HD, ctx, 0.0884, 1,
                  caches[0][2], caches[0][3], window)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for c in caches:
                jllm.call("jllm_hip_flash_attention_decode", out, q, c[0], c[1], H, KV, HD, HD, ctx, 0.0884, 1,
                          c[2], c[3], window)
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (5 * L)
        eff = min(ctx, window) if window > 0 else ctx
        by = eff * (2 * KV * HD + 2 * KV * 4) + 2 * 8192
        res[f"ctx{ctx}_win{window}"] = {"us_per_call": round(us, 2), "GB/s": round(by / (us * 1e-6) / 1e9, 1),
                                        "hbm_frac": round(by / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        del caches
    return res


def bench_e2e(np, torch, dev, n_prompt=512, n_gen=128):
    """random-init Qwen3-4B-shaped decoder in Q4_K_M layout (36 layers,
    Q6_K lm_head and every other ffn_down, fp32 norms ~ 1+N(0,0.02), RoPE base 1e6,
    INT8 KV), a random 512-token prompt, then greedy decode to 128 tokens.  TTFT =
    prefill of the prompt + first-token sampling; decode tok/s over the remaining
    127 steps.  Everything runs through the decoder's C ABI on one stream."""
    import decoder
    shape = decoder.QWEN3_4B
    model = decoder.synth_device(shape, 4242, dev)
    torch.cuda.synchronize()
    d = decoder.Decoder(shape, model, n_prompt + n_gen, max_batch=n_prompt)
    prompt = torch.randint(0, shape.vocab_size, (n_prompt,), dtype=torch.int32, device=dev,
                           generator=torch.Generator(device=dev).manual_seed(1))
    toks = torch.zeros(n_gen, dtype=torch.int32, device=dev)
    d.generate(prompt, 8, toks)                                   # warm-up (code objects, allocations)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    ev[0].record()
    d.prefill(prompt, 0, toks[0:1])
    ev[1].record()
    for i in range(1, n_gen):
        d.step(toks[i - 1:i], n_prompt + i - 1, toks[i:i + 1])
    ev[2].record()
    torch.cuda.synchronize()
    ttft = ev[0].elapsed_time(ev[1])
    dec_ms = ev[1].elapsed_time(ev[2])
    gen = toks.cpu().numpy()
    d.close()
    del model
    torch.cuda.empty_cache()
    return {"workload": "configs[4]: Qwen3-4B-shaped Q4_K_M decoder, 36 layers, INT8 KV, prompt 512, "
                        "128 greedy tokens", "ttft_ms": round(ttft, 2),
            "prefill_tok_s": round(n_prompt / (ttft * 1e-3), 1),
            "decode_tok_s": round((n_gen - 1) / (dec_ms * 1e-3), 1),
            "decode_ms_per_token": round(dec_ms / (n_gen - 1), 3),
            "distinct_tokens": int(len(set(gen.tolist()))), "first_tokens": gen[:8].tolist()}


def cpu_baseline(np, synth, seconds):
    """The oracle's C restatement of the reference's host scalar path gemv_quant_cpu
    (gemv_q4.cu:2519-2631) on configs[0] (Q4_K 9728 x 2560, fp16 x, fp32 y), on this
    box's CPU: single thread (as the reference runs it), repeated for ~`seconds`."""
    import oracle
    g = synth.rng(7)
    M, K = 9728, 2560
    W, x = synth.q4k(g, M, K), synth.x_f16(g, K)
    by = mat_bytes(Q4, M, K) + 2 * K + 4 * M
    oracle.gemv_quant_cpu(W, Q4, x, M, K)
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.gemv_quant_cpu(W, Q4, x, M, K)
        calls += 1
    dt = (time.perf_counter() - t0) / calls
    threads = min(16, os.cpu_count() or 1)
    tm0, mcalls = time.perf_counter(), 0
    while time.perf_counter() - tm0 < max(1.0, seconds / 4):
        oracle.gemv_quant_cpu(W, Q4, x, M, K, threads=threads)
        mcalls += 1
    dtm = (time.perf_counter() - tm0) / mcalls
    return {"value": round(by / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"configs[0] Q4_K GEMV 9728x2560 (14.05 MB/call), {calls} calls, {dt * 1e3:.1f} ms/call",
            "all_cores": {"value": round(by / dtm / 1e9, 3), "unit": "GB/s", "cores": threads,
                          "ms_per_call": round(dtm * 1e3, 2)}}


if __name__ == "__main__":
    main()
