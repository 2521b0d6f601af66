"""Benchmark of the denoiser attention block hot path on one MI355X.

One step = one pass of the hot path at the 4608-token Boogu Turbo shape over resident synthetic
inputs: the four packed-Q4 projection GEMMs (M 4608; K x N = 3072x9216 QKV, 3072x3072 O,
3072x12288 MLP up, 12288x3072 MLP down; bf16 activations, f32 outputs) and the joint flash
attention (B1 H24 S4608 D128, bf16 Q/K/V, f32 output).  Prints one JSON line.  After the timed
steps it also times, as extra keys:
  * the fused SwiGLU projection (both 3072x12288 up weights in one pass);
  * the whole modulated denoise block (SingleStreamBlock.forward: modulation GEMV, three glue
    passes, the QKV projection with the Q/K norm + RoPE epilogue, attention, O, fused SwiGLU,
    down) at
    4608 tokens x hidden 3072, 24 heads of 128, SwiGLU 12288, bf16 activations
    (`ms_per_denoise_block`), next to the sum of its GEMM and attention kernels;
  * the small-M route (one modulation row, 1 x 3072 x 12288, and 16 x 3072 x 9216) in GB/s over
    >= 1 GB of rotating weights, replayed from a HIP graph.

    python bench.py [--steps 20] [--warmup 3] [--no-cpu] [--cpu-runs 5]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16/fp16 MFMA
PEAK_HBM_GBS = 8000.0

M_TOKENS = 4608
GEMMS = [("qkv", 3072, 9216), ("o", 3072, 3072), ("mlp_up", 3072, 12288), ("mlp_down", 12288, 3072)]
ATTN = dict(B=1, H=24, S=4608, D=128)


def gemm_flops(M, K, N):
    return 2.0 * M * K * N


def attn_flops(B, H, S, D):
    return 4.0 * B * H * D * S * S


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_gemm_attention_4608tok_hbm_traffic.json")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes (copy-kernel calibrated); None when that measurement is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if kernel == "q4_gemm":
        return t.get("q4_gemm_traffic_bytes_per_launch")
    return t.get("per_launch", {}).get(kernel, {}).get("traffic_bytes")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-rows", type=int, default=4608,
                    help="query rows / activation rows of the CPU sample (4608 = the whole step)")
    ap.add_argument("--cpu-runs", type=int, default=5,
                    help="timed CPU runs per op after one warm-up run (the median is reported)")
    return ap.parse_args()


def cpu_baseline(args, words_np, scales_np, x_np, q_np, k_np, v_np):
    """Restated Burn NdArray CPU path on the same workload: the four Q4 GEMMs over the first
    `cpu_rows` activation rows (dequantise + f32 matmul) and the joint attention over the first
    `cpu_rows` query rows of every head (query-chunked f32 softmax).  By default `cpu_rows` is
    all 4608 rows, so one whole step is timed (a few seconds on 16 host threads); a smaller
    sample times each op on its rows and extrapolates the step op by op."""
    from oracle import oracle as O
    O.build()
    rows = args.cpu_rows
    runs = max(1, args.cpu_runs)
    t_total = 0.0
    threads = 1
    detail = {}

    def median_time(fn):
        fn()  # warm-up (page-in, thread pool start)
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    for (name, K, N) in GEMMS:
        xs = np.ascontiguousarray(x_np[name][:rows])
        box = {}
        dt = median_time(lambda: box.update(t=O.cpu_q4_linear_f32(xs, words_np[name], scales_np[name], 1, 128, N)[1]))
        threads = box["t"]
        rate = gemm_flops(rows, K, N) / dt
        detail[name] = rate / 1e12
        t_total += gemm_flops(M_TOKENS, K, N) / rate
    dt = median_time(lambda: O.cpu_attention_f32(q_np, k_np, v_np, requested_chunk=8192, q_rows=rows))
    rate = (4.0 * ATTN["H"] * ATTN["D"] * rows * ATTN["S"]) / dt
    detail["attention"] = rate / 1e12
    t_total += attn_flops(**ATTN) / rate
    step_flops = sum(gemm_flops(M_TOKENS, K, N) for _, K, N in GEMMS) + attn_flops(**ATTN)
    if rows >= M_TOKENS:
        scope = ("the whole step: all 4608 rows of each Q4 GEMM and all 4608 query rows x 24 heads "
                 "of the attention")
    else:
        scope = (f"the first {rows} of 4608 rows of each Q4 GEMM and {rows} query rows x 24 heads "
                 f"of the attention; per-op rates extrapolated to one full step")
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": step_flops / t_total / 1e12,
        "unit": "TFLOP/s",
        "cores": int(threads),
        "kind": "port",
        "sample": ("restated Burn NdArray CPU path (dequantise + f32 matmul; query-chunked f32 "
                   "attention, chunk policy of attention.rs:36-45) on " + scope +
                   f"; median of {runs} runs per op after one warm-up"),
        "cpu_model": cpu_model,
        "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
        "nproc": os.cpu_count(),
        "per_op_tflops": {k: round(v, 5) for k, v in detail.items()},
        "ms_per_step": t_total * 1e3,
    }


def time_denoise_block(B, W, dev, weights, w3, args):
    """SingleStreamBlock.forward (block.rs:84-134) at 4608 x 3072: modulation GEMV, three glue
    passes, the QKV projection with the Q/K norm + RoPE epilogue, attention, O, fused SwiGLU,
    down; bf16 activations.
    Returns the mean ms per forward (events around each call)."""
    import torch
    from burn_image_amd import block as BL
    from burn_image_amd import rope as R
    Wd, H, D, C = 3072, 24, 128, 1024
    ones = lambda n: torch.ones(n, device=dev)  # noqa: E731
    wm, sm = W.q4_weight(3, 11, C, 4 * Wd, layout=1)
    mod = B.from_packed(torch.from_numpy(wm.view(np.int32)).to(dev), torch.from_numpy(sm).to(dev), 1, 128, (C, 4 * Wd))
    attn = BL.GqaAttention(None, None, None, B.Linear(weights["o"]), B.RmsNorm(ones(D)), B.RmsNorm(ones(D)),
                           H, H, D, qkv=B.Linear(weights["qkv"]))
    blk = BL.SingleStreamBlock(
        norm1=BL.RmsNormZero(B.Linear(mod, torch.zeros(4 * Wd, device=dev)), B.RmsNorm(ones(Wd))),
        attn=attn, norm2=B.RmsNorm(ones(Wd)), ffn_norm1=B.RmsNorm(ones(Wd)), ffn_norm2=B.RmsNorm(ones(Wd)),
        feed_forward=B.LuminaFeedForward(B.Linear(weights["mlp_up"]), B.Linear(weights["mlp_down"]), B.Linear(w3)),
        activation_dtype=torch.bfloat16)
    ids = W.boogu_joint_ids(2)
    cos, sin = R.rope_values(ids, [32, 48, 48], 1.0e4)
    rope = (torch.from_numpy(cos[None]).to(dev), torch.from_numpy(sin[None]).to(dev))
    gen = torch.Generator(device=dev).manual_seed(7)
    tokens = torch.randn((1, M_TOKENS, Wd), device=dev, generator=gen)
    cond = torch.randn((1, C), device=dev, generator=gen)
    for _ in range(args.warmup):
        blk.forward(tokens, rope, cond)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for e0, e1 in evs:
        e0.record(stream)
        blk.forward(tokens, rope, cond)
        e1.record(stream)
    torch.cuda.synchronize()
    return float(np.mean([e0.elapsed_time(e1) for e0, e1 in evs]))


def time_released(B, dev):
    """The reference's own throughput harnesses, at the released model's geometry:
    * packed-Q4 projection 9261 x 3360 x 3360, f32 activations, weights quantised from the
      harness's pattern by the Boogu quantizer (block 32 for K = 3360), fastest of 3 timed calls
      after a warm-up (artifacts.rs:10588-10655);
    * the 1.5K fused Q/K norm + RoPE + attention, 28 query / 4 key-value heads, S = 18579, D = 120,
      f32 in and out, median of 5 timed calls after a warm-up (native_flash.rs:3736-3823; here
      through execute_gqa_with_qk_norm_rope on token-major tensors).
    Events around each call on the current stream."""
    import torch
    out = {}
    stream = torch.cuda.current_stream(dev)
    gen = torch.Generator(device=dev).manual_seed(13)

    def timed(fn, n):
        fn()
        torch.cuda.synchronize()
        ms = []
        for _ in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1))
        return ms

    M, K, N = 9261, 3360, 3360
    idx = torch.arange(K * N, device=dev)
    w = ((((idx // N) + (idx % N) * 3) % 15).to(torch.float32) - 7.0) * (1.0 / 64.0)
    q = B.quantize_row_layout_q4s_block_up_to128_f32(w.reshape(K, N))
    x = torch.randn((M, K), device=dev, generator=gen)
    y = torch.empty((M, N), device=dev)
    ms = min(timed(lambda: B.q_matmul(x, q, out=y), 3))
    fl = gemm_flops(M, K, N)
    out["q4_9261x3360x3360"] = {"ms": round(ms, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
                                "frac_peak": round(fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                                "block": q.block, "x_dtype": "f32", "timing": "fastest of 3"}
    del x, y, q, w, idx
    S, Hq, Hkv, D = 18579, 28, 4, 120
    qt = torch.randn((1, S, Hq, D), device=dev, generator=gen)
    kt = torch.randn((1, S, Hkv, D), device=dev, generator=gen)
    vt = torch.randn((1, S, Hkv, D), device=dev, generator=gen)
    nq, nk = B.RmsNorm(torch.ones(D, device=dev)), B.RmsNorm(torch.ones(D, device=dev))
    rope = (torch.ones((1, S, D), device=dev), torch.zeros((1, S, D), device=dev))
    run = lambda: B.NativeQ4FlashAttention.execute_gqa_with_qk_norm_rope(qt, kt, vt, nq, nk, rope, 16384)  # noqa: E731
    ms = float(np.median(timed(run, 5)))
    fl = attn_flops(B=1, H=Hq, S=S, D=D)
    out["attention_1k5_s18579_h28_kv4_d120"] = {
        "ms": round(ms, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
        "frac_peak": round(fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "includes": "fused Q/K norm + RoPE prep (f32 -> f16) and attention (f32 out)", "timing": "median of 5"}
    del qt, kt, vt
    torch.cuda.empty_cache()
    return out


def time_small_m(B, dev):
    """The small-M route at the modulation rows (1 x 3072 x 12288 block 128, the 3072-wide step's
    RmsNormZero projection, and 1 x 3360 x 13440 block 32, the released model's; f32 activations)
    and at 16 x 3072 x 9216 (bf16 activations), each over >= 1 GB of distinct weights (the 256 MB
    MALL cannot hold them), replayed from a HIP graph; GB/s = algorithmic bytes / time."""
    import torch
    out = {}
    gen = torch.Generator(device=dev).manual_seed(11)
    for (M, K, N, blk, xdt) in ((1, 3072, 12288, 128, torch.float32), (1, 3360, 13440, 32, torch.float32),
                                (16, 3072, 9216, 128, torch.bfloat16)):
        wbytes = K * N // 2 + (K // blk) * N * 4
        copies = int(np.ceil(1.0e9 / wbytes))
        ws = [B.from_packed(torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), dtype=torch.int32, device=dev,
                                          generator=gen),
                            torch.rand((K // blk, N), device=dev, generator=gen) * 0.015 + 0.005, 1, blk, (K, N))
              for _ in range(copies)]
        x = torch.randn((M, K), device=dev, generator=gen).to(xdt)
        y = torch.empty((M, N), device=dev)
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            B.q_matmul(x, ws[0], out=y)  # sizes the stream's workspace outside capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for w in ws:
                B.q_matmul(x, w, out=y)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / copies
        nbytes = wbytes + M * K * x.element_size() + M * N * 4
        out[f"{M}x{K}x{N}" + ("" if blk == 128 else f"_blk{blk}")] = {"us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1),
                               "frac_hbm": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4),
                               "weight_copies": copies}
        del ws, graph
        torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the hot path is measured on "
                                   "a single MI355X; --gpus above 1 is not supported"}))
        sys.exit(2)
    import torch

    import burn_image_amd as B
    from burn_image_amd import workloads as W

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    gen = torch.Generator(device=dev).manual_seed(1234)

    # ---------------- resident synthetic inputs -------------------------------------------
    weights, xs, outs = {}, {}, {}
    words_np, scales_np, x_np = {}, {}, {}
    for i, (name, K, N) in enumerate(GEMMS):
        wn, sn = W.q4_weight(3, 2 * i + 1, K, N, layout=1)
        words_np[name], scales_np[name] = wn, sn
        weights[name] = B.from_packed(torch.from_numpy(wn.view(np.int32)).to(dev),
                                      torch.from_numpy(sn).to(dev), 1, 128, (K, N))
        xn = W.activations(3, 2 * i, M_TOKENS, K, "bf16")
        x_np[name] = xn
        xs[name] = torch.from_numpy(xn).to(torch.bfloat16).to(dev)
        outs[name] = torch.empty((M_TOKENS, N), dtype=torch.float32, device=dev)
    q_np, k_np, v_np = W.boogu_attention(2)
    q, k, v = (torch.from_numpy(a).to(torch.bfloat16).to(dev) for a in (q_np, k_np, v_np))
    o = torch.empty((1, 24, 4608, 128), dtype=torch.float32, device=dev)

    ops = [(name, (lambda n=name: B.q_matmul(xs[n], weights[n], out=outs[n]))) for name, _, _ in GEMMS[:1]]
    ops.append(("attention", lambda: B.attention(q, k, v, out=o)))
    ops += [(name, (lambda n=name: B.q_matmul(xs[n], weights[n], out=outs[n]))) for name, _, _ in GEMMS[1:]]
    flops = {name: gemm_flops(M_TOKENS, K, N) for name, K, N in GEMMS}
    flops["attention"] = attn_flops(**ATTN)
    step_flops = sum(flops.values())

    for _ in range(args.warmup):
        for _, fn in ops:
            fn()
    torch.cuda.synchronize()

    # ---------------- timed region: K steps, events around every launch --------------------
    stream = torch.cuda.current_stream(dev)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(ops) + 1)] for _ in range(args.steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for s in range(args.steps):
        evs[s][0].record(stream)
        for j, (_, fn) in enumerate(ops):
            fn()
            evs[s][j + 1].record(stream)
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms_per_step = total_ms / args.steps
    per_op_ms = {name: float(np.mean([evs[s][j].elapsed_time(evs[s][j + 1]) for s in range(args.steps)]))
                 for j, (name, _) in enumerate(ops)}

    # ---------------- fused SwiGLU (outside the step): silu(x W1) * (x W3) at the MLP-up shape,
    # the reference block's two up projections in one pass (feed_forward.rs:32-36) -----------
    _, Ku, Nu = GEMMS[2]
    w3n, s3n = W.q4_weight(3, 9, Ku, Nu, layout=1)
    w3 = B.from_packed(torch.from_numpy(w3n.view(np.int32)).to(dev), torch.from_numpy(s3n).to(dev),
                       1, 128, (Ku, Nu))
    gated = torch.empty((M_TOKENS, Nu), dtype=torch.bfloat16, device=dev)
    glu = lambda: B.q_matmul_swiglu(xs["mlp_up"], weights["mlp_up"], w3, out=gated)  # noqa: E731
    for _ in range(args.warmup):
        glu()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    g0.record(stream)
    for _ in range(args.steps):
        glu()
    g1.record(stream)
    torch.cuda.synchronize()
    glu_ms = g0.elapsed_time(g1) / args.steps
    glu_fl = 2 * gemm_flops(M_TOKENS, Ku, Nu)

    block_measured_ms = time_denoise_block(B, W, dev, weights, w3, args)
    small_m = time_small_m(B, dev)
    released = time_released(B, dev)

    gemm_ms = sum(per_op_ms[n] for n, _, _ in GEMMS)
    gemm_fl = sum(flops[n] for n, _, _ in GEMMS)
    attn_ms = per_op_ms["attention"]
    per_kernel = {n: {"ms": round(per_op_ms[n], 4),
                      "tflops": round(flops[n] / (per_op_ms[n] * 1e-3) / 1e12, 2),
                      "frac_peak": round(flops[n] / (per_op_ms[n] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
                  for n in per_op_ms}
    if gemm_ms >= attn_ms:
        dom, dom_fl, dom_ms, dom_launches = "q4_gemm", gemm_fl, gemm_ms, len(GEMMS)
    else:
        dom, dom_fl, dom_ms, dom_launches = "attention", flops["attention"], attn_ms, 1
    achieved = dom_fl / (dom_ms * 1e-3) / 1e12
    # Sum of the block's GEMM and attention kernels (block.rs:84-134 via feed_forward.rs:32-36):
    # QKV + attention + O + two SwiGLU up projections + down, from the step's kernel times.
    block_ms = per_op_ms["qkv"] + attn_ms + per_op_ms["o"] + 2 * per_op_ms["mlp_up"] + per_op_ms["mlp_down"]

    result = {
        "metric": "attn + Q4-GEMM TFLOP/s and % MFMA peak @4608-tok DiT; ms per denoise block",
        "value": round(step_flops / (ms_per_step * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "boogu-turbo-1024px-4608tok: Q4 QKV/O/MLP-up/MLP-down GEMMs "
                               "(M4608, hidden 3072, block-128 f32 scales, bf16 activations) + "
                               "joint attention B1 H24 S4608 D128 bf16",
                   "tokens": M_TOKENS, "hidden": 3072, "heads": 24, "head_dim": 128,
                   "parallelism": "single-gpu"},
        "frac_peak": round(step_flops / (ms_per_step * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "ms_per_denoise_block": round(block_measured_ms, 4),
        "denoise_block": ("SingleStreamBlock.forward measured end to end (events): modulation GEMV, "
                          "3 glue passes, QKV projection with the Q/K norm+RoPE epilogue, attention, O, fused SwiGLU, down; "
                          "4608 tok x 3072, 24x128 heads, SwiGLU 12288, bf16 activations"),
        "denoise_block_tflops": round(1.652e12 / (block_measured_ms * 1e-3) / 1e12, 2),
        "ms_sum_block_kernels": round(block_ms, 4),
        "ms_sum_block_kernels_1xup": round(block_ms - per_op_ms["mlp_up"], 4),
        "ms_sum_block_kernels_fused_swiglu": round(
            per_op_ms["qkv"] + attn_ms + per_op_ms["o"] + glu_ms + per_op_ms["mlp_down"], 4),
        "small_m": small_m,
        "released_geometry": released,
        "per_kernel": per_kernel,
        "fused_swiglu": {"ms": round(glu_ms, 4), "tflops": round(glu_fl / (glu_ms * 1e-3) / 1e12, 2),
                         "frac_peak": round(glu_fl / (glu_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                         "shape": f"M{M_TOKENS} K{Ku} N{Nu} x2 weights, bf16 in, bf16 gated out"},
        "roofline": {"bound": "mfma", "kernel": dom, "launches_per_step": dom_launches,
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic(dom)},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args, words_np, scales_np, x_np, q_np, k_np, v_np)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
