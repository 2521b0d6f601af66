"""Per-operator microbenchmarks of libbiq on one GPU (HIP-event timing, JSON output).

    python -m burn_image_amd.perf q4_linear --M 4608 --K 3072 --N 9216 [--layout 1] [--block 128]
                                            [--xdtype bf16] [--ydtype f32] [--iters 50] [--swiglu]
    python -m burn_image_amd.perf attention --B 1 --H 24 --Hkv 24 --S 4608 --D 128 [--dtype bf16]
                                            [--causal] [--segments 1024:64:512]
    python -m burn_image_amd.perf qk_prep --S 4608 --Hq 24 --Hkv 24 --D 128 [--dtype f32]
    python -m burn_image_amd.perf glue --S 4608 --W 3072 [--dtype bf16]
    python -m burn_image_amd.perf qkv_prep --S 4608 [--Hq 24 --Hkv 24]
    python -m burn_image_amd.perf block --S 4608   (SingleStreamBlock.forward, 3072 wide)
    python -m burn_image_amd.perf copy --mib 512   (a plain device copy of known size: the
                                                    calibration kernel for HBM byte counters)
    (every op also takes --iters, --warmup and --graph)

Inputs are random and resident on the GPU before timing; weights rotate over enough distinct
copies (``--rotate-bytes``, default 0) to defeat the 256 MB MALL when measuring HBM-bound shapes.
"""
from __future__ import annotations

import argparse
import json
import sys

import numpy as np
import torch

from . import _lib
from .attention import RmsNorm, attention, qk_norm_rope
from .linear import q_matmul, q_matmul_swiglu
from .q4 import from_packed

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
PEAK_TFLOPS = 2500.0
PEAK_GBS = 8000.0


_GRAPH = False


def _time(fn, iters: int, warmup: int) -> float:
    """Average microseconds per call.  With --graph the `iters` calls are captured once in a HIP
    graph and replayed, so short kernels are timed without the host's per-call cost between
    them (every call here writes a preallocated output and allocates nothing)."""
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if _GRAPH:
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):  # per-stream library state (workspace) is sized here
            fn(0)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(iters):
                fn(i)
        graph.replay()
        torch.cuda.synchronize()
        s.record()
        graph.replay()
        e.record()
    else:
        s.record()
        for i in range(iters):
            fn(i)
        e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters * 1e3  # microseconds


def bench_q4_linear(a) -> dict:
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    K, N, M = a.K, a.N, a.M
    wshape = (K // 8, N) if a.layout == 1 else (N, K // 8)
    sshape = (K // a.block, N) if a.layout == 1 else (N, K // a.block)
    wbytes = K * N // 2 + (K // a.block) * N * 4
    copies = max(1, int(np.ceil(a.rotate_bytes / wbytes))) if a.rotate_bytes else 1
    weights = []
    for _ in range(copies):
        words = torch.randint(-2 ** 31, 2 ** 31 - 1, wshape, dtype=torch.int32, device=dev, generator=g)
        scales = torch.rand(sshape, device=dev, generator=g) * 0.015 + 0.005
        weights.append(from_packed(words, scales, a.layout, a.block, (K, N) if a.layout == 1 else (N, K)))
    x = torch.randn((M, K), device=dev, generator=g).to(DT[a.xdtype])
    y = torch.empty((M, N), dtype=DT[a.ydtype], device=dev)
    if a.swiglu:  # silu(x W1) * (x W3): consecutive weight copies serve as W1 and W3
        if copies == 1:
            weights.append(from_packed(weights[0].words.clone(), weights[0].scales.clone(), a.layout,
                                       a.block, weights[0].shape))
        nw = len(weights)
        us = _time(lambda i: q_matmul_swiglu(x, weights[i % nw], weights[(i + 1) % nw], out=y),
                   a.iters, a.warmup)
        flops, wbytes = 4.0 * M * N * K, 2 * wbytes
    else:
        us = _time(lambda i: q_matmul(x, weights[i % copies], out=y), a.iters, a.warmup)
        flops = 2.0 * M * N * K
    ebytes = {"f32": 4, "f16": 2, "bf16": 2}
    bytes_ = wbytes + M * K * ebytes[a.xdtype] + M * N * ebytes[a.ydtype]
    return {"op": "q4_linear_swiglu" if a.swiglu else "q4_linear", "M": M, "K": K, "N": N,
            "layout": a.layout, "block": a.block,
            "xdtype": a.xdtype, "ydtype": a.ydtype, "weight_copies": copies, "us": round(us, 3),
            "tflops": round(flops / us / 1e6, 2), "frac_mfma_peak": round(flops / us / 1e6 / PEAK_TFLOPS, 4),
            "gbs": round(bytes_ / us / 1e3, 1), "frac_hbm_peak": round(bytes_ / us / 1e3 / PEAK_GBS, 4)}


def _segments(spec: str, S: int) -> np.ndarray:
    total, lo, hi = (int(v) for v in spec.split(":"))
    from .workloads import c5_segments
    return c5_segments(total if total else S, lo, hi)


def bench_attention(a) -> dict:
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    dt = DT[a.dtype]
    if a.token_major:  # [B, S, H, D] storage viewed as [B, H, S, D] (the block's GQA layout)
        q = torch.randn((a.B, a.S, a.H, a.D), device=dev, generator=g).to(dt).permute(0, 2, 1, 3)
        k = torch.randn((a.B, a.S, a.Hkv, a.D), device=dev, generator=g).to(dt).permute(0, 2, 1, 3)
        v = torch.randn((a.B, a.S, a.Hkv, a.D), device=dev, generator=g).to(dt).permute(0, 2, 1, 3)
        o = torch.empty((a.B, a.S, a.H, a.D), dtype=DT[a.odtype], device=dev).permute(0, 2, 1, 3)
    else:
        q = torch.randn((a.B, a.H, a.S, a.D), device=dev, generator=g).to(dt)
        k = torch.randn((a.B, a.Hkv, a.S, a.D), device=dev, generator=g).to(dt)
        v = torch.randn((a.B, a.Hkv, a.S, a.D), device=dev, generator=g).to(dt)
        o = torch.empty((a.B, a.H, a.S, a.D), dtype=DT[a.odtype], device=dev)
    cu = None
    pairs = a.S * a.S
    if a.segments:
        cu_np = _segments(a.segments, a.S)
        cu = torch.from_numpy(cu_np).to(dev)
        L = np.diff(cu_np.astype(np.int64))
        pairs = int(np.sum(L * (L + 1) // 2)) if a.causal else int(np.sum(L * L))
    elif a.causal:
        pairs = a.S * (a.S + 1) // 2
    us = _time(lambda i: attention(q, k, v, out=o, is_causal=a.causal, cu_seqlens=cu), a.iters, a.warmup)
    flops = 4.0 * a.B * a.H * a.D * pairs
    return {"op": "attention", "B": a.B, "H": a.H, "Hkv": a.Hkv, "S": a.S, "D": a.D,
            "dtype": a.dtype, "odtype": a.odtype, "causal": a.causal, "segments": a.segments,
            "us": round(us, 3), "tflops": round(flops / us / 1e6, 2),
            "frac_mfma_peak": round(flops / us / 1e6 / PEAK_TFLOPS, 4)}


def bench_qk_prep(a) -> dict:
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    dt = DT[a.dtype]
    q = torch.randn((1, a.S, a.Hq, a.D), device=dev, generator=g).to(dt)
    k = torch.randn((1, a.S, a.Hkv, a.D), device=dev, generator=g).to(dt)
    v = torch.randn((1, a.S, a.Hkv, a.D), device=dev, generator=g).to(dt)
    nq = RmsNorm(torch.ones(a.D, device=dev))
    nk = RmsNorm(torch.ones(a.D, device=dev))
    cs = torch.rand((1, a.S, a.D), device=dev, generator=g)
    sn = torch.rand((1, a.S, a.D), device=dev, generator=g)
    us = _time(lambda i: qk_norm_rope(q, k, v, nq, nk, cs, sn), a.iters, a.warmup)
    esz = {"f32": 4, "f16": 2, "bf16": 2}[a.dtype]
    rows = a.S * (a.Hq + 2 * a.Hkv)
    bytes_ = rows * a.D * (esz + 2) + 2 * a.S * a.D * 4
    return {"op": "qk_prep", "S": a.S, "Hq": a.Hq, "Hkv": a.Hkv, "D": a.D, "dtype": a.dtype,
            "us": round(us, 3), "gbs": round(bytes_ / us / 1e3, 1),
            "frac_hbm_peak": round(bytes_ / us / 1e3 / PEAK_GBS, 4)}


def bench_glue(a) -> dict:
    """The block's middle glue pass (block.rs:91-111): r = x + rmsnorm(branch) * tanh(gate) into a
    new residual, then rmsnorm(r) * (1 + scale) in bf16 for the next projection."""
    from .block import block_glue
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    S, Wd = a.S, a.W
    branch = torch.randn((1, S, Wd), device=dev, generator=g).to(DT[a.dtype])
    x = torch.randn((1, S, Wd), device=dev, generator=g)
    r = torch.empty_like(x)
    gate = torch.randn((1, Wd), device=dev, generator=g)
    scale = torch.randn((1, Wd), device=dev, generator=g)
    n1, n2 = RmsNorm(torch.ones(Wd, device=dev)), RmsNorm(torch.ones(Wd, device=dev))
    us = _time(lambda i: block_glue(branch, residual=x, branch_norm=n1, gate=gate, residual_out=r,
                                    next_norm=n2, next_scale=scale, next_dtype=torch.bfloat16),
               a.iters, a.warmup)
    esz = {"f32": 4, "f16": 2, "bf16": 2}[a.dtype]
    bytes_ = S * Wd * (esz + 4 + 4 + 2)  # branch and residual in, residual and bf16 rows out
    return {"op": "glue", "S": S, "W": Wd, "dtype": a.dtype, "us": round(us, 3),
            "gbs": round(bytes_ / us / 1e3, 1), "frac_hbm_peak": round(bytes_ / us / 1e3 / PEAK_GBS, 4)}


def bench_block(a) -> dict:
    """SingleStreamBlock.forward (block.rs:84-134) at S tokens x 3072, 24 x 128 heads, SwiGLU
    12288, bf16 activations, random packed weights: modulation GEMV, three glue passes, the QKV
    projection with the Q/K norm + RoPE epilogue, attention, O, fused SwiGLU, down (eager launches,
    as a caller runs it)."""
    from . import block as BL
    from . import linear as LN
    from . import rope as R
    from .workloads import boogu_joint_ids
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    Wd, H, D, C, F = 3072, 24, 128, 1024, 12288

    def q4(K, N):
        words = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), dtype=torch.int32, device=dev, generator=g)
        scales = torch.rand((K // 128, N), device=dev, generator=g) * 0.015 + 0.005
        return from_packed(words, scales, 1, 128, (K, N))
    ones = lambda n: torch.ones(n, device=dev)  # noqa: E731
    attn = BL.GqaAttention(None, None, None, LN.Linear(q4(Wd, Wd)), RmsNorm(ones(D)), RmsNorm(ones(D)),
                           H, H, D, qkv=LN.Linear(q4(Wd, 3 * Wd)))
    blk = BL.SingleStreamBlock(
        norm1=BL.RmsNormZero(LN.Linear(q4(C, 4 * Wd), torch.zeros(4 * Wd, device=dev)), RmsNorm(ones(Wd))),
        attn=attn, norm2=RmsNorm(ones(Wd)), ffn_norm1=RmsNorm(ones(Wd)), ffn_norm2=RmsNorm(ones(Wd)),
        feed_forward=BL.LuminaFeedForward(LN.Linear(q4(Wd, F)), LN.Linear(q4(F, Wd)), LN.Linear(q4(Wd, F))),
        activation_dtype=torch.bfloat16)
    ids = boogu_joint_ids(2)[: a.S]
    cos, sin = R.rope_values(ids, [32, 48, 48], 1.0e4)
    rope = (torch.from_numpy(cos[None]).to(dev), torch.from_numpy(sin[None]).to(dev))
    tokens = torch.randn((1, a.S, Wd), device=dev, generator=g)
    cond = torch.randn((1, C), device=dev, generator=g)
    us = _time(lambda i: blk.forward(tokens, rope, cond), a.iters, a.warmup)
    return {"op": "block", "S": a.S, "hidden": Wd, "heads": H, "head_dim": D, "ffn": F, "us": round(us, 3)}


def bench_qkv_prep(a) -> dict:
    """The fused self-attention input launch (biq_q4_linear_qk_norm_rope): tokens [1, S, 3072]
    bf16 times a packed q | k | v weight (block 128) with the Q/K RMSNorm + RoPE + f16 cast in the
    epilogue.  GB/s counts the algorithmic bytes: activations, words, scales, cos / sin tables
    read once, f16 Q / K / V written."""
    from . import block as BL
    from . import linear as LN
    from . import rope as R
    from .workloads import boogu_joint_ids
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    Wd, H, Hkv, D = 3072, a.Hq, a.Hkv, 128
    N = (H + 2 * Hkv) * D
    words = torch.randint(-2 ** 31, 2 ** 31 - 1, (Wd // 8, N), dtype=torch.int32, device=dev, generator=g)
    scales = torch.rand((Wd // 128, N), device=dev, generator=g) * 0.015 + 0.005
    w = LN.Linear(from_packed(words, scales, 1, 128, (Wd, N)))
    ids = boogu_joint_ids(2)[: a.S]
    cos, sin = R.rope_values(ids, [32, 48, 48], 1.0e4)
    rope = (torch.from_numpy(cos[None]).to(dev), torch.from_numpy(sin[None]).to(dev))
    x = torch.randn((1, a.S, Wd), device=dev, generator=g).to(torch.bfloat16)
    n = RmsNorm(torch.ones(D, device=dev))
    us = _time(lambda i: BL.project_qkv_norm_rope(w, x, n, n, rope, H, Hkv, D), a.iters, a.warmup)
    flops = 2.0 * a.S * Wd * N
    nbytes = a.S * Wd * 2 + Wd * N // 2 + (Wd // 128) * N * 4 + 2 * a.S * D * 4 + a.S * N * 2
    return {"op": "qkv_prep", "S": a.S, "K": Wd, "N": N, "us": round(us, 3),
            "tflops": round(flops / (us * 1e-6) / 1e12, 2),
            "frac_mfma_peak": round(flops / (us * 1e-6) / 1e12 / 2500.0, 4),
            "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}


def bench_copy(a) -> dict:
    dev = torch.device("cuda:0")
    n = (a.kib << 10) if a.kib else (a.mib << 20)
    src = torch.ones(n // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    us = _time(lambda i: dst.copy_(src), a.iters, a.warmup)
    return {"op": "copy", "bytes_read": n, "bytes_written": n, "us": round(us, 3),
            "gbs": round(2 * n / us / 1e3, 1)}


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m burn_image_amd.perf")
    sub = ap.add_subparsers(dest="op", required=True)
    p = sub.add_parser("q4_linear")
    p.add_argument("--M", type=int, default=4608)
    p.add_argument("--K", type=int, default=3072)
    p.add_argument("--N", type=int, default=9216)
    p.add_argument("--layout", type=int, default=1)
    p.add_argument("--block", type=int, default=128)
    p.add_argument("--xdtype", default="bf16", choices=list(DT))
    p.add_argument("--ydtype", default="f32", choices=list(DT))
    p.add_argument("--rotate-bytes", type=float, default=0.0)
    p.add_argument("--swiglu", action="store_true", help="fused silu(x W1) * (x W3) over two weights")
    p = sub.add_parser("attention")
    p.add_argument("--B", type=int, default=1)
    p.add_argument("--H", type=int, default=24)
    p.add_argument("--Hkv", type=int, default=24)
    p.add_argument("--S", type=int, default=4608)
    p.add_argument("--D", type=int, default=128)
    p.add_argument("--dtype", default="bf16", choices=list(DT))
    p.add_argument("--odtype", default="f32", choices=list(DT))
    p.add_argument("--causal", action="store_true")
    p.add_argument("--segments", default="", help="total:min:max segment draw (as the C5 workload)")
    p.add_argument("--token-major", action="store_true", help="Q/K/V/O stored [B, S, H, D]")
    p = sub.add_parser("qk_prep")
    p.add_argument("--S", type=int, default=4608)
    p.add_argument("--Hq", type=int, default=24)
    p.add_argument("--Hkv", type=int, default=24)
    p.add_argument("--D", type=int, default=128)
    p.add_argument("--dtype", default="f32", choices=list(DT))
    p = sub.add_parser("glue")
    p.add_argument("--S", type=int, default=4608)
    p.add_argument("--W", type=int, default=3072)
    p.add_argument("--dtype", default="bf16", choices=list(DT))
    p = sub.add_parser("block")
    p.add_argument("--S", type=int, default=4608)
    p = sub.add_parser("qkv_prep")
    p.add_argument("--S", type=int, default=4608)
    p.add_argument("--Hq", type=int, default=24)
    p.add_argument("--Hkv", type=int, default=24)
    p = sub.add_parser("copy")
    p.add_argument("--mib", type=int, default=512)
    p.add_argument("--kib", type=int, default=0, help="size in KiB instead (a launch-cost floor)")
    for p in sub.choices.values():
        p.add_argument("--iters", type=int, default=50)
        p.add_argument("--warmup", type=int, default=5)
        p.add_argument("--graph", action="store_true", help="replay the calls from a HIP graph")
    a = ap.parse_args(argv)
    global _GRAPH
    _GRAPH = a.graph
    _lib.load()
    fn = {"q4_linear": bench_q4_linear, "attention": bench_attention, "qk_prep": bench_qk_prep,
          "glue": bench_glue, "block": bench_block, "qkv_prep": bench_qkv_prep,
          "copy": bench_copy}[a.op]
    print(json.dumps(fn(a)), flush=True)


if __name__ == "__main__":
    sys.exit(main())
