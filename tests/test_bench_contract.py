"""bench.py's host-side contract (CPU only): more than one GPU is refused with a JSON message
before any GPU work, and the CPU baseline leg reports the fields the result line documents,
with `value` equal to the step's FLOP over the step time it reports."""
import json
import os
import subprocess
import sys
import types

from conftest import ROOT


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_cpu_baseline_leg_fields(oracle):
    import bench
    from burn_image_amd import workloads as W

    words_np, scales_np, x_np = {}, {}, {}
    for i, (name, K, N) in enumerate(bench.GEMMS):
        words_np[name], scales_np[name] = W.q4_weight(3, 2 * i + 1, K, N, layout=1)
        x_np[name] = W.activations(3, 2 * i, bench.M_TOKENS, K, "bf16")
    q_np, k_np, v_np = W.boogu_attention(2)
    rows = 32
    r = bench.cpu_baseline(types.SimpleNamespace(cpu_rows=rows, cpu_runs=2), words_np, scales_np, x_np,
                           q_np, k_np, v_np)
    assert r["kind"] == "port" and r["unit"] == "TFLOP/s"
    assert r["cores"] >= 1 and r["value"] > 0
    assert f"first {rows} of 4608 rows" in r["sample"] and "median of 2 runs" in r["sample"]
    assert "cpu_model" in r and r["nproc"] >= 1
    assert set(r["per_op_tflops"]) == {"qkv", "o", "mlp_up", "mlp_down", "attention"}
    step_flops = (sum(bench.gemm_flops(bench.M_TOKENS, K, N) for _, K, N in bench.GEMMS)
                  + bench.attn_flops(**bench.ATTN))
    assert abs(step_flops / (r["ms_per_step"] / 1e3) / 1e12 - r["value"]) <= 1e-9 * r["value"]
