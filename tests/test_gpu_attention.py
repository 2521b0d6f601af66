"""GPU parity of the flash-attention kernel (through the C ABI) against the float64 oracle.
Gate: max-abs <= 2e-3 and mean|a-b|/mean|b| <= 1e-3 against the reference's f32 result."""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import assert_parity, dev, host

pytestmark = pytest.mark.gpu

import burn_image_amd as B  # noqa: E402
from burn_image_amd import workloads as W  # noqa: E402


def torch_fp32_attention(q, k, v, scale, chunk=1024):
    """fp32 reference on the GPU (plain matmul + softmax in query chunks; inputs contiguous)."""
    q, k, v = q.float().contiguous(), k.float().contiguous(), v.float().contiguous()
    rep = q.shape[1] // k.shape[1]
    if rep > 1:
        k = k.repeat_interleave(rep, dim=1).contiguous()
        v = v.repeat_interleave(rep, dim=1).contiguous()
    kt = k.transpose(2, 3).contiguous()
    outs = []
    for s in range(0, q.shape[2], chunk):
        sc = torch.matmul(q[:, :, s:s + chunk].contiguous(), kt) * scale
        outs.append(torch.matmul(torch.softmax(sc, dim=-1), v))
    return torch.cat(outs, dim=2)


def sample_rows(S, n=32, seed=0):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, S - 1], rng.integers(0, S, n)]))


def test_gpu_c1_attention_golden(gpu):
    g = np.load(os.path.join(GOLDEN, "c1_attention.npz"), allow_pickle=False)
    out = B.attention(dev(g["q"], device=gpu), dev(g["k"], device=gpu), dev(g["v"], device=gpu),
                      scale=1.0 / 8.0)
    assert out.dtype == torch.float32
    assert_parity(host(out), g["out"], "c1_attention")


@pytest.mark.parametrize("config", [2, 4])
def test_gpu_boogu_joint_attention_full_shape(gpu, oracle, config):
    """C2 (S = 4608) and C4 (S = 18944): sampled query rows of every head against the float64
    oracle, every element against a chunked fp32 reference."""
    q, k, v = W.boogu_attention(config)
    S = q.shape[2]
    qd, kd, vd = (dev(a, torch.bfloat16, gpu) for a in (q, k, v))
    out = B.attention(qd, kd, vd, out_dtype=torch.float32)
    rows = sample_rows(S, n=24 if config == 4 else 48, seed=config)
    ref = oracle.attention_f64(q, k, v, rows=rows).astype(np.float32)
    assert_parity(host(out[:, :, torch.from_numpy(rows).to(gpu)]), ref, f"c{config}_sampled")
    full = torch_fp32_attention(qd, kd, vd, 1.0 / np.sqrt(128.0))
    assert_parity(host(out), host(full), f"c{config}_full_vs_fp32")


def test_gpu_c5_causal_segment_gqa(gpu, oracle):
    q, k, v, cu = W.c5_attention()
    qd, kd, vd = (dev(a, torch.bfloat16, gpu) for a in (q, k, v))
    cud = torch.from_numpy(cu).to(gpu)
    out = B.attention(qd, kd, vd, is_causal=True, cu_seqlens=cud, out_dtype=torch.float32)
    ref = oracle.attention_f64(q, k, v, causal=True, cu_seqlens=cu).astype(np.float32)
    assert_parity(host(out), ref, "c5_causal_segment_gqa")
    # segment-only (vision per-frame) and causal-only (text) variants
    out_s = B.attention(qd, kd, vd, cu_seqlens=cud, out_dtype=torch.float32)
    ref_s = oracle.attention_f64(q, k, v, cu_seqlens=cu).astype(np.float32)
    assert_parity(host(out_s), ref_s, "c5_segment_gqa")
    out_c = B.attention(qd, kd, vd, is_causal=True, out_dtype=torch.float32)
    ref_c = oracle.attention_f64(q, k, v, causal=True).astype(np.float32)
    assert_parity(host(out_c), ref_c, "c5_causal_gqa")


def test_gpu_real_head_width_gqa_token_major(gpu, oracle):
    """Released geometry: 28 query / 7 KV heads, D = 120 (no padded copy), token-major
    [B, S, H, D] tensors through execute_gqa; f32 inputs (the F32 -> F16 bridge)."""
    rng = np.random.default_rng(21)
    S = 333
    q = rng.standard_normal((1, S, 28, 120)).astype(np.float32)
    k = rng.standard_normal((1, S, 7, 120)).astype(np.float32)
    v = rng.standard_normal((1, S, 7, 120)).astype(np.float32)
    out = B.NativeQ4FlashAttention.execute_gqa(dev(q, device=gpu), dev(k, device=gpu),
                                               dev(v, device=gpu), 8192)
    assert tuple(out.shape) == (1, S, 28, 120)
    ref = oracle.attention_f64(q.transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3),
                               v.transpose(0, 2, 1, 3)).transpose(0, 2, 1, 3).astype(np.float32)
    assert_parity(host(out), ref, "real_d120_gqa_token_major")


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_gpu_dtypes_tails_and_batches(gpu, oracle, dt):
    rng = np.random.default_rng(22)
    Bt, H, Sq, D = 2, 3, 200, 64
    q = rng.standard_normal((Bt, H, Sq, D)).astype(np.float32)
    k = rng.standard_normal((Bt, H, 77, D)).astype(np.float32)
    v = rng.standard_normal((Bt, H, 77, D)).astype(np.float32)
    if dt == torch.bfloat16:
        q, k, v = (W.round_to_bf16(a) for a in (q, k, v))
    elif dt == torch.float16:
        q, k, v = (W.round_to_f16(a) for a in (q, k, v))
    out = B.attention(dev(q, dt, gpu), dev(k, dt, gpu), dev(v, dt, gpu), out_dtype=torch.float32)
    ref = oracle.attention_f64(q, k, v).astype(np.float32)
    assert_parity(host(out), ref, f"tails_{dt}")


def test_gpu_closed_forms(gpu):
    rng = np.random.default_rng(23)
    q = dev(rng.standard_normal((1, 2, 130, 128)).astype(np.float32), torch.float16, gpu)
    v1 = rng.standard_normal((1, 2, 1, 128)).astype(np.float32)
    k1 = dev(rng.standard_normal((1, 2, 1, 128)).astype(np.float32), torch.float16, gpu)
    out = B.attention(q, k1, dev(v1, torch.float16, gpu), out_dtype=torch.float32)
    assert np.max(np.abs(host(out) - W.round_to_f16(v1))) == 0.0  # S_kv = 1: O = V exactly
    ones = torch.ones((1, 2, 300, 128), dtype=torch.float16, device=gpu)
    kr = dev(rng.standard_normal((1, 2, 300, 128)).astype(np.float32), torch.float16, gpu)
    out = B.attention(q, kr, ones, out_dtype=torch.float32)
    assert np.max(np.abs(host(out) - 1.0)) <= 1e-3  # V = 1: O = 1


def test_gpu_output_dtypes_and_strided_output(gpu, oracle):
    q, k, v = W.boogu_attention(2, heads=2, seq_limit=700)
    qd, kd, vd = (dev(a, torch.bfloat16, gpu) for a in (q, k, v))
    ref = oracle.attention_f64(q, k, v).astype(np.float32)
    for odt, tol in ((torch.float16, 2.0 ** -10), (torch.bfloat16, 2.0 ** -7)):
        o = host(B.attention(qd, kd, vd, out_dtype=odt))
        assert np.max(np.abs(o - ref)) <= tol * np.max(np.abs(ref)) + 1e-4
    # write into a token-major view of a larger buffer
    buf = torch.zeros((1, 700, 2, 128), dtype=torch.float32, device=gpu)
    B.attention(qd, kd, vd, out=buf.permute(0, 2, 1, 3))
    assert_parity(host(buf.permute(0, 2, 1, 3)), ref, "strided_out")


def test_gpu_invalid_arguments_fail_closed(gpu):
    x = torch.zeros((1, 4, 8, 64), dtype=torch.bfloat16, device=gpu)
    k3 = torch.zeros((1, 3, 8, 64), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(B.InvalidArgument, match="divisible"):
        B.attention(x, k3, k3)
    with pytest.raises(B.InvalidArgument):
        B.AttentionKernel.execute(x, x, x, 0)
