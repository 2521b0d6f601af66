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


def _prep_inputs(S=160, Hq=4, Hkv=2, D=120, seed=31):
    from burn_image_amd import rope as R
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((1, S, Hq, D)) * 2.0).astype(np.float32)
    k = (rng.standard_normal((1, S, Hkv, D)) * 0.5).astype(np.float32)
    v = rng.standard_normal((1, S, Hkv, D)).astype(np.float32)
    gq = (1.0 + 0.25 * rng.standard_normal(D)).astype(np.float32)
    gk = (1.0 + 0.25 * rng.standard_normal(D)).astype(np.float32)
    ids = R.position_ids(32, [], (40, 40), 2)[:S]
    cos, sin = R.rope_values(ids, [40, 40, 40] if D == 120 else [32, 48, 48], 1.0e4)
    return q, k, v, gq, gk, cos, sin


def test_gpu_qk_norm_rope_prep_matches_oracle(gpu, oracle):
    """Fused strict-F32 RMSNorm + interleaved RoPE + f16 cast (native_flash.rs:395-583) against
    the oracle's composition rms_norm -> apply_rope -> f16; differences stay within one f16
    rounding of the value."""
    q, k, v, gq, gk, cos, sin = _prep_inputs()
    norm_q = B.RmsNorm(dev(gq, device=gpu), 1e-5)
    norm_k = B.RmsNorm(dev(gk, device=gpu), 1e-5)
    qo, ko, vo = B.qk_norm_rope(dev(q, device=gpu), dev(k, device=gpu), dev(v, device=gpu),
                                          norm_q, norm_k, dev(cos[None], device=gpu),
                                          dev(sin[None], device=gpu))
    assert qo.dtype == torch.float16 and tuple(qo.shape) == q.shape
    for name, x, g, out in (("q", q, gq, qo), ("k", k, gk, ko)):
        exp = oracle.apply_rope_interleaved(oracle.rms_norm(x, g, 1e-5), np.broadcast_to(cos[None, :, None, :], x.shape),
                                            np.broadcast_to(sin[None, :, None, :], x.shape))
        got = host(out)
        tol = np.abs(exp) * 2.0 ** -10 + 1e-6
        assert np.all(np.abs(got - exp) <= tol), f"{name}: {np.max(np.abs(got - exp) - tol)}"
    assert np.array_equal(host(vo), W.round_to_f16(v))


def test_gpu_execute_gqa_with_qk_norm_rope_matches_composition(gpu, oracle):
    """The seam's third method (attention.rs:107-134; packed-Q4 route :447-496): F32 raw
    projections in, F32 attention out, against the float64 oracle of norm -> RoPE -> GQA attention."""
    q, k, v, gq, gk, cos, sin = _prep_inputs(S=300, Hq=28, Hkv=7, D=120, seed=32)
    out = B.NativeQ4FlashAttention.execute_gqa_with_qk_norm_rope(
        dev(q, device=gpu), dev(k, device=gpu), dev(v, device=gpu),
        B.RmsNorm(dev(gq, device=gpu), 1e-5), B.RmsNorm(dev(gk, device=gpu), 1e-5),
        (dev(cos[None], device=gpu), dev(sin[None], device=gpu)), 8192)
    assert out.dtype == torch.float32 and tuple(out.shape) == q.shape
    cs = np.broadcast_to(cos[None, :, None, :], q.shape)
    sn = np.broadcast_to(sin[None, :, None, :], q.shape)
    qn = oracle.apply_rope_interleaved(oracle.rms_norm(q, gq, 1e-5), cs, sn)
    kn = oracle.apply_rope_interleaved(oracle.rms_norm(k, gk, 1e-5), cs[:, :, :7], sn[:, :, :7])
    ref = oracle.attention_f64(qn.transpose(0, 2, 1, 3), kn.transpose(0, 2, 1, 3),
                               v.transpose(0, 2, 1, 3)).transpose(0, 2, 1, 3).astype(np.float32)
    assert_parity(host(out), ref, "execute_gqa_with_qk_norm_rope")
    with pytest.raises(B.Unsupported):
        B.NativeQ4FlashAttention.execute_gqa_with_qk_norm_rope(
            dev(q, device=gpu), dev(k, device=gpu), dev(v, device=gpu),
            B.RmsNorm(dev(gq, device=gpu)), B.RmsNorm(dev(gk, device=gpu)),
            (dev(cos[None], device=gpu), dev(sin[None], device=gpu)), 8192,
            rms_norm_policy=B.F16_STORAGE_F32_ACCUM)


@pytest.mark.parametrize("odt", [torch.float32, torch.bfloat16])
def test_gpu_many_items_ragged_keys(gpu, oracle, odt):
    """600 query blocks (more than one resident round of workgroups), ragged keys (S = 1800, not
    a multiple of the 64-key tile, so the last tile's prefetch runs past the sequence), D = 120,
    GQA 40:10; sampled rows of every head against the f64 oracle and every element against an
    fp32 reference; bit-identical on a repeat call."""
    rng = np.random.default_rng(44)
    Bn, H, Hkv, S, D = 1, 40, 10, 1800, 120
    q = W.round_to_bf16(rng.standard_normal((Bn, H, S, D)).astype(np.float32))
    k = W.round_to_bf16(rng.standard_normal((Bn, Hkv, S, D)).astype(np.float32))
    v = W.round_to_bf16(rng.standard_normal((Bn, Hkv, S, D)).astype(np.float32))
    qd, kd, vd = (dev(a, torch.bfloat16, gpu) for a in (q, k, v))
    out = B.attention(qd, kd, vd, out_dtype=odt)
    assert torch.equal(out, B.attention(qd, kd, vd, out_dtype=odt))
    rows = sample_rows(S, n=20, seed=44)
    ref = oracle.attention_f64(q, k, v, rows=rows).astype(np.float32)
    got = host(out[:, :, torch.from_numpy(rows).to(gpu)])
    if odt == torch.float32:
        assert_parity(got, ref, "many_items_sampled")
        kx = kd.repeat_interleave(H // Hkv, dim=1).contiguous()
        vx = vd.repeat_interleave(H // Hkv, dim=1).contiguous()
        full = torch_fp32_attention(qd, kx, vx, 1.0 / np.sqrt(D))
        assert_parity(host(out), host(full), "many_items_full_vs_fp32")
    else:
        assert np.max(np.abs(got - ref)) <= np.max(np.abs(ref)) * 2.0 ** -7 + 2e-3


# ---------------------------------------------------------------------------------------------
# key masks (Qwen attention_mask, Burn key-padding masks) and wider mask coverage
# ---------------------------------------------------------------------------------------------

def test_gpu_c5_padded_batch_key_mask(gpu, oracle):
    """C5 geometry (Hq 32, Hkv 8, D 128, S 1024) as a B = 2 padded batch: left padding in batch
    0, right padding in batch 1, causal GQA with the key-padding mask (text.rs:146-185).  Rows of
    batch 0 before its first valid token see no key: with the -1e30 fill mode they average V
    over every key, as the reference computes them."""
    q, k, v, valid = W.c5_padded_attention()
    qd, kd, vd = (dev(a, torch.bfloat16, gpu) for a in (q, k, v))
    vm = torch.from_numpy(valid).to(gpu)
    out = B.attention(qd, kd, vd, is_causal=True, key_mask=vm,
                      key_mask_mode=B._lib.KEY_MASK_VALID_FILL_MEAN, out_dtype=torch.float32)
    ref = oracle.attention_f64(q, k, v, causal=True, key_valid=valid, fill_mean=True).astype(np.float32)
    assert_parity(host(out), ref, "c5_padded_causal_fill_mean")
    # zero mode: identical except the empty rows, which are exactly zero
    out0 = B.attention(qd, kd, vd, is_causal=True, key_mask=vm.to(torch.uint8), out_dtype=torch.float32)
    ref0 = oracle.attention_f64(q, k, v, causal=True, key_valid=valid).astype(np.float32)
    assert_parity(host(out0), ref0, "c5_padded_causal_zero")
    assert torch.count_nonzero(out0[0, :, :137]).item() == 0
    assert torch.equal(out0[:, :, 137:][0], out[0, :, 137:]) and torch.equal(out0[1], out[1])
    # Burn polarity (True = masked) through the op mirror gives the zero-mode result bitwise
    outb = B.burn_attention(qd, kd, vd, (~vm)[:, None, None, :], is_causal=True)
    assert torch.equal(outb.float(), out0.to(torch.bfloat16).float())


@pytest.mark.parametrize("mode", ["keys", "keys_segment", "keys_causal_segment"])
def test_gpu_key_mask_combinations(gpu, oracle, mode):
    """Key masks on the unmasked 8-wave, per-segment 8-wave and causal 4-wave forms (f16, GQA
    4:2, D 128, B 2), with masked keys scattered (not only padding)."""
    rng = np.random.default_rng(31)
    S = 700
    q, k, v = (W.round_to_f16(rng.standard_normal((2, h, S, 128), dtype=np.float32)) for h in (4, 2, 2))
    valid = rng.random((2, S)) < 0.7
    cu = np.array([0, 90, 300, 301, 700], np.int32)
    causal = mode == "keys_causal_segment"
    seg = None if mode == "keys" else cu
    qd, kd, vd = (dev(a, torch.float16, gpu) for a in (q, k, v))
    out = B.attention(qd, kd, vd, is_causal=causal, cu_seqlens=seg, key_mask=torch.from_numpy(valid).to(gpu),
                      key_mask_mode=B._lib.KEY_MASK_VALID_FILL_MEAN, out_dtype=torch.float32)
    ref = oracle.attention_f64(q, k, v, causal=causal, cu_seqlens=seg, key_valid=valid,
                               fill_mean=True).astype(np.float32)
    assert_parity(host(out), ref, f"key_mask_{mode}")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("D", [64, 120])
@pytest.mark.parametrize("causal", [False, True])
def test_gpu_segment_masks_dtypes_widths_batches(gpu, oracle, dtype, D, causal):
    """Per-segment masks (8-wave form) and causal + segment (4-wave form) for f16 and f32 inputs,
    D in {64, 120} and B = 2 (the per-segment 8-wave form's register-set and V-group variants)."""
    rng = np.random.default_rng(40 + D + (1 if causal else 0))
    S = 640
    rnd = W.round_to_f16 if dtype == "f16" else (lambda a: a)
    q, k, v = (rnd(rng.standard_normal((2, h, S, D), dtype=np.float32)) for h in (4, 2, 2))
    cu = np.array([0, 64, 70, 333, 512, 640], np.int32)
    tdt = torch.float16 if dtype == "f16" else torch.float32
    qd, kd, vd = (dev(a, tdt, gpu) for a in (q, k, v))
    out = B.attention(qd, kd, vd, is_causal=causal, cu_seqlens=cu, out_dtype=torch.float32)
    ref = oracle.attention_f64(q, k, v, causal=causal, cu_seqlens=cu).astype(np.float32)
    assert_parity(host(out), ref, f"segment_{dtype}_D{D}_causal{int(causal)}")


# ---------------------------------------------------------------------------------------------
# fused Q/K preparation: 16-bit inputs (rms cast to the input dtype), bf16 outputs, rotate-half
# ---------------------------------------------------------------------------------------------

def _ulp(a, dt):
    """Spacing of the output dtype at |a| (f16: 11-bit significand, bf16: 8-bit)."""
    bits = 11 if dt == torch.float16 else 8
    e = np.floor(np.log2(np.maximum(np.abs(a), 2.0 ** -14)))
    return 2.0 ** (e - (bits - 1))


@pytest.mark.parametrize("in_dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("out_dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layout", ["interleaved", "half"])
def test_gpu_qk_prep_dtypes_and_layouts(gpu, oracle, in_dt, out_dt, layout):
    """Every input dtype (F32, F16, BF16) x output dtype (F16, BF16) x RoPE layout (Boogu pairs,
    Qwen rotate-half) against the oracle's restatement (the rms cast to the input dtype before the
    division, native_flash.rs:446-449), within one unit of the output dtype: the oracle rounds
    each step the same way; a division at a midpoint of F can land one unit apart."""
    rng = np.random.default_rng(80 + len(in_dt) + (7 if out_dt == torch.bfloat16 else 0))
    Bn, S, Hq, Hkv, D = 2, 33, 4, 2, 128
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[in_dt]
    q, k, v = (oracle.round_to(rng.standard_normal((Bn, S, h, D)).astype(np.float32) * 2.5, in_dt)
               for h in (Hq, Hkv, Hkv))
    gq = (1 + 0.25 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.25 * rng.standard_normal(D)).astype(np.float32)
    ang = rng.uniform(0, 6.3, (Bn, S, D // 2))
    rep = (lambda a: np.repeat(a, 2, axis=-1)) if layout == "interleaved" else (lambda a: np.concatenate([a, a], -1))
    cos, sin = rep(np.cos(ang)).astype(np.float32), rep(np.sin(ang)).astype(np.float32)
    lay = B._lib.ROPE_INTERLEAVED if layout == "interleaved" else B._lib.ROPE_HALF
    qo, ko, vo = B.qk_norm_rope(dev(q, tdt, gpu), dev(k, tdt, gpu), dev(v, tdt, gpu),
                                B.RmsNorm(dev(gq, device=gpu), 1e-5), B.RmsNorm(dev(gk, device=gpu), 1e-6),
                                dev(cos, device=gpu), dev(sin, device=gpu), out_dtype=out_dt, rope_layout=lay)
    assert qo.dtype == out_dt
    odt = "f16" if out_dt == torch.float16 else "bf16"
    for name, x, g, eps, out in (("q", q, gq, 1e-5, qo), ("k", k, gk, 1e-6, ko)):
        cs = np.broadcast_to(cos[:, :, None, :], x.shape)
        sn = np.broadcast_to(sin[:, :, None, :], x.shape)
        exp = oracle.round_to(oracle.qk_norm_rope_ref(x, g, eps, cs, sn, in_dt, layout), odt)
        got = host(out)
        bad = np.abs(got - exp) > _ulp(exp, out_dt) * 1.0001
        assert not bad.any(), f"{name}: {bad.sum()} elements beyond one unit, max {np.max(np.abs(got - exp))}"
        assert np.mean(got == exp) > 0.99
    assert np.array_equal(host(vo), oracle.round_to(v, odt))
