"""GPU parity of the fused self-attention input launch (biq_q4_linear_qk_norm_rope through the C
ABI): the packed-Q4 q | k | v projection with strict-F32 RMSNorm + interleaved RoPE of the q and
k heads and the cast, in the projection's epilogue.  Checked against the two-call path
(biq_q4_linear, then biq_qk_norm_rope) and against the float64 oracle's composition; the
GqaAttention that routes through it against the oracle's attention composite."""
import numpy as np
import pytest
import torch

from gpu_util import assert_parity, dev, dev_words, host

pytestmark = pytest.mark.gpu

import burn_image_amd as B  # noqa: E402
from burn_image_amd import block as BL  # noqa: E402
from burn_image_amd import workloads as W  # noqa: E402

TORCH_DT = {"bf16": torch.bfloat16, "f16": torch.float16}
ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}  # one unit of the output, relative

# (x dtype, output dtype, block, batch, tokens, q heads, kv heads, K, per-batch RoPE tables,
#  head-major outputs)
CASES = [
    # 600 rows: two whole 256-row tiles and a ragged third; GQA 4:2
    ("bf16", torch.float16, 128, 2, 300, 4, 2, 512, False, False),
    # 3 + 2 heads: one tile holds a q and a k head, the last tile half lies past N; K % 64 == 32
    ("f16", torch.bfloat16, 32, 1, 257, 3, 1, 352, False, True),
    # 33 tokens: rows change batch inside an MFMA tile; cos / sin per (batch, token)
    ("bf16", torch.float16, 64, 3, 33, 2, 2, 192, True, False),
    # the same with head-major outputs (the batch index enters the output offset)
    ("bf16", torch.float16, 64, 3, 33, 2, 2, 192, True, True),
    # GQA 4:2 head-major over two batches
    ("f16", torch.float16, 128, 2, 300, 4, 2, 512, False, True),
]


def _case_inputs(i, xdt, block, Bn, S, Hq, Hkv, K, per_batch):
    D = 128
    N = (Hq + 2 * Hkv) * D
    x = W.activations(70 + i, 1, Bn * S, K, xdt)
    words, scales = W.q4_weight(70 + i, 2, K, N, layout=1, block=block)
    rng = np.random.default_rng(70 + i)
    gq = (1.0 + 0.25 * rng.standard_normal(D)).astype(np.float32)
    gk = (1.0 + 0.25 * rng.standard_normal(D)).astype(np.float32)
    rb = Bn if per_batch else 1
    # independent values per element (not per pair), so a swapped pair index shows
    cos = rng.uniform(-1.0, 1.0, (rb, S, D)).astype(np.float32)
    sin = rng.uniform(-1.0, 1.0, (rb, S, D)).astype(np.float32)
    return x, words, scales, gq, gk, cos, sin


def _within_one_unit(got, exp, dt, label, atol=2e-5):
    tol = np.abs(exp) * ULP[dt] + atol
    err = np.abs(got - exp) - tol
    assert np.all(err <= 0), f"{label}: exceeds one output unit by {np.max(err):.3e}"


@pytest.mark.parametrize("case", range(len(CASES)))
def test_gpu_fused_qkv_norm_rope_matches_two_calls_and_oracle(gpu, oracle, case):
    xdt, odt, block, Bn, S, Hq, Hkv, K, per_batch, head_major = CASES[case]
    D = 128
    x, words, scales, gq, gk, cos, sin = _case_inputs(case, xdt, block, Bn, S, Hq, Hkv, K, per_batch)
    N = (Hq + 2 * Hkv) * D
    w = B.from_packed(dev_words(words, gpu), dev(scales, device=gpu), 1, block, (K, N))
    xd = dev(x, TORCH_DT[xdt], gpu).reshape(Bn, S, K)
    nq, nk = B.RmsNorm(dev(gq, device=gpu), 1e-5), B.RmsNorm(dev(gk, device=gpu), 1e-6)
    rope = (dev(cos, device=gpu), dev(sin, device=gpu))
    q1, k1, v1 = B.project_qkv_norm_rope(B.Linear(w), xd, nq, nk, rope, Hq, Hkv, D, out_dtype=odt,
                                         head_major=head_major)
    if head_major:
        assert tuple(q1.shape) == (Bn, Hq, S, D) and tuple(v1.shape) == (Bn, Hkv, S, D) and q1.is_contiguous()
        q1, k1, v1 = (t.permute(0, 2, 1, 3) for t in (q1, k1, v1))
    assert q1.dtype == odt and tuple(q1.shape) == (Bn, S, Hq, D) and tuple(v1.shape) == (Bn, S, Hkv, D)

    # two calls: f32 projection, then the preparation kernel on its q / k / v views
    y = B.q_matmul(xd.reshape(Bn * S, K), w).view(Bn, S, Hq + 2 * Hkv, D)
    q2, k2, v2 = B.qk_norm_rope(y[:, :, :Hq], y[:, :, Hq:Hq + Hkv], y[:, :, Hq + Hkv:], nq, nk,
                                rope[0], rope[1], out_dtype=odt)
    for name, a, b in (("q", q1, q2), ("k", k1, k2), ("v", v1, v2)):
        _within_one_unit(host(a), host(b), odt, f"{name} vs two calls")

    # float64 oracle: projection, then norm -> RoPE, then the output type's rounding
    proj = oracle.q4_linear_f64(x, words, scales, 1, block, N).reshape(Bn, S, Hq + 2 * Hkv, D)
    cs = np.broadcast_to(cos[:, :, None, :], (Bn, S, 1, D))
    sn = np.broadcast_to(sin[:, :, None, :], (Bn, S, 1, D))
    qe = oracle.apply_rope_interleaved(oracle.rms_norm(proj[:, :, :Hq], gq, 1e-5),
                                       np.broadcast_to(cs, (Bn, S, Hq, D)), np.broadcast_to(sn, (Bn, S, Hq, D)))
    ke = oracle.apply_rope_interleaved(oracle.rms_norm(proj[:, :, Hq:Hq + Hkv], gk, 1e-6),
                                       np.broadcast_to(cs, (Bn, S, Hkv, D)), np.broadcast_to(sn, (Bn, S, Hkv, D)))
    ve = proj[:, :, Hq + Hkv:]
    for name, a, e in (("q", q1, qe), ("k", k1, ke), ("v", v1, ve)):
        _within_one_unit(host(a), np.asarray(e, np.float64), odt, f"{name} vs oracle")


def test_gpu_fused_qkv_norm_rope_unsupported_and_invalid(gpu):
    """Head widths other than 128, f32 tokens and blocks below 32 are refused (the caller makes
    the two calls); bad arguments fail closed."""
    K, D = 256, 120
    words, scales = W.q4_weight(75, 1, K, 4 * D, layout=1, block=128)
    w = B.from_packed(dev_words(words, gpu), dev(scales, device=gpu), 1, 128, (K, 4 * D))
    x = dev(W.activations(75, 1, 8, K, "bf16"), torch.bfloat16, gpu).reshape(1, 8, K)
    n = B.RmsNorm(dev(np.ones(D, np.float32), device=gpu))
    rope = (torch.ones((1, 8, D), device=gpu), torch.zeros((1, 8, D), device=gpu))
    with pytest.raises(B.Unsupported):
        B.project_qkv_norm_rope(B.Linear(w), x, n, n, rope, 2, 1, D)
    K, D = 256, 128
    words, scales = W.q4_weight(75, 2, K, 3 * D, layout=1, block=128)
    w = B.from_packed(dev_words(words, gpu), dev(scales, device=gpu), 1, 128, (K, 3 * D))
    n = B.RmsNorm(dev(np.ones(D, np.float32), device=gpu))
    rope = (torch.ones((1, 8, D), device=gpu), torch.zeros((1, 8, D), device=gpu))
    xf = dev(W.activations(75, 2, 8, K, "f32"), torch.float32, gpu).reshape(1, 8, K)
    with pytest.raises(B.Unsupported):
        B.project_qkv_norm_rope(B.Linear(w), xf, n, n, rope, 1, 1, D)
    words16, scales16 = W.q4_weight(75, 3, K, 3 * D, layout=1, block=16)
    w16 = B.from_packed(dev_words(words16, gpu), dev(scales16, device=gpu), 1, 16, (K, 3 * D))
    xb = xf.to(torch.bfloat16)
    with pytest.raises(B.Unsupported):
        B.project_qkv_norm_rope(B.Linear(w16), xb, n, n, rope, 1, 1, D)
    with pytest.raises(B.InvalidArgument):  # RoPE tables for another token count
        B.project_qkv_norm_rope(B.Linear(w), xb, n, n, (rope[0][:, :4], rope[1][:, :4]), 1, 1, D)
    with pytest.raises(B.InvalidArgument):  # eps must be positive
        B.project_qkv_norm_rope(B.Linear(w), xb, B.RmsNorm(n.gamma, 0.0), n, rope, 1, 1, D)


def test_gpu_gqa_attention_fused_route_matches_composition(gpu, oracle):
    """GqaAttention with the packed q | k | v weight and bf16 tokens takes the fused launch;
    the whole self attention (projection, norm + RoPE, GQA attention, output projection) against
    the oracle's f64 composition, at the hot path's gate."""
    from burn_image_amd import rope as R
    rng = np.random.default_rng(77)
    Bn, S, Wd, H, Hkv, D = 2, 160, 256, 4, 2, 128
    x = W.round_to_bf16(rng.standard_normal((Bn, S, Wd)).astype(np.float32))
    ids = R.position_ids(32, [], (40, 40), 2)[:S]
    cos, sin = R.rope_values(ids, [32, 48, 48], 1.0e4)
    gq = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    Nqkv = (H + 2 * Hkv) * D
    wqkv, sqkv = W.q4_weight(77, 1, Wd, Nqkv, layout=1)
    wo, so = W.q4_weight(77, 2, H * D, Wd, layout=1)
    qkv = B.Linear(B.from_packed(dev_words(wqkv, gpu), dev(sqkv, device=gpu), 1, 128, (Wd, Nqkv)))
    to_out = B.Linear(B.from_packed(dev_words(wo, gpu), dev(so, device=gpu), 1, 128, (H * D, Wd)))
    attn = BL.GqaAttention(None, None, None, to_out, B.RmsNorm(dev(gq, device=gpu), 1e-5),
                           B.RmsNorm(dev(gk, device=gpu), 1e-5), H, Hkv, D, qkv=qkv)
    xd = dev(x, torch.bfloat16, gpu)
    assert BL._fused_qkv_applies(qkv, xd, D)
    out = attn.forward(xd, xd, (dev(cos[None], device=gpu), dev(sin[None], device=gpu)))
    proj = oracle.q4_linear_f64(x.reshape(-1, Wd), wqkv, sqkv, 1, 128, Nqkv).reshape(Bn, S, H + 2 * Hkv, D)
    q, k, v = proj[:, :, :H], proj[:, :, H:H + Hkv], proj[:, :, H + Hkv:]
    qn = oracle.apply_rope_interleaved(oracle.rms_norm(q, gq, 1e-5), np.broadcast_to(cos[None, :, None, :], q.shape),
                                       np.broadcast_to(sin[None, :, None, :], q.shape))
    kn = oracle.apply_rope_interleaved(oracle.rms_norm(k, gk, 1e-5), np.broadcast_to(cos[None, :, None, :], k.shape),
                                       np.broadcast_to(sin[None, :, None, :], k.shape))
    att = oracle.attention_f64(qn.transpose(0, 2, 1, 3), kn.transpose(0, 2, 1, 3),
                               v.transpose(0, 2, 1, 3).astype(np.float32)).transpose(0, 2, 1, 3)
    ref = oracle.q4_linear_f64(att.reshape(-1, H * D).astype(np.float32), wo, so, 1, 128, Wd).reshape(Bn, S, Wd)
    assert_parity(host(out), ref.astype(np.float32), "gqa_fused_route")
