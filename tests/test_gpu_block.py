"""GPU parity of the block glue kernel and of the modulated DiT block composite
(crates/burn_boogu/src/model/block.rs:84-111) against the oracle's float composition."""
import numpy as np
import pytest
import torch

from gpu_util import assert_parity, dev, dev_words, host

pytestmark = pytest.mark.gpu

import burn_image_amd as B  # noqa: E402
from burn_image_amd import block as BL  # noqa: E402
from burn_image_amd import workloads as W  # noqa: E402


def _f64(a):
    return np.asarray(a, dtype=np.float64)


def glue_ref(oracle, x, branch, g_b, eps_b, gate, g_n, eps_n, scale, S):
    """r = x + rmsnorm(branch) * tanh(gate); next = rmsnorm(r) * (1 + scale) (block.rs:91-111)."""
    b_idx = np.arange(branch.shape[0] * S) // S
    rows = branch.reshape(-1, branch.shape[-1])
    if x is None:
        r = _f64(rows)
    else:
        nb = _f64(oracle.rms_norm(rows, g_b, eps_b))
        if gate is not None:
            nb = nb * np.tanh(_f64(gate))[b_idx]
        r = _f64(x.reshape(rows.shape)) + nb
    nxt = None
    if g_n is not None:
        nxt = _f64(oracle.rms_norm(r.astype(np.float32), g_n, eps_n))
        if scale is not None:
            nxt = nxt * (1.0 + _f64(scale))[b_idx]
    return r.astype(np.float32), (None if nxt is None else nxt.astype(np.float32))


def test_gpu_block_glue_residual_and_modulation(gpu, oracle):
    rng = np.random.default_rng(40)
    Bn, S, Wd = 2, 33, 520
    x = rng.standard_normal((Bn, S, Wd)).astype(np.float32)
    br = (rng.standard_normal((Bn, S, Wd)) * 3.0).astype(np.float32)
    gb = (1 + 0.2 * rng.standard_normal(Wd)).astype(np.float32)
    gn = (1 + 0.2 * rng.standard_normal(Wd)).astype(np.float32)
    gate = rng.standard_normal((Bn, Wd)).astype(np.float32)
    scale = (0.3 * rng.standard_normal((Bn, Wd))).astype(np.float32)
    r_ref, n_ref = glue_ref(oracle, x, br, gb, 1e-5, gate, gn, 1e-6, scale, S)
    xd = dev(x, device=gpu)
    nxt = BL.block_glue(dev(br, device=gpu), residual=xd, branch_norm=B.RmsNorm(dev(gb, device=gpu), 1e-5),
                        gate=dev(gate, device=gpu), residual_out=xd,
                        next_norm=B.RmsNorm(dev(gn, device=gpu), 1e-6), next_scale=dev(scale, device=gpu),
                        next_dtype=torch.float32)
    assert_parity(host(xd).reshape(r_ref.shape), r_ref, "glue_residual_in_place", max_abs=1e-5, mean_rel=1e-6)
    assert_parity(host(nxt).reshape(n_ref.shape), n_ref, "glue_next", max_abs=1e-5, mean_rel=1e-6)
    # first norm of the block: no residual, bf16 output for the projections
    _, n0 = glue_ref(oracle, None, x, None, 0, None, gn, 1e-5, scale, S)
    nb16 = BL.block_glue(dev(x, device=gpu), next_norm=B.RmsNorm(dev(gn, device=gpu), 1e-5),
                         next_scale=dev(scale, device=gpu), next_dtype=torch.bfloat16)
    assert nb16.dtype == torch.bfloat16
    assert np.max(np.abs(host(nb16).reshape(n0.shape) - n0)) <= np.max(np.abs(n0)) * 2.0 ** -8
    # unmodulated residual (plain block, block.rs:113-131): no gate, bf16 branch
    br16 = W.round_to_bf16(br)
    r1, _ = glue_ref(oracle, x, br16, gb, 1e-5, None, None, 0, None, S)
    out = torch.empty((Bn, S, Wd), device=gpu)
    BL.block_glue(dev(br16, torch.bfloat16, gpu), residual=dev(x, device=gpu),
                  branch_norm=B.RmsNorm(dev(gb, device=gpu), 1e-5), residual_out=out)
    assert_parity(host(out).reshape(r1.shape), r1, "glue_plain", max_abs=1e-5, mean_rel=1e-6)
    with pytest.raises(B.InvalidArgument):
        BL.block_glue(dev(br, device=gpu), residual=xd)  # nothing to write


def _q4(seed, idx, K, N, gpu):
    words, scales = W.q4_weight(seed, idx, K, N, layout=1)
    return words, scales, B.from_packed(dev_words(words, gpu), dev(scales, device=gpu), 1, 128, (K, N))


def test_gpu_single_stream_block_matches_composition(gpu, oracle):
    """The whole modulated block on libbiq kernels against the oracle's f64 composition of the
    same steps (modulation GEMV, norms, Q4 projections, Q/K norm + RoPE, exact GQA attention,
    SwiGLU FFN, tanh-gated residuals).  The attention operands are f16, as on the reference's
    F32 -> F16 bridge, so the gate is the hot path's: max-abs 2e-3, mean-rel 1e-3."""
    from burn_image_amd import rope as R
    rng = np.random.default_rng(41)
    Bn, S, Wd, H, D, C, inner = 2, 96, 256, 2, 128, 128, 384
    tokens = rng.standard_normal((Bn, S, Wd)).astype(np.float32)
    cond = rng.standard_normal((Bn, C)).astype(np.float32)
    ids = R.position_ids(32, [], (40, 40), 2)[:S]
    cos, sin = R.rope_values(ids, [32, 48, 48], 1.0e4)
    g = {n: (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
         for n, d in (("n1", Wd), ("n2", Wd), ("f1", Wd), ("f2", Wd), ("q", D), ("k", D))}
    mods = {}
    wm, sm, qm = _q4(42, 0, C, 4 * Wd, gpu)
    bias_m = (0.1 * rng.standard_normal(4 * Wd)).astype(np.float32)
    for i, (n, K, N) in enumerate((("q", Wd, H * D), ("k", Wd, H * D), ("v", Wd, H * D), ("o", H * D, Wd),
                                    ("w1", Wd, inner), ("w2", inner, Wd), ("w3", Wd, inner))):
        mods[n] = _q4(42, i + 1, K, N, gpu)
    lin = {n: B.Linear(m[2]) for n, m in mods.items()}
    rn = lambda n, eps=1e-5: B.RmsNorm(dev(g[n], device=gpu), eps)  # noqa: E731
    blk = BL.SingleStreamBlock(
        norm1=BL.RmsNormZero(B.Linear(qm, dev(bias_m, device=gpu)), rn("n1")),
        attn=BL.GqaAttention(lin["q"], lin["k"], lin["v"], lin["o"], rn("q"), rn("k"), H, H, D),
        norm2=rn("n2"), ffn_norm1=rn("f1"), ffn_norm2=rn("f2"),
        feed_forward=B.LuminaFeedForward(lin["w1"], lin["w2"], lin["w3"]))
    out = blk.forward(dev(tokens, device=gpu), (dev(cos[None], device=gpu), dev(sin[None], device=gpu)),
                      dev(cond, device=gpu))

    # ---- oracle composition
    def lin64(x, n):
        w, s, _ = mods[n]
        return oracle.q4_linear_f64(x.reshape(-1, x.shape[-1]).astype(np.float32), w, s, 1, 128,
                                    w.shape[1]).reshape(*x.shape[:-1], w.shape[1])
    silu = lambda a: a / (1.0 + np.exp(-a))  # noqa: E731
    mod = oracle.q4_linear_f64(silu(_f64(cond)).astype(np.float32), wm, sm, 1, 128, 4 * Wd, bias=bias_m)
    sc_msa, gt_msa, sc_mlp, gt_mlp = (mod[:, i * Wd:(i + 1) * Wd].astype(np.float32) for i in range(4))
    _, n1 = glue_ref(oracle, None, tokens, None, 0, None, g["n1"], 1e-5, sc_msa, S)
    n1 = n1.reshape(Bn, S, Wd)
    q = lin64(n1, "q").reshape(Bn, S, H, D)
    k = lin64(n1, "k").reshape(Bn, S, H, D)
    v = lin64(n1, "v").reshape(Bn, S, H, D)
    cs = np.broadcast_to(cos[None, :, None, :], q.shape)
    sn = np.broadcast_to(sin[None, :, None, :], q.shape)
    qn = oracle.apply_rope_interleaved(oracle.rms_norm(q, g["q"], 1e-5), cs, sn)
    kn = oracle.apply_rope_interleaved(oracle.rms_norm(k, g["k"], 1e-5), cs, sn)
    att = oracle.attention_f64(qn.transpose(0, 2, 1, 3), kn.transpose(0, 2, 1, 3),
                               v.transpose(0, 2, 1, 3).astype(np.float32)).transpose(0, 2, 1, 3)
    o = lin64(att.reshape(Bn, S, H * D).astype(np.float32), "o")
    t1, mlp_in = glue_ref(oracle, tokens, o.astype(np.float32), g["n2"], 1e-5, gt_msa, g["f1"], 1e-5, sc_mlp, S)
    h = silu(_f64(lin64(mlp_in.reshape(Bn, S, Wd), "w1"))) * _f64(lin64(mlp_in.reshape(Bn, S, Wd), "w3"))
    mlp = lin64(h.astype(np.float32), "w2")
    ref, _ = glue_ref(oracle, t1, mlp.astype(np.float32), g["f2"], 1e-5, gt_mlp, None, 0, None, S)
    assert_parity(host(out).reshape(ref.shape), ref, "single_stream_block")
