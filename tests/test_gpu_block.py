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


@pytest.mark.parametrize("Wd", [520, 1600, 3072, 4096, 522, 4100])
def test_gpu_block_glue_residual_and_modulation(gpu, oracle, Wd):
    """Rows of <= 4096 elements in whole 4-vectors take the row-in-registers kernel, instantiated
    per vectors per thread (520: 1, the last vectors of a row held by some threads only; 1600: 2;
    3072, the block width: 3; 4096: 4); 522 (not whole vectors) and 4100 (wider than the
    registers hold) take the workgroup-per-row kernel."""
    rng = np.random.default_rng(40)
    Bn, S = 2, 33
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
    # the bf16 output is the f32 one rounded once to nearest even (the hardware conversion)
    nf32 = BL.block_glue(dev(x, device=gpu), next_norm=B.RmsNorm(dev(gn, device=gpu), 1e-5),
                         next_scale=dev(scale, device=gpu), next_dtype=torch.float32)
    assert np.array_equal(host(nb16).view(np.uint32), W.round_to_bf16(host(nf32)).view(np.uint32))
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


# ---------------------------------------------------------------------------------------------
# dual-stream attention and block (attention.rs:499-720, block.rs:138-350)
# ---------------------------------------------------------------------------------------------

class _Q4Set:
    """Random packed Q4 weights for named [K, N] projections, with the oracle's f64 product."""

    def __init__(self, gpu, oracle, seed, shapes, block=None):
        self.gpu, self.oracle, self.m = gpu, oracle, {}
        for i, (n, (K, N)) in enumerate(shapes.items()):
            blk = block or oracle.q4_kn_block(K, N)
            words, scales = W.q4_weight(seed, i, K, N, layout=1, block=blk)
            self.m[n] = (words, scales, blk, B.from_packed(dev_words(words, gpu), dev(scales, device=gpu), 1, blk, (K, N)))

    def lin(self, n):
        return B.Linear(self.m[n][3])

    def f64(self, x, n, rows=None):
        w, s, blk, _ = self.m[n]
        x2 = np.ascontiguousarray(x.reshape(-1, x.shape[-1]), np.float32)
        y = self.oracle.q4_linear_f64(x2, w, s, 1, blk, w.shape[1], rows=rows)
        return y if rows is not None else y.reshape(*x.shape[:-1], w.shape[1])


def _dual_attention(gpu, oracle, seed, width, H, Hkv, D, St, Si, Bn, block=None):
    rng = np.random.default_rng(seed)
    kvw = Hkv * D
    q4 = _Q4Set(gpu, oracle, seed, {"iq": (width, H * D), "ik": (width, kvw), "iv": (width, kvw),
                                     "tq": (width, H * D), "tk": (width, kvw), "tv": (width, kvw),
                                     "io": (H * D, width), "to": (H * D, width), "out": (width, width)}, block)
    gq = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    mod = BL.DoubleStreamAttention(q4.lin("iq"), q4.lin("ik"), q4.lin("iv"), q4.lin("tq"), q4.lin("tk"),
                                   q4.lin("tv"), q4.lin("io"), q4.lin("to"), q4.lin("out"),
                                   B.RmsNorm(dev(gq, device=gpu), 1e-5), B.RmsNorm(dev(gk, device=gpu), 1e-5),
                                   H, Hkv, D)
    img = rng.standard_normal((Bn, Si, width)).astype(np.float32)
    ins = rng.standard_normal((Bn, St, width)).astype(np.float32)
    S = St + Si
    ang = rng.uniform(0, 2 * np.pi, (S, D // 2)).astype(np.float64)
    cos = np.repeat(np.cos(ang), 2, axis=1).astype(np.float32)
    sin = np.repeat(np.sin(ang), 2, axis=1).astype(np.float32)
    return q4, mod, img, ins, (gq, gk), (cos, sin)


def _dual_attention_ref(oracle, q4, img, ins, g, rope, H, Hkv, D, rows):
    """f64 composition of DoubleStreamAttention::forward (attention.rs:637-693) for token rows
    `rows` of the joint [instruction, image] sequence; returns the to_out projection of those
    rows (row < St: instruction stream, else image stream)."""
    Bn, St, _ = ins.shape
    S = St + img.shape[1]
    cos, sin = rope
    cat = lambda a, b: np.concatenate([a, b], axis=1)  # noqa: E731
    k = cat(q4.f64(ins, "tk"), q4.f64(img, "ik")).reshape(Bn, S, Hkv, D)
    v = cat(q4.f64(ins, "tv"), q4.f64(img, "iv")).reshape(Bn, S, Hkv, D)
    q = cat(q4.f64(ins, "tq"), q4.f64(img, "iq")).reshape(Bn, S, H, D)
    cs = np.broadcast_to(cos[None, :, None, :], q.shape)
    sn = np.broadcast_to(sin[None, :, None, :], q.shape)
    qn = oracle.apply_rope_interleaved(oracle.rms_norm(q, g[0], 1e-5), cs, sn)
    kn = oracle.apply_rope_interleaved(oracle.rms_norm(k, g[1], 1e-5), cs[:, :, :Hkv], sn[:, :, :Hkv])
    att = oracle.attention_f64(qn.transpose(0, 2, 1, 3), kn.transpose(0, 2, 1, 3),
                               v.transpose(0, 2, 1, 3).astype(np.float32), rows=rows).transpose(0, 2, 1, 3)
    att = att.reshape(Bn, len(rows), H * D).astype(np.float32)
    out = np.zeros((Bn, len(rows), q4.m["out"][0].shape[1]), np.float64)
    for j, r in enumerate(rows):
        proj = q4.f64(att[:, j], "to" if r < St else "io")
        out[:, j] = q4.f64(proj.astype(np.float32), "out")
    return out.astype(np.float32)


@pytest.mark.parametrize("split", [True, False])
def test_gpu_double_stream_attention_matches_composition(gpu, oracle, split):
    """Eight Q4 projections, joint GQA attention over [instruction, image] with Q/K norm + RoPE,
    per-stream output projections and the shared to_out, split or joint (B = 2, GQA 2:1)."""
    H, Hkv, D, St, Si, Bn = 2, 1, 128, 24, 72, 2
    q4, mod, img, ins, g, rope = _dual_attention(gpu, oracle, 60, 256, H, Hkv, D, St, Si, Bn)
    kern = type("K", (B.NativeQ4FlashAttention,), {"SPLIT_DOUBLE_STREAM_SHARED_PROJECTION": split})
    mod.kernel = kern
    img_o, ins_o = mod.forward(dev(img, device=gpu), dev(ins, device=gpu),
                               (dev(rope[0][None], device=gpu), dev(rope[1][None], device=gpu)))
    assert img_o.shape == (Bn, Si, 256) and ins_o.shape == (Bn, St, 256)
    rows = np.arange(St + Si)
    ref = _dual_attention_ref(oracle, q4, img, ins, g, rope, H, Hkv, D, rows)
    assert_parity(host(ins_o), ref[:, :St], f"dual_attention_instruction_split{int(split)}")
    assert_parity(host(img_o), ref[:, St:], f"dual_attention_image_split{int(split)}")


def test_gpu_double_stream_attention_released_geometry(gpu, oracle):
    """Released widths: hidden 3360 (block-32 scales), 28 query / 7 KV heads of D = 120 (kv width
    840); 40 instruction + 216 image tokens; sampled rows of both streams against the oracle.
    Three chained 3360-wide projections of N(0, 1) tokens give outputs of RMS ~6, so the max-abs
    bound of the gate is applied relative to the output RMS (2e-3 * rms); mean-rel stays 1e-3."""
    H, Hkv, D, St, Si = 28, 7, 120, 40, 216
    q4, mod, img, ins, g, rope = _dual_attention(gpu, oracle, 61, 3360, H, Hkv, D, St, Si, 1)
    img_o, ins_o = mod.forward(dev(img, device=gpu), dev(ins, device=gpu),
                               (dev(rope[0][None], device=gpu), dev(rope[1][None], device=gpu)))
    rows = np.array([0, 17, 39, 40, 41, 130, 255])
    ref = _dual_attention_ref(oracle, q4, img, ins, g, rope, H, Hkv, D, rows)
    got = np.concatenate([host(ins_o), host(img_o)], axis=1)[:, rows]
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    assert rms > 1.0
    assert_parity(got, ref, "dual_attention_released", max_abs=2e-3 * rms)


def test_gpu_double_stream_block_matches_composition(gpu, oracle):
    """The dual-stream block (block.rs:248-350): five adaptive norms sharing two RMS reductions,
    joint attention, image self attention, per-stream SwiGLU FFNs on the (1 + scale) * base +
    shift input, tanh-gated residuals -- against the oracle's f64 composition."""
    rng = np.random.default_rng(62)
    H, Hkv, D, St, Si, Bn, Wd, C, inner = 2, 1, 128, 24, 72, 1, 256, 96, 384
    q4a, jattn, img, ins, g, rope = _dual_attention(gpu, oracle, 63, Wd, H, Hkv, D, St, Si, Bn)
    shapes = {"sq": (Wd, H * D), "sk": (Wd, Hkv * D), "sv": (Wd, Hkv * D), "so": (H * D, Wd)}
    for p in ("i", "t"):
        shapes.update({p + "w1": (Wd, inner), p + "w2": (inner, Wd), p + "w3": (Wd, inner)})
    for n in ("in1", "in2", "in3", "tn1", "tn2"):
        shapes["m" + n] = (C, 4 * Wd)
    q4 = _Q4Set(gpu, oracle, 64, shapes)
    gam = {n: (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
           for n, d in [(n, Wd) for n in ("in1", "in2", "in3", "tn1", "tn2", "ia", "is", "if1", "if2",
                                          "ta", "tf1", "tf2")] + [("sq", D), ("sk", D)]}
    bias = {n: (0.1 * rng.standard_normal(4 * Wd)).astype(np.float32) for n in ("in1", "in2", "in3", "tn1", "tn2")}
    rn = lambda n: B.RmsNorm(dev(gam[n], device=gpu), 1e-5)  # noqa: E731
    rz = lambda n: BL.RmsNormZero(B.Linear(q4.m["m" + n][3], dev(bias[n], device=gpu)), rn(n))  # noqa: E731
    ffn = lambda p: B.LuminaFeedForward(q4.lin(p + "w1"), q4.lin(p + "w2"), q4.lin(p + "w3"))  # noqa: E731
    blk = BL.DoubleStreamBlock(
        joint_attn=jattn,
        image_self_attn=BL.GqaAttention(q4.lin("sq"), q4.lin("sk"), q4.lin("sv"), q4.lin("so"), rn("sq"), rn("sk"),
                                        H, Hkv, D),
        image_ffn=ffn("i"), instruction_ffn=ffn("t"),
        image_norm1=rz("in1"), image_norm2=rz("in2"), image_norm3=rz("in3"),
        instruction_norm1=rz("tn1"), instruction_norm2=rz("tn2"),
        image_attn_norm=rn("ia"), image_self_norm=rn("is"), image_ffn_norm1=rn("if1"), image_ffn_norm2=rn("if2"),
        instruction_attn_norm=rn("ta"), instruction_ffn_norm1=rn("tf1"), instruction_ffn_norm2=rn("tf2"))
    cond = rng.standard_normal((Bn, C)).astype(np.float32)
    ang = rng.uniform(0, 2 * np.pi, (Si, D // 2))
    icos = np.repeat(np.cos(ang), 2, axis=1).astype(np.float32)
    isin = np.repeat(np.sin(ang), 2, axis=1).astype(np.float32)
    dv = lambda a: dev(a, device=gpu)  # noqa: E731
    img_o, ins_o = blk.forward(dv(img), dv(ins), (dv(icos[None]), dv(isin[None])),
                               (dv(rope[0][None]), dv(rope[1][None])), dv(cond))

    # ---- oracle composition (f64 where the reference computes in f32)
    silu = lambda a: a / (1.0 + np.exp(-a))  # noqa: E731
    sc = silu(_f64(cond)).astype(np.float32)
    mods = {n: oracle.q4_linear_f64(sc, q4.m["m" + n][0], q4.m["m" + n][1], 1, q4.m["m" + n][2], 4 * Wd,
                                    bias=bias[n]).astype(np.float32) for n in bias}
    ch = lambda n, i: mods[n][:, i * Wd:(i + 1) * Wd]  # noqa: E731

    def rms(x, gamma=None):
        return _f64(oracle.rms_norm(np.ascontiguousarray(x, np.float32), np.ones(x.shape[-1], np.float32)
                                    if gamma is None else gamma, 1e-5))

    def adaptive(x, n):
        return (rms(x, gam[n]) * (1.0 + _f64(ch(n, 0)))[:, None, :]).astype(np.float32)

    def gated(x, branch, gname, gate):
        return _f64(x) + rms(branch, gam[gname]) * np.tanh(_f64(gate))[:, None, :]

    def ffn_ref(x, p):
        h = silu(_f64(q4.f64(x, p + "w1"))) * _f64(q4.f64(x, p + "w3"))
        return q4.f64(h.astype(np.float32), p + "w2").astype(np.float32)

    img_joint, img_base, img_self = adaptive(img, "in1"), adaptive(img, "in2"), adaptive(img, "in3")
    ins_joint, ins_base = adaptive(ins, "tn1"), adaptive(ins, "tn2")
    joint = _dual_attention_ref(oracle, q4a, img_joint, ins_joint, g, rope, H, Hkv, D, np.arange(St + Si))
    ins_attn, img_attn = joint[:, :St], joint[:, St:]
    # image self attention (GqaAttention on the third adaptive norm's tokens)
    q = q4.f64(img_self, "sq").reshape(Bn, Si, H, D)
    k = q4.f64(img_self, "sk").reshape(Bn, Si, Hkv, D)
    v = q4.f64(img_self, "sv").reshape(Bn, Si, Hkv, D)
    cs = np.broadcast_to(icos[None, :, None, :], q.shape)
    sn = np.broadcast_to(isin[None, :, None, :], q.shape)
    qn = oracle.apply_rope_interleaved(oracle.rms_norm(q, gam["sq"], 1e-5), cs, sn)
    kn = oracle.apply_rope_interleaved(oracle.rms_norm(k, gam["sk"], 1e-5), cs[:, :, :Hkv], sn[:, :, :Hkv])
    att = oracle.attention_f64(qn.transpose(0, 2, 1, 3), kn.transpose(0, 2, 1, 3),
                               v.transpose(0, 2, 1, 3).astype(np.float32)).transpose(0, 2, 1, 3)
    img_self_out = q4.f64(att.reshape(Bn, Si, H * D).astype(np.float32), "so")
    x = gated(img, img_attn, "ia", ch("in1", 1))
    x = gated(x, img_self_out, "is", ch("in3", 1))
    mlp_in = _f64(img_base) * (1.0 + _f64(ch("in1", 2)))[:, None, :] + _f64(ch("in2", 1))[:, None, :]
    img_ref = gated(x, ffn_ref(rms(mlp_in, gam["if1"]).astype(np.float32), "i"), "if2", ch("in1", 3))
    y = gated(ins, ins_attn, "ta", ch("tn1", 1))
    mlp_in = _f64(ins_base) * (1.0 + _f64(ch("tn1", 2)))[:, None, :] + _f64(ch("tn2", 1))[:, None, :]
    ins_ref = gated(y, ffn_ref(rms(mlp_in, gam["tf1"]).astype(np.float32), "t"), "tf2", ch("tn1", 3))
    assert_parity(host(img_o), img_ref.astype(np.float32), "dual_block_image")
    assert_parity(host(ins_o), ins_ref.astype(np.float32), "dual_block_instruction")
