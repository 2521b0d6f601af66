"""GPU parity of the Qwen3-VL text attention composite (crates/burn_qwen3_vl/src/text.rs:103-192)
on libbiq against the oracle's composition: Q4 [N, K] projections, q/k RMSNorm + rotate-half
RoPE, causal GQA with the key-padding mask, o_proj."""
import numpy as np
import pytest
import torch

from gpu_util import assert_parity, dev, dev_words, host

pytestmark = pytest.mark.gpu

import burn_image_amd as B  # noqa: E402
from burn_image_amd import rope as R  # noqa: E402
from burn_image_amd import workloads as W  # noqa: E402


def test_gpu_qwen_text_attention_c5_padded_batch(gpu, oracle):
    """C5 geometry: 1024 tokens as a batch of two 512-token prompts (batch 0 left-padded by 61,
    batch 1 right-padded by 97), hidden 4096, 32 query / 8 KV heads of 128, Qwen-layout Q4
    projections (block 128).  Sampled rows (including the left-padding rows, which see no valid
    key and take the mean of V) against the f64 oracle composition."""
    Bn, S, Wd, H, Hkv, D = 2, 512, 4096, 32, 8, 128
    rng = np.random.default_rng(90)
    hid = rng.standard_normal((Bn, S, Wd)).astype(np.float32)
    valid = np.ones((Bn, S), bool)
    valid[0, :61] = False
    valid[1, S - 97:] = False
    pos = np.stack([np.maximum(np.arange(S) - 61, 0), np.arange(S)])
    tabs = [R.text_rope_values(pos[b], D, 5.0e6) for b in range(Bn)]
    cos = np.stack([t[0] for t in tabs]).astype(np.float32)
    sin = np.stack([t[1] for t in tabs]).astype(np.float32)
    mats = {}
    for i, (n, N) in enumerate((("q", H * D), ("k", Hkv * D), ("v", Hkv * D), ("o", Wd))):
        words, scales = W.q4_weight(5, 40 + i, Wd if n != "o" else H * D, N, layout=0)
        K = Wd if n != "o" else H * D
        mats[n] = (words, scales, B.from_packed(dev_words(words, gpu), dev(scales, device=gpu), 0, 128, (N, K)))
    gq = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    attn = B.Qwen3VlTextAttention(B.Linear(mats["q"][2]), B.Linear(mats["k"][2]), B.Linear(mats["v"][2]),
                                  B.Linear(mats["o"][2]), B.RmsNorm(dev(gq, device=gpu), 1e-6),
                                  B.RmsNorm(dev(gk, device=gpu), 1e-6), H, Hkv, D)
    out = attn.forward(dev(hid, device=gpu), dev(cos, device=gpu), dev(sin, device=gpu),
                       torch.from_numpy(valid).to(gpu))
    assert out.shape == (Bn, S, Wd) and out.dtype == torch.float32

    # ---- oracle composition at sampled rows
    rows = np.array([0, 30, 60, 61, 62, 200, 414, 415, 450, 511])
    # float64 products of the bit-exact dequantised [N, K] weights (the full K / V projections
    # are too large for the oracle's row loop; its GEMM is pinned against this same product)
    deq = {n: oracle.q4_dequant(mats[n][0], mats[n][1], 0, 128, mats[n][0].shape[1] * 8,
                                mats[n][0].shape[0]).astype(np.float64) for n in mats}
    lin = lambda x, n: np.asarray(x, np.float64) @ deq[n].T  # noqa: E731
    flat = hid.reshape(Bn * S, Wd)
    k = lin(flat, "k").reshape(Bn, S, Hkv, D)
    v = lin(flat, "v").reshape(Bn, S, Hkv, D).astype(np.float32)
    q = np.zeros((Bn, S, H, D), np.float32)
    q[:, rows] = lin(hid[:, rows].reshape(-1, Wd), "q").reshape(Bn, len(rows), H, D)
    cs = lambda h: np.broadcast_to(cos[:, :, None, :], (Bn, S, h, D))  # noqa: E731
    sn = lambda h: np.broadcast_to(sin[:, :, None, :], (Bn, S, h, D))  # noqa: E731
    qn = oracle.apply_rope_half(oracle.rms_norm(q, gq, 1e-6), cs(H), sn(H))
    kn = oracle.apply_rope_half(oracle.rms_norm(k, gk, 1e-6), cs(Hkv), sn(Hkv))
    att = oracle.attention_f64(qn.transpose(0, 2, 1, 3), kn.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3),
                               causal=True, key_valid=valid, fill_mean=True, rows=rows)
    att = att.transpose(0, 2, 1, 3).reshape(Bn * len(rows), H * D).astype(np.float32)
    ref = lin(att, "o").reshape(Bn, len(rows), Wd).astype(np.float32)
    got = host(out)[:, rows]
    # o_proj sums 4096 attention features: outputs have RMS ~7, so the max-abs bound is taken
    # relative to the output RMS (the attention's f16 operands give ~3e-4 relative error)
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    assert_parity(got, ref, "qwen_text_attention_c5", max_abs=max(2e-3, 2e-3 * rms))
    # the left-padding rows (tokens 0, 30, 60 of batch 0) all take o_proj(mean of V): identical
    assert np.array_equal(got[0, 0], got[0, 1]) and np.array_equal(got[0, 0], got[0, 2])
