"""Write the committed golden fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

Every fixture is produced by the C oracle and cross-checked against the numpy restatement
before it is written; the tests then pin both oracles (and the GPU path) to these files.

  kat_probe.npz    reference known-answer probe (crates/bevy_image/src/browser_boogu/
                   runtime.rs:4511-4545,4737-4781): lhs ((17 i) % 29 - 14) / 128 [4, 128],
                   weights ((k + 3 n) % 15 - 7) / 64 [128, 128] (exactly quantisable: scale 1/64),
                   its Boogu-layout Q4S words/scales and the exact float64 product.
  roundtrip.npz    reference round-trip case (crates/burn_boogu/src/artifacts.rs:10413-10440):
                   values [128, 128], Qwen-layout words/scales, input vector and both products.
  c1_linear.npz    C1 Q4 linear M256 K512 N512: f32 activations, both layouts, and the float64
                   result rounded to f32 (the reference's f32 result).
  c1_attention.npz C1 attention B1 H4 S256 D64 f32 and its float64 result rounded to f32.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from burn_image_amd import workloads as W  # noqa: E402
from oracle import oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def kat_probe():
    rows, inner, out = 4, 128, 128
    i = np.arange(rows * inner)
    lhs = (((i * 17) % 29).astype(np.float32) - 14.0) * np.float32(1.0 / 128.0)
    lhs = lhs.reshape(rows, inner)
    j = np.arange(inner * out)
    w = ((((j // out) + (j % out) * 3) % 15).astype(np.float32) - 7.0) * np.float32(1.0 / 64.0)
    w = w.reshape(inner, out)
    words, scales, blk = O.q4_quantize_kn(w)
    nw, ns, nb = O.np_q4_quantize_kn(w)
    assert blk == nb == 128 and np.array_equal(words, nw) and np.array_equal(scales, ns)
    expected = lhs.astype(np.float64) @ w.astype(np.float64)
    got = O.q4_linear_f64(lhs, words, scales, 1, blk, out)
    assert np.array_equal(got, expected)
    np.savez_compressed(os.path.join(HERE, "kat_probe.npz"), lhs=lhs, weight=w, words=words,
                        scales=scales, expected=expected)


def roundtrip():
    idx = np.arange(128 * 128)
    wave = (((idx * 37) % 509).astype(np.float32) - 254.0) / np.float32(1536.0)
    values = (wave + ((idx % 128).astype(np.float32) - np.float32(63.5)) / np.float32(8192.0)).astype(np.float32)
    values = values.reshape(128, 128)
    words, scales = O.q4_quantize_nk(values)
    nw, ns = O.np_q4_quantize_nk(values)
    assert np.array_equal(words, nw) and np.array_equal(scales, ns)
    inp = ((((np.arange(128) * 19) % 97).astype(np.float32) - 48.0) / np.float32(128.0))
    recon = O.q4_dequant(words, scales, 0, 128, 128, 128)  # [N=128 rows of 128] flattened chunks
    reference = inp.astype(np.float64) @ values.astype(np.float64)
    actual = inp.astype(np.float64) @ recon.astype(np.float64)
    np.savez_compressed(os.path.join(HERE, "roundtrip.npz"), values=values, words=words,
                        scales=scales, input=inp, reference=reference, actual=actual)


def c1_linear():
    M, K, N = 256, 512, 512
    x = W.activations(1, 3, M, K, "f32")
    wk, sk = W.q4_weight(1, 4, K, N, layout=1)
    wn, sn = W.q4_weight(1, 5, K, N, layout=0)
    yk = O.q4_linear_f64(x, wk, sk, 1, 128, N)
    yn = O.q4_linear_f64(x, wn, sn, 0, 128, N)
    # numpy cross-check
    dk = O.np_q4_dequant(wk, sk, 1, 128, K, N).astype(np.float64)
    dn = O.np_q4_dequant(wn, sn, 0, 128, K, N).astype(np.float64)
    assert np.allclose(x.astype(np.float64) @ dk, yk, rtol=0, atol=1e-9)
    assert np.allclose(x.astype(np.float64) @ dn.T, yn, rtol=0, atol=1e-9)
    np.savez_compressed(os.path.join(HERE, "c1_linear.npz"), x=x, words_kn=wk, scales_kn=sk,
                        words_nk=wn, scales_nk=sn, y_kn=yk.astype(np.float32),
                        y_nk=yn.astype(np.float32))


def c1_attention():
    q, k, v = W.c1_attention()
    out = O.attention_f64(q, k, v, scale=1.0 / 8.0)
    ref = O.np_attention(q, k, v, scale=1.0 / 8.0)
    assert np.max(np.abs(out - ref)) < 1e-12
    np.savez_compressed(os.path.join(HERE, "c1_attention.npz"), q=q, k=k, v=v,
                        out=out.astype(np.float32))


if __name__ == "__main__":
    O.build()
    kat_probe()
    roundtrip()
    c1_linear()
    c1_attention()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
