"""Pins of the RoPE / RMSNorm restatements (CPU)."""
import math

import numpy as np

from burn_image_amd import rope as R


def test_position_ids_text_reference_generated_order_reference():
    """crates/burn_boogu/src/rope.rs:100-121."""
    ids = R.position_ids(2, [(4, 6)], (4, 4), 2)
    assert list(ids[0]) == [0, 0, 0]
    assert list(ids[1]) == [1, 1, 1]
    assert list(ids[2]) == [2, 0, 0]
    assert list(ids[7]) == [2, 1, 2]
    assert list(ids[8]) == [5, 0, 0]
    assert ids.shape[0] == 2 + 6 + 4


def test_c4_geometry_ids_correctness():
    """512 text + 96x96 reference (axis0 = 512) + 96x96 target (axis0 = 512 + 96)."""
    ids = R.position_ids(512, [(192, 192)], (192, 192), 2)
    assert ids.shape == (18944, 3)
    assert list(ids[512]) == [512, 0, 0]
    assert list(ids[512 + 9216]) == [608, 0, 0]
    assert list(ids[-1]) == [608, 95, 95]


def test_rope_values_match_c_oracle_and_closed_form_correctness(oracle):
    """rope_values (crates/burn_boogu/src/model/denoiser.rs:992-1034) at the 1.5K geometry:
    the C oracle (libm f64 cos/sin, as Rust) and the package table agree, and pair 0 of every
    axis has inverse frequency 1 so its phase is the id itself."""
    ids = R.position_ids(147, [(32, 32)], (64, 64), 2)
    cs, sn = oracle.rope_values(ids, [40, 40, 40], 1.0e4)
    pc, ps = R.rope_values(ids, [40, 40, 40], 1.0e4)
    assert np.max(np.abs(cs - pc)) <= 1.2e-7 and np.max(np.abs(sn - ps)) <= 1.2e-7
    for s in (0, 5, 200, ids.shape[0] - 1):
        for axis in range(3):
            col = 40 * axis
            assert cs[s, col] == np.float32(math.cos(float(ids[s, axis])))
            assert sn[s, col + 1] == np.float32(math.sin(float(ids[s, axis])))
    assert np.allclose(cs ** 2 + sn ** 2, 1.0, atol=1e-6)
    # last pair of an axis: inverse frequency theta^(-38/40)
    inv = 1.0e4 ** (-38.0 / 40.0)
    s = 300
    assert cs[s, 38] == np.float32(math.cos(float(ids[s, 0]) * inv))


def test_interleaved_rope_rotates_pairs_correctness(oracle):
    """attention.rs:916-928: a pair (x0, x1) rotates by its phase; norms are preserved."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 8)).astype(np.float32)
    phase = rng.uniform(-3, 3, (6, 4))
    cs = np.repeat(np.cos(phase), 2, axis=1).astype(np.float32)
    sn = np.repeat(np.sin(phase), 2, axis=1).astype(np.float32)
    y = oracle.apply_rope_interleaved(x, cs, sn)
    z = (x[:, 0::2] + 1j * x[:, 1::2]) * np.exp(1j * phase)
    assert np.max(np.abs(y[:, 0::2] - z.real)) < 1e-5 and np.max(np.abs(y[:, 1::2] - z.imag)) < 1e-5


def test_rotate_half_rope_correctness(oracle):
    """crates/burn_qwen3_vl/src/text.rs:407-440: halves (a, b) rotate as a complex pair."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 8)).astype(np.float32)
    cs, sn = R.text_rope_values(np.arange(5), 8, 5.0e6)
    y = oracle.apply_rope_half(x, cs, sn)
    phase = np.arange(5)[:, None] * (5.0e6 ** (-np.arange(0, 8, 2) / 8.0))[None, :]
    z = (x[:, :4] + 1j * x[:, 4:]) * np.exp(1j * phase)
    assert np.max(np.abs(y[:, :4] - z.real)) < 1e-5 and np.max(np.abs(y[:, 4:] - z.imag)) < 1e-5


def test_strict_rms_norm_reference(oracle):
    """native_flash.rs:2962-3010: inputs ((29 i + 11) % 101 - 50) / 23, gamma 0.75 + (i % 17)/31,
    against an f32 scalar loop, max_abs <= 2e-6; plus scale invariance of x / rms(x)."""
    D = 120
    n = 2 * 3 * 4 * D
    x = ((((np.arange(n) * 29 + 11) % 101).astype(np.float32) - 50.0) / np.float32(23.0)).reshape(-1, D)
    gamma = (0.75 + (np.arange(D) % 17).astype(np.float32) / np.float32(31.0)).astype(np.float32)
    y = oracle.rms_norm(x, gamma, 1e-5)
    rms = np.sqrt(np.sum(x * x, axis=1, dtype=np.float32) / np.float32(D) + np.float32(1e-5)).astype(np.float32)
    ref = x / rms[:, None] * gamma
    assert np.max(np.abs(y - ref)) <= 2e-6
    y2 = oracle.rms_norm(x * np.float32(4.0), gamma, 0.0)
    y1 = oracle.rms_norm(x, gamma, 0.0)
    assert np.max(np.abs(y2 - y1)) <= 2e-6


def test_qk_prep_oracle_f32_reduces_to_pinned_norm_and_rope(oracle):
    """For F32 inputs the fused preparation is the pinned strict RMSNorm followed by the pinned
    RoPE restatements (interleaved pairs and rotate-half)."""
    rng = np.random.default_rng(70)
    x = rng.standard_normal((9, 64)).astype(np.float32) * 3
    g = (1 + 0.1 * rng.standard_normal(64)).astype(np.float32)
    cs = np.cos(rng.uniform(0, 6, (9, 64))).astype(np.float32)
    sn = np.sin(rng.uniform(0, 6, (9, 64))).astype(np.float32)
    n = oracle.rms_norm(x, g, 1e-5)
    for layout, rope in (("interleaved", oracle.apply_rope_interleaved), ("half", oracle.apply_rope_half)):
        y = oracle.qk_norm_rope_ref(x, g, 1e-5, cs, sn, "f32", layout)
        assert np.max(np.abs(y - rope(n, cs, sn))) <= 4e-6 * np.max(np.abs(y))


def test_qk_prep_oracle_16bit_rms_cast_to_input_dtype(oracle):
    """native_flash.rs:446-449 casts the strict-F32 rms to the input dtype F before dividing: with
    gamma = 1, cos = 1, sin = 0 the output is round_F(x / round_F(rms)), checked against exact
    rational division; dividing by the unrounded f32 rms instead (a plausible mistake) differs."""
    from fractions import Fraction
    rng = np.random.default_rng(71)
    for dt, npdt in (("f16", np.float16), ("bf16", None)):
        x = oracle.round_to(rng.standard_normal((6, 32)).astype(np.float32) * 5, dt)
        ones, zeros = np.ones((6, 32), np.float32), np.zeros((6, 32), np.float32)
        y = oracle.qk_norm_rope_ref(x, np.ones(32, np.float32), 1e-6, ones, zeros, dt, "interleaved")
        wrong = 0
        for r in range(6):
            rms32 = np.float32(np.sqrt(np.float32(np.sum(x[r].astype(np.float64) ** 2)) / np.float32(32) + np.float32(1e-6)))
            rms_f = oracle.round_to(np.array([rms32]), dt)[0]
            for d in range(32):
                exact = Fraction(float(x[r, d])) / Fraction(float(rms_f))
                want = oracle.round_to(np.array([float(exact)], np.float32), dt)[0]
                assert y[r, d] == want, (dt, r, d)
                wrong += oracle.round_to(np.array([np.float32(x[r, d]) / rms32]), dt)[0] != want
        assert wrong > 0, dt  # the f32-rms variant is distinguishable on these rows
