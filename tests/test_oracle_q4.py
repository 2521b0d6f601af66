"""Pins of the Q4S oracle (CPU): reference known answers, round-trip gates, importer contracts,
C oracle == numpy restatement, and the mathematics of the format."""
import os

import numpy as np
import pytest

from conftest import GOLDEN


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_kat_probe_quantizes_exactly_and_product_is_exact_reference(oracle):
    """Browser probe (crates/bevy_image/src/browser_boogu/runtime.rs:4511-4545): the weights
    ((k + 3n) % 15 - 7) / 64 quantise exactly (alpha = 7/64, scale = 1/64), so the Q4 GEMM equals
    the float product of the original weights; the reference gates max_abs <= 5e-4 (:4771-4777)."""
    g = load("kat_probe.npz")
    words, scales, blk = oracle.q4_quantize_kn(g["weight"])
    assert blk == 128
    assert np.all(scales == np.float32(1.0 / 64.0))
    assert np.array_equal(words, g["words"]) and np.array_equal(scales, g["scales"])
    assert np.array_equal(oracle.q4_dequant(words, scales, 1, 128, 128, 128), g["weight"])
    y = oracle.q4_linear_f64(g["lhs"], words, scales, 1, 128, 128)
    assert np.array_equal(y, g["expected"])
    # independent check of the known answer itself: a plain f32 triple loop (the probe's reference)
    f32 = g["lhs"].astype(np.float32) @ g["weight"].astype(np.float32)
    assert np.max(np.abs(f32 - g["expected"])) <= 5e-4


def test_roundtrip_gates_reference(oracle):
    """artifacts.rs:10413-10498: max weight error < 0.025, relative RMSE < 0.08, cosine > 0.996,
    and the byte count values/2 + values/128 * 4."""
    g = load("roundtrip.npz")
    values = g["values"]
    words, scales = oracle.q4_quantize_nk(values)
    assert np.array_equal(words, g["words"]) and np.array_equal(scales, g["scales"])
    assert words.nbytes + scales.nbytes == values.size // 2 + values.size // 128 * 4
    recon = oracle.q4_dequant(words, scales, 0, 128, 128, 128)
    assert np.max(np.abs(recon - values)) < 0.025
    ref = g["input"].astype(np.float64) @ values.astype(np.float64)
    act = g["input"].astype(np.float64) @ recon.astype(np.float64)
    rel_rmse = np.sqrt(np.sum((act - ref) ** 2) / np.sum(ref ** 2))
    cos = np.dot(act, ref) / (np.linalg.norm(act) * np.linalg.norm(ref))
    assert rel_rmse < 0.08 and cos > 0.996
    assert np.allclose(ref, g["reference"]) and np.allclose(act, g["actual"])


def test_storage_block_policy_and_importer_contract_reference(oracle):
    """q4s_storage_block_and_axis (artifacts.rs:513-525) and the importer contract
    (crates/burn_boogu/src/bin/boogu_import.rs:1693-1719)."""
    assert oracle.q4_kn_block(64, 3360) == 64          # q4s-block64x1-f32-packed-axis1
    assert oracle.q4_kn_block(3360, 3360) == 32        # released hidden width
    assert oracle.q4_kn_block(13568, 3360) == 128
    assert oracle.q4_kn_block(3072, 9216) == 128
    assert oracle.q4_kn_block(24, 16) == 8
    assert oracle.q4_kn_block(12, 16) == 0             # no exact block
    assert oracle.q4_kn_block(128, 12) == 0            # output not divisible by 8
    # Qwen [256, 128] stores 256*128/2 + 256*4 bytes
    words, scales = oracle.q4_quantize_nk(np.ones((256, 128), np.float32))
    assert words.nbytes + scales.nbytes == 256 * 128 // 2 + 256 * 4


def test_quantizers_reject_invalid_sources_correctness(oracle):
    """artifacts.rs:10880-10885 and the row-layout error paths."""
    with pytest.raises(oracle.OracleError):
        oracle.q4_quantize_nk(np.full((1, 128), np.nan, np.float32))
    with pytest.raises(oracle.OracleError):
        oracle.q4_quantize_nk(np.zeros((1, 127), np.float32))
    with pytest.raises(oracle.OracleError):
        oracle.q4_quantize_nk(np.zeros((0,), np.float32))
    with pytest.raises(oracle.OracleError):
        oracle.q4_quantize_kn(np.full((8, 8), np.inf, np.float32))
    with pytest.raises(oracle.OracleError):
        oracle.q4_quantize_kn(np.zeros((12, 8), np.float32))


@pytest.mark.parametrize("K,N", [(128, 64), (64, 40), (96, 24), (48, 16), (24, 8), (3360, 16)])
def test_row_layout_quantizer_matches_numpy_restatement_correctness(oracle, K, N):
    rng = np.random.default_rng(K * 1000 + N)
    w = rng.standard_normal((K, N)).astype(np.float32) * rng.uniform(0.01, 3.0, size=(1, N)).astype(np.float32)
    w[:, 0] = 0.0  # all-zero column: scale f32::MIN_POSITIVE, all nibbles 0
    words, scales, blk = oracle.q4_quantize_kn(w)
    nw, ns, nb = oracle.np_q4_quantize_kn(w)
    assert blk == nb and np.array_equal(words, nw) and np.array_equal(scales, ns)
    assert np.all(scales[:, 0] == np.float32(1.1754944e-38)) and np.all(words[:, 0] == 0)


def test_quantizer_rounding_is_half_away_from_zero_and_clamped_correctness(oracle):
    """Values landing exactly on .5 multiples of the scale round away from zero; the block
    maximum maps to +-7 and nothing reaches the -8 code."""
    col = np.array([7.0, 3.5, -3.5, 2.5, -2.5, 0.5, -0.5, 0.0], np.float32)  # scale = 1
    w = np.tile(col[:, None], (1, 8))
    words, scales, blk = oracle.q4_quantize_kn(w)
    assert blk == 8 and np.all(scales == 1.0)
    q = oracle.np_unpack_q4(words)[0, 0]
    assert list(q) == [7, 4, -4, 3, -3, 1, -1, 0]


def test_nibble_decoding_is_twos_complement_including_minus_eight_correctness(oracle):
    """Stored nibbles are `(q as u8) & 0xf` (artifacts.rs:7273,7370): 0x8 decodes to -8."""
    word = np.array([[0x76543210 ^ 0x0]], np.uint32)  # nibbles 0..7
    word2 = np.array([[0xFEDCBA98]], np.uint32)          # nibbles 8..15 -> -8..-1
    assert list(oracle.np_unpack_q4(word)[0, 0]) == [0, 1, 2, 3, 4, 5, 6, 7]
    assert list(oracle.np_unpack_q4(word2)[0, 0]) == [-8, -7, -6, -5, -4, -3, -2, -1]
    scales = np.ones((1, 1), np.float32) * np.float32(0.5)
    d = oracle.q4_dequant(word2, scales, 1, 8, 8, 1)
    assert list(d[:, 0]) == [-4.0, -3.5, -3.0, -2.5, -2.0, -1.5, -1.0, -0.5]


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("block", [8, 16, 32, 64, 128])
def test_dequant_c_matches_numpy_bit_exact_correctness(oracle, layout, block):
    from burn_image_amd import workloads as W
    K, N = 256, 48
    words, scales = W.q4_weight(9, block + layout, K, N, layout=layout, block=block)
    a = oracle.q4_dequant(words, scales, layout, block, K, N)
    b = oracle.np_q4_dequant(words, scales, layout, block, K, N)
    assert a.tobytes() == b.tobytes()


def test_q4_linear_f64_matches_independent_float64_product_correctness(oracle):
    """The f64 GEMM oracle against numpy's float64 matmul of the numpy-dequantised weight, with
    row sampling and bias."""
    from burn_image_amd import workloads as W
    M, K, N = 37, 384, 72
    x = W.activations(9, 1, M, K, "bf16")
    words, scales = W.q4_weight(9, 2, K, N, layout=1, block=32)
    bias = np.linspace(-1, 1, N).astype(np.float32)
    rows = np.array([0, 5, 36])
    y = oracle.q4_linear_f64(x, words, scales, 1, 32, N, rows=rows, bias=bias)
    ref = x[rows].astype(np.float64) @ oracle.np_q4_dequant(words, scales, 1, 32, K, N).astype(np.float64) + bias
    assert np.max(np.abs(y - ref)) < 1e-9
    wn, sn = W.q4_weight(9, 3, K, N, layout=0, block=128)
    y0 = oracle.q4_linear_f64(x, wn, sn, 0, 128, N)
    ref0 = x.astype(np.float64) @ oracle.np_q4_dequant(wn, sn, 0, 128, K, N).astype(np.float64).T
    assert np.max(np.abs(y0 - ref0)) < 1e-9


def test_c1_linear_golden_reference(oracle):
    g = load("c1_linear.npz")
    yk = oracle.q4_linear_f64(g["x"], g["words_kn"], g["scales_kn"], 1, 128, 512)
    yn = oracle.q4_linear_f64(g["x"], g["words_nk"], g["scales_nk"], 0, 128, 512)
    assert np.array_equal(yk.astype(np.float32), g["y_kn"])
    assert np.array_equal(yn.astype(np.float32), g["y_nk"])


def test_cpu_baseline_linear_agrees_with_oracle_correctness(oracle):
    """The restated Burn CPU path (dequantise, f32 matmul) stays within f32 summation error."""
    g = load("c1_linear.npz")
    y, threads = oracle.cpu_q4_linear_f32(g["x"], g["words_kn"], g["scales_kn"], 1, 128, 512)
    assert threads >= 1
    assert np.max(np.abs(y - g["y_kn"])) < 1e-3
