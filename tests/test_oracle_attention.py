"""Pins of the attention oracle (CPU): closed forms, dense == chunked, GQA == materialised
expansion, causal-prefix and segment invariants, the reference's chunk policy table, the
D = 120 padding identity, and agreement with an independent numpy softmax."""
import os

import numpy as np
import pytest

from conftest import GOLDEN


def det(shape, offset):
    """Reference test generator ((i + off) * 17 + 5) % 43 -> (x - 21) / 13
    (crates/burn_boogu/src/model/attention.rs:957-970)."""
    n = int(np.prod(shape))
    i = np.arange(n)
    return ((((i + offset) * 17 + 5) % 43).astype(np.float32) - 21.0) / np.float32(13.0)


def det2(shape, offset):
    """((i + off) * 19 + 7) % 53 -> (x - 26) / 17 (native_flash.rs:2697-2710)."""
    n = int(np.prod(shape))
    i = np.arange(n)
    return (((((i + offset) * 19 + 7) % 53).astype(np.float32) - 26.0) / np.float32(17.0)).reshape(shape)


def test_effective_query_chunk_policy_table_reference(oracle):
    """attention.rs:1014-1022."""
    table = [(45, 1024, 45), (129, 1024, 128), (1024, 1024, 256), (2304, 1024, 576),
             (4096, 1024, 1024), (4141, 1024, 1024), (9261, 1024, 1024)]
    for q, req, exp in table:
        assert oracle.effective_query_chunk(q, req) == exp
    from burn_image_amd.attention import effective_portable_query_chunk_size
    for q, req, exp in table:
        assert effective_portable_query_chunk_size(q, req) == exp


def test_closed_forms_correctness(oracle):
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 2, 5, 16)).astype(np.float32)
    v = rng.standard_normal((1, 2, 1, 16)).astype(np.float32)
    # S_kv = 1: softmax is 1, O = V
    out = oracle.attention_f64(q, rng.standard_normal((1, 2, 1, 16)).astype(np.float32), v)
    assert np.allclose(out, np.broadcast_to(v, out.shape), atol=1e-12)
    # constant keys: uniform weights, O = mean(V)
    k = np.ones((1, 2, 7, 16), np.float32)
    v7 = rng.standard_normal((1, 2, 7, 16)).astype(np.float32)
    out = oracle.attention_f64(q, k, v7)
    assert np.allclose(out, v7.astype(np.float64).mean(axis=2, keepdims=True), atol=1e-12)
    # constant values: O = 1
    out = oracle.attention_f64(q, rng.standard_normal((1, 2, 7, 16)).astype(np.float32), np.ones((1, 2, 7, 16), np.float32))
    assert np.allclose(out, 1.0, atol=1e-12)
    # two keys: closed-form logistic weights
    k2 = rng.standard_normal((1, 1, 2, 16)).astype(np.float32)
    v2 = rng.standard_normal((1, 1, 2, 16)).astype(np.float32)
    q1 = q[:, :1]
    s = (q1[0, 0].astype(np.float64) @ k2[0, 0].T.astype(np.float64)) / 4.0
    w1 = 1.0 / (1.0 + np.exp(s[:, 0] - s[:, 1]))
    exp = (1 - w1)[:, None] * v2[0, 0, 0] + w1[:, None] * v2[0, 0, 1]
    assert np.allclose(oracle.attention_f64(q1, k2, v2)[0, 0], exp, atol=1e-12)


def test_matches_numpy_dense_softmax_correctness(oracle):
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 4, 33, 24)).astype(np.float32)
    k = rng.standard_normal((2, 2, 33, 24)).astype(np.float32)
    v = rng.standard_normal((2, 2, 33, 24)).astype(np.float32)
    cu = np.array([0, 5, 20, 33], np.int32)
    for causal in (False, True):
        for seg in (None, cu):
            a = oracle.attention_f64(q, k, v, causal=causal, cu_seqlens=seg)
            b = oracle.np_attention(q, k, v, causal=causal, cu_seqlens=seg)
            assert np.max(np.abs(a - b)) < 1e-12


def test_chunked_matches_dense_correctness(oracle):
    """attention.rs:973-999 (chunk 2 over [2, 3, 5, 4] x [2, 3, 7, 4]) with max_abs <= 1e-6:
    the chunked f32 CPU path against the dense f64 oracle."""
    q = det((2, 3, 5, 4), 0).reshape(2, 3, 5, 4)
    k = det((2, 3, 7, 4), 3).reshape(2, 3, 7, 4)
    v = det((2, 3, 7, 6), 9).reshape(2, 3, 7, 6)
    dense = oracle.attention_f64(q, k, v)
    chunked, _ = oracle.cpu_attention_f32(q, k, v, requested_chunk=2)
    assert np.max(np.abs(dense - chunked)) <= 1e-6


def test_gqa_equals_materialised_expansion_correctness(oracle):
    """attention.rs:1025-1052: token-major [1, 5, 4, 4] queries over [1, 7, 2, 4] K/V."""
    q = det((1, 5, 4, 4), 1).reshape(1, 5, 4, 4).transpose(0, 2, 1, 3)
    k = det((1, 7, 2, 4), 4).reshape(1, 7, 2, 4).transpose(0, 2, 1, 3)
    v = det((1, 7, 2, 4), 8).reshape(1, 7, 2, 4).transpose(0, 2, 1, 3)
    gqa = oracle.attention_f64(q, k, v)
    expanded = oracle.attention_f64(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1))
    assert np.max(np.abs(gqa - expanded)) <= 1e-12


def test_padded_head_width_transform_preserves_attention_correctness(oracle):
    """native_flash.rs:2738-2782: zero-padding D = 120 to 128 and scaling Q by sqrt(128/120)
    leaves the output unchanged (the kernel computes D = 120 directly)."""
    q = det2((1, 2, 3, 120), 1)
    k = det2((1, 2, 5, 120), 5)
    v = det2((1, 2, 5, 120), 9)
    ref = oracle.attention_f64(q, k, v)
    pad = lambda x: np.concatenate([x, np.zeros(x.shape[:3] + (8,), np.float32)], axis=3)
    qs = (q.astype(np.float64) * np.sqrt(128.0 / 120.0)).astype(np.float32)
    out = oracle.attention_f64(pad(qs), pad(k), pad(v))[..., :120]
    assert np.max(np.abs(out - ref)) <= 2e-6


def test_causal_prefix_independent_of_future_tokens_correctness(oracle):
    """crates/burn_qwen3_vl/src/text.rs:475-515: changing the last token leaves earlier rows."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 2, 9, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 9, 8)).astype(np.float32)
    v = rng.standard_normal((1, 2, 9, 8)).astype(np.float32)
    a = oracle.attention_f64(q, k, v, causal=True)
    k[:, :, -1] += 5.0
    v[:, :, -1] -= 3.0
    b = oracle.attention_f64(q, k, v, causal=True)
    assert np.array_equal(a[:, :, :-1], b[:, :, :-1])
    assert not np.allclose(a[:, :, -1], b[:, :, -1])


def test_segments_do_not_cross_attend_correctness(oracle):
    """crates/burn_qwen3_vl/src/vision.rs:686-719: a packed frame's output ignores other frames,
    and equals attention over that frame alone."""
    rng = np.random.default_rng(6)
    cu = np.array([0, 4, 8], np.int32)
    q = rng.standard_normal((1, 2, 8, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 8, 8)).astype(np.float32)
    v = rng.standard_normal((1, 2, 8, 8)).astype(np.float32)
    a = oracle.attention_f64(q, k, v, cu_seqlens=cu)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 4:] = -0.8
    v2[:, :, 4:] = 1.7
    b = oracle.attention_f64(q, k2, v2, cu_seqlens=cu)
    assert np.array_equal(a[:, :, :4], b[:, :, :4])
    alone = oracle.attention_f64(q[:, :, :4], k[:, :, :4], v[:, :, :4])
    assert np.max(np.abs(a[:, :, :4] - alone)) < 1e-12


def test_c1_attention_golden_reference(oracle):
    g = np.load(os.path.join(GOLDEN, "c1_attention.npz"), allow_pickle=False)
    out = oracle.attention_f64(g["q"], g["k"], g["v"], scale=1.0 / 8.0)
    assert np.array_equal(out.astype(np.float32), g["out"])
    chunked, _ = oracle.cpu_attention_f32(g["q"], g["k"], g["v"], scale=1.0 / 8.0, requested_chunk=128)
    assert np.max(np.abs(chunked - g["out"])) < 1e-5


def test_sampled_rows_equal_full_evaluation_correctness(oracle):
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 3, 40, 16)).astype(np.float32)
    k = rng.standard_normal((1, 3, 40, 16)).astype(np.float32)
    v = rng.standard_normal((1, 3, 40, 16)).astype(np.float32)
    rows = np.array([0, 7, 39])
    full = oracle.attention_f64(q, k, v, causal=True)
    part = oracle.attention_f64(q, k, v, causal=True, rows=rows)
    assert np.array_equal(full[:, :, rows], part)


def test_c5_segment_generator_properties_correctness():
    from burn_image_amd import workloads as W
    cu = W.c5_segments(1024)
    L = np.diff(cu)
    assert cu[0] == 0 and cu[-1] == 1024
    assert np.all(L >= 64) and np.all(L <= 512)


def test_key_mask_equals_attention_over_kept_keys_correctness(oracle):
    """Qwen's key-padding mask (text.rs:163-170): masked keys contribute nothing, so the result
    equals attention over the kept keys alone (non-causal; GQA 4:2)."""
    rng = np.random.default_rng(11)
    q = rng.standard_normal((2, 4, 12, 16)).astype(np.float32)
    k = rng.standard_normal((2, 2, 20, 16)).astype(np.float32)
    v = rng.standard_normal((2, 2, 20, 16)).astype(np.float32)
    valid = rng.random((2, 20)) < 0.6
    valid[:, 3] = True
    out = oracle.attention_f64(q, k, v, key_valid=valid)
    for b in range(2):
        keep = np.nonzero(valid[b])[0]
        alone = oracle.attention_f64(q[b:b + 1], k[b:b + 1][:, :, keep], v[b:b + 1][:, :, keep])
        assert np.max(np.abs(out[b:b + 1] - alone)) < 1e-12
    dense = oracle.np_attention(q, k, v, key_valid=valid)
    assert np.max(np.abs(out - dense)) < 1e-12


def test_key_mask_left_padding_causal_rows_correctness(oracle):
    """Left padding (processor.rs:379-385) under the causal mask: row i >= pad equals causal
    attention over keys [pad, i]; rows i < pad see no key and average V over every key with the
    reference's -1e30 fill (text.rs:177-182), or are zero without it."""
    rng = np.random.default_rng(12)
    S, pad = 10, 3
    q = rng.standard_normal((1, 2, S, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, S, 8)).astype(np.float32)
    v = rng.standard_normal((1, 2, S, 8)).astype(np.float32)
    valid = np.ones((1, S), bool)
    valid[0, :pad] = False
    filled = oracle.attention_f64(q, k, v, causal=True, key_valid=valid, fill_mean=True)
    zeroed = oracle.attention_f64(q, k, v, causal=True, key_valid=valid)
    tail = oracle.attention_f64(q[:, :, pad:], k[:, :, pad:], v[:, :, pad:], causal=True)
    assert np.max(np.abs(filled[:, :, pad:] - tail)) < 1e-12
    assert np.array_equal(filled[:, :, pad:], zeroed[:, :, pad:])
    mean_v = v.astype(np.float64).mean(axis=2, keepdims=True)
    assert np.max(np.abs(filled[:, :, :pad] - mean_v)) < 1e-12
    assert np.all(zeroed[:, :, :pad] == 0.0)
    # the literal statement: scores filled with -1e30 before a dense softmax
    literal = oracle.np_attention(q, k, v, causal=True, key_valid=valid, fill_value=-1.0e30)
    assert np.max(np.abs(filled - literal)) < 1e-12


def test_key_mask_with_segments_and_right_padding_correctness(oracle):
    """Right padding plus per-frame segments: padded keys drop out of their segment only."""
    rng = np.random.default_rng(13)
    cu = np.array([0, 5, 12], np.int32)
    q = rng.standard_normal((2, 2, 12, 8)).astype(np.float32)
    k = rng.standard_normal((2, 2, 12, 8)).astype(np.float32)
    v = rng.standard_normal((2, 2, 12, 8)).astype(np.float32)
    valid = np.ones((2, 12), bool)
    valid[1, 9:] = False
    for causal in (False, True):
        a = oracle.attention_f64(q, k, v, causal=causal, cu_seqlens=cu, key_valid=valid)
        b = oracle.np_attention(q, k, v, causal=causal, cu_seqlens=cu, key_valid=valid)
        assert np.max(np.abs(a - b)) < 1e-12
    # batch 0 has no padding: identical to the unmasked call
    a0 = oracle.attention_f64(q[:1], k[:1], v[:1], cu_seqlens=cu, key_valid=valid[:1])
    assert np.array_equal(a0, oracle.attention_f64(q[:1], k[:1], v[:1], cu_seqlens=cu))
