"""Seeded synthetic inputs of the five benchmark workloads (numpy PCG64, host side).

Seeds: 20261201 + 16 * config + tensor index.  Values are drawn in float32 and rounded to the
workload's input dtype on the host; every checker receives the same rounded values.

  C1  op-level plumbing: attention B1 H4 S256 D64 f32; Q4 linear M256 K512 N512 f32 activations
  C2  Boogu Turbo 1024px joint attention: B1 H24 D128, S = 512 text + 64x64 image = 4608, bf16
  C3  Boogu DiT Q4 projections at M4608, hidden 3072: (K, N) in
      (3072, 9216) QKV, (3072, 3072) O, (3072, 12288) MLP up, (12288, 3072) MLP down; bf16
  C4  Boogu Edit Turbo 1.5K joint attention: S = 512 + 96x96 reference + 96x96 target = 18944
  C5  Qwen3-VL-style prefill: causal segment-masked GQA Hq32 Hkv8 D128 S1024 bf16, and Q4
      projections (Qwen layout) M1024 K4096 N in (6144, 4096)
"""
from __future__ import annotations

import numpy as np

from .rope import position_ids, rope_values, text_rope_values

BASE_SEED = 20261201

C3_SHAPES = {"qkv": (3072, 9216), "o": (3072, 3072), "mlp_up": (3072, 12288),
             "mlp_down": (12288, 3072)}
C5_SHAPES = {"qkv": (4096, 6144), "o": (4096, 4096)}


def rng(config: int, index: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(BASE_SEED + 16 * config + index))


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16, returned as float32 values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000))
    return r.view(np.float32)


def round_to_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def rms_normalize(x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x = np.asarray(x, np.float32)
    rms = np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True) + eps)
    return (x / rms).astype(np.float32)


def apply_rope_interleaved(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [..., S, D] with cos/sin [S, D]: pairs (x0, x1) -> (x0 c - x1 s, x1 c + x0 s)."""
    rot = np.empty_like(x)
    rot[..., 0::2] = -x[..., 1::2]
    rot[..., 1::2] = x[..., 0::2]
    return (x * cos + rot * sin).astype(np.float32)


def apply_rope_half(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    h = x.shape[-1] // 2
    rot = np.concatenate([-x[..., h:], x[..., :h]], axis=-1)
    return (x * cos + rot * sin).astype(np.float32)


# ---------------------------------------------------------------------------------------------
# Q4 weights: signed nibbles ~ U{-8..7}, f32 block scales ~ U(0.005, 0.02)
# ---------------------------------------------------------------------------------------------

def pack_kn(q: np.ndarray) -> np.ndarray:
    """q int [K, N] -> words uint32 [K/8, N] (word (kw, n) holds k = 8 kw + lane)."""
    K, N = q.shape
    nib = (q.astype(np.int64) & 0xF).astype(np.uint32).reshape(K // 8, 8, N)
    words = np.zeros((K // 8, N), np.uint32)
    for lane in range(8):
        words |= nib[:, lane, :] << np.uint32(4 * lane)
    return words


def pack_nk(q: np.ndarray) -> np.ndarray:
    """q int [N, K] -> words uint32 [N, K/8] (eight consecutive k per word)."""
    N, K = q.shape
    nib = (q.astype(np.int64) & 0xF).astype(np.uint32).reshape(N, K // 8, 8)
    words = np.zeros((N, K // 8), np.uint32)
    for lane in range(8):
        words |= nib[:, :, lane] << np.uint32(4 * lane)
    return words


def q4_weight(config: int, index: int, K: int, N: int, layout: int, block: int = 128):
    """Random packed weight: returns (words, scales) for layout 1 ([K/8, N], [K/blk, N]) or
    layout 0 ([N, K/8], [N, K/blk])."""
    g = rng(config, index)
    if layout == 1:
        q = g.integers(-8, 8, size=(K, N), dtype=np.int8)
        scales = g.uniform(0.005, 0.02, size=(K // block, N)).astype(np.float32)
        return pack_kn(q), scales
    q = g.integers(-8, 8, size=(N, K), dtype=np.int8)
    scales = g.uniform(0.005, 0.02, size=(N, K // block)).astype(np.float32)
    return pack_nk(q), scales


def activations(config: int, index: int, M: int, K: int, dtype: str) -> np.ndarray:
    x = rng(config, index).standard_normal((M, K), dtype=np.float32)
    return round_to_bf16(x) if dtype == "bf16" else (round_to_f16(x) if dtype == "f16" else x)


# ---------------------------------------------------------------------------------------------
# attention inputs
# ---------------------------------------------------------------------------------------------

def c1_attention():
    """B1 H4 S256 D64 float32 N(0, 1); scale 1/8."""
    shape = (1, 4, 256, 64)
    return tuple(rng(1, i).standard_normal(shape, dtype=np.float32) for i in range(3))


def boogu_joint_ids(config: int) -> np.ndarray:
    if config == 2:
        return position_ids(512, [], (128, 128), 2)
    if config == 4:
        return position_ids(512, [(192, 192)], (192, 192), 2)
    raise ValueError(config)


def boogu_attention(config: int, heads: int = 24, head_dim: int = 128, seq_limit: int = 0):
    """Q/K: N(0,1) rows RMS-normalised per head (eps 1e-5, gamma 1) then Boogu interleaved RoPE
    (theta 1e4, axis dims [32, 48, 48]); V: N(0,1).  All rounded to bf16.  Layout [1, H, S, D].
    seq_limit > 0 truncates the sequence (for quick checks)."""
    ids = boogu_joint_ids(config)
    if seq_limit:
        ids = ids[:seq_limit]
    S = ids.shape[0]
    cos, sin = rope_values(ids, [32, 48, 48], 1.0e4)
    out = []
    for i in range(3):
        x = rng(config, i).standard_normal((1, heads, S, head_dim), dtype=np.float32)
        if i < 2:
            x = apply_rope_interleaved(rms_normalize(x), cos, sin)
        out.append(round_to_bf16(x))
    return tuple(out)


def c5_segments(total: int = 1024, lo: int = 64, hi: int = 512, config: int = 5) -> np.ndarray:
    """Segment lengths ~ U{64..512} drawn until the remainder is < 64; the remainder is folded
    into the last segment (split in two if that exceeds 512).  Returns cu_seqlens int32."""
    g = rng(config, 15)
    lengths = []
    remaining = total
    while remaining >= lo:
        L = int(g.integers(lo, hi + 1))
        if L > remaining:
            L = remaining
        lengths.append(L)
        remaining -= L
    if remaining:
        if lengths:
            lengths[-1] += remaining
        else:
            lengths.append(remaining)
        if lengths[-1] > hi:
            last = lengths.pop()
            lengths.extend([last // 2, last - last // 2])
    cu = np.zeros(len(lengths) + 1, np.int32)
    cu[1:] = np.cumsum(lengths)
    return cu


def c5_attention(heads: int = 32, kv_heads: int = 8, head_dim: int = 128, S: int = 1024):
    """bf16 Q [1, 32, S, D], K/V [1, 8, S, D] ~ N(0,1) with Qwen rotate_half RoPE (theta 5e6,
    positions restarting per segment) on Q and K; cu_seqlens of the packed segments."""
    cu = c5_segments(S)
    pos = np.concatenate([np.arange(cu[i + 1] - cu[i]) for i in range(len(cu) - 1)])
    cos, sin = text_rope_values(pos, head_dim, 5.0e6)
    q = rng(5, 0).standard_normal((1, heads, S, head_dim), dtype=np.float32)
    k = rng(5, 1).standard_normal((1, kv_heads, S, head_dim), dtype=np.float32)
    v = rng(5, 2).standard_normal((1, kv_heads, S, head_dim), dtype=np.float32)
    q = apply_rope_half(q, cos, sin)
    k = apply_rope_half(k, cos, sin)
    return round_to_bf16(q), round_to_bf16(k), round_to_bf16(v), cu


def attention_flops(B: int, H: int, D: int, pairs: int) -> float:
    """4 * B * H * D * (number of unmasked (i, j) pairs)."""
    return 4.0 * B * H * D * pairs


def segment_causal_pairs(cu: np.ndarray) -> int:
    L = np.diff(np.asarray(cu, np.int64))
    return int(np.sum(L * (L + 1) // 2))


def c5_padded_attention(heads: int = 32, kv_heads: int = 8, head_dim: int = 128, S: int = 1024,
                        left_pad: int = 137, right_pad: int = 301):
    """The C5 shape as a padded batch of two prompts (crates/burn_qwen3_vl/src/processor.rs:
    379-392): batch 0 left-padded by `left_pad` tokens, batch 1 right-padded by `right_pad`.
    bf16 Q [2, 32, S, D], K/V [2, 8, S, D] ~ N(0,1) with rotate_half RoPE (theta 5e6) at the
    valid tokens' positions; returns (q, k, v, key_valid [2, S] bool)."""
    valid = np.ones((2, S), bool)
    valid[0, :left_pad] = False
    valid[1, S - right_pad:] = False
    pos = np.stack([np.maximum(np.arange(S) - left_pad, 0), np.arange(S)])
    out = []
    for i, h in enumerate((heads, kv_heads, kv_heads)):
        x = rng(5, 8 + i).standard_normal((2, h, S, head_dim), dtype=np.float32)
        if i < 2:
            for b in range(2):
                cos, sin = text_rope_values(pos[b], head_dim, 5.0e6)
                x[b] = apply_rope_half(x[b], cos, sin)
        out.append(round_to_bf16(x))
    return out[0], out[1], out[2], valid
