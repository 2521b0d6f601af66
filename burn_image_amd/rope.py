"""Host-side RoPE tables and position ids (computed once per request on the host, as in the
reference).

* ``position_ids``  <- crates/burn_boogu/src/rope.rs:28-92 (text, references, generated image)
* ``rope_values``   <- crates/burn_boogu/src/model/denoiser.rs:992-1034 (f64 phase, f32 cos/sin,
  each value repeated for the two interleaved lanes of its pair)
* ``text_rope_values`` <- Qwen rotate_half tables (1-D positions, theta 5e6 for Qwen3-VL text;
  crates/burn_qwen3_vl/src/config.rs:327-328), cos/sin duplicated over the two halves.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np


def position_ids(text_len: int, references: Sequence[Tuple[int, int]], generated: Tuple[int, int],
                 patch: int) -> np.ndarray:
    """[S, 3] uint32 ids: text [i, i, i]; each reference [axis0, row, col] with axis0 advanced by
    max(rows, cols) after it; the generated image last."""
    if patch == 0:
        raise ValueError("RoPE patch must be non-zero")
    values: List[Tuple[int, int, int]] = [(i, i, i) for i in range(text_len)]
    axis_zero = text_len
    for (height, width) in references:
        if height % patch or width % patch:
            raise ValueError("reference latent is not divisible by patch size")
        rows, cols = height // patch, width // patch
        values.extend((axis_zero, r, c) for r in range(rows) for c in range(cols))
        axis_zero += max(rows, cols)
    height, width = generated
    if height % patch or width % patch:
        raise ValueError("generated latent is not divisible by patch size")
    rows, cols = height // patch, width // patch
    values.extend((axis_zero, r, c) for r in range(rows) for c in range(cols))
    return np.asarray(values, dtype=np.uint32).reshape(-1, 3)


def rope_values(ids: np.ndarray, axis_dims: Sequence[int], theta: float):
    """cos, sin [S, sum(axis_dims)] float32 for Boogu's interleaved-pair RoPE."""
    ids = np.asarray(ids, dtype=np.uint32)
    cols_cos, cols_sin = [], []
    for axis, dim in enumerate(axis_dims):
        pairs = np.arange(dim // 2, dtype=np.float64)
        inv = np.power(np.float64(theta), -(2.0 * pairs) / float(dim))
        phase = ids[:, axis].astype(np.float64)[:, None] * inv[None, :]
        c = np.cos(phase).astype(np.float32)
        s = np.sin(phase).astype(np.float32)
        cols_cos.append(np.repeat(c, 2, axis=1))
        cols_sin.append(np.repeat(s, 2, axis=1))
    return np.concatenate(cols_cos, axis=1), np.concatenate(cols_sin, axis=1)


def text_rope_values(positions: np.ndarray, head_dim: int, theta: float):
    """cos, sin [S, head_dim] float32 for rotate_half RoPE: frequency theta^(-2i/d) for
    i < d/2, the table repeated over both halves."""
    pos = np.asarray(positions, dtype=np.float64)
    inv = np.power(np.float64(theta), -np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    phase = pos[:, None] * inv[None, :]
    c = np.cos(phase).astype(np.float32)
    s = np.sin(phase).astype(np.float32)
    return np.concatenate([c, c], axis=1), np.concatenate([s, s], axis=1)
