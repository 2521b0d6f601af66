"""CPU oracle for the denoiser attention block (TEST INFRASTRUCTURE ONLY).

Two independent statements of the reference algorithms live here:

* ``C``: ctypes bindings to ``oracle/liboracle.so`` built from ``oracle/oracle.c`` (the primary
  oracle: byte-exact Q4S quantizers, float64 GEMM and attention, and the CPU baseline that
  restates Burn's NdArray path);
* ``np_*``: vectorised numpy restatements used to cross-check the C oracle on small inputs.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module, and only to check results against; the product library never calls it.  Reference citations are
``file:line`` relative to the reference repository root.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

FLT_MIN = np.float32(1.1754944e-38)

_lib = None


def build(force: bool = False) -> str:
    """Compile ``oracle/liboracle.so`` with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-C", HERE, "-B" if force else "-s", "liboracle.so"], check=True,
                       stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.orc_q4_kn_block.argtypes = [I64, I64]
        L.orc_q4_kn_block.restype = ctypes.c_int
        L.orc_q4_quantize_kn.argtypes = [P, I64, I64, P, P, P]
        L.orc_q4_quantize_kn.restype = ctypes.c_int
        L.orc_q4_quantize_nk.argtypes = [P, I64, I64, P, P]
        L.orc_q4_quantize_nk.restype = ctypes.c_int
        L.orc_q4_dequant.argtypes = [P, P, ctypes.c_int, ctypes.c_int, I64, I64, P]
        L.orc_q4_dequant.restype = None
        L.orc_q4_linear_f64.argtypes = [P, I64, P, I64, P, P, ctypes.c_int, ctypes.c_int, I64, P, P]
        L.orc_q4_linear_f64.restype = None
        L.orc_cpu_q4_linear_f32.argtypes = [P, I64, I64, P, P, ctypes.c_int, ctypes.c_int, I64, P]
        L.orc_cpu_q4_linear_f32.restype = ctypes.c_int
        L.orc_effective_query_chunk.argtypes = [I64, I64]
        L.orc_effective_query_chunk.restype = I64
        L.orc_attention_f64.argtypes = [P, P, P, I64, I64, I64, I64, I64, I64, I64, ctypes.c_double,
                                        ctypes.c_int, P, I64, P, ctypes.c_int, P, I64, P]
        L.orc_attention_f64.restype = None
        L.orc_cpu_attention_f32.argtypes = [P, P, P, I64, I64, I64, I64, I64, I64, I64,
                                            ctypes.c_float, I64, I64, P]
        L.orc_cpu_attention_f32.restype = ctypes.c_int
        L.orc_rope_values.argtypes = [P, I64, P, ctypes.c_double, P, P]
        L.orc_rope_values.restype = None
        L.orc_rms_norm_f32.argtypes = [P, I64, I64, P, ctypes.c_float, P]
        L.orc_rms_norm_f32.restype = None
        L.orc_apply_rope_interleaved.argtypes = [P, I64, I64, P, P, P]
        L.orc_apply_rope_interleaved.restype = None
        L.orc_apply_rope_half.argtypes = [P, I64, I64, P, P, P]
        L.orc_apply_rope_half.restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ----------------------------------------------------------------------------------------------
# C oracle wrappers
# ----------------------------------------------------------------------------------------------

class OracleError(ValueError):
    """The reference would return an error for this input."""


def q4_kn_block(K: int, N: int) -> int:
    """Largest exact Boogu block (artifacts.rs:519-523); 0 when none applies."""
    return int(lib().orc_q4_kn_block(K, N))


def q4_quantize_kn(w: np.ndarray):
    """quantize_row_layout_q4s_block_up_to128_f32 (artifacts.rs:7296-7388).

    w: [K, N] float32 (float16 input is widened first, as the reference converts to F32).
    Returns (words [K/8, N] uint32, scales [K/blk, N] float32, blk)."""
    w = _c(np.asarray(w).astype(np.float32), np.float32)
    if w.ndim != 2:
        raise OracleError("runtime Q4S denoiser quantization requires a rank-two matrix")
    K, N = w.shape
    blk = q4_kn_block(K, N)
    if blk == 0:
        raise OracleError(f"no supported exact block for shape {w.shape}")
    words = np.zeros((K // 8, N), np.uint32)
    scales = np.zeros((K // blk, N), np.float32)
    out_blk = ctypes.c_int(0)
    rc = lib().orc_q4_quantize_kn(_p(w), K, N, _p(words), _p(scales), ctypes.byref(out_blk))
    if rc != 0:
        raise OracleError("cannot quantize a non-finite denoiser checkpoint value")
    return words, scales, out_blk.value


def q4_quantize_nk(values: np.ndarray):
    """quantize_q4s_block128_f32 (artifacts.rs:7203-7288) for a [rows, inner] matrix.

    Returns (words [rows, inner/8] uint32, scales [rows, inner/128] float32)."""
    values = _c(values, np.float32)
    if values.ndim < 1 or values.size == 0:
        raise OracleError("Q4S block tensor must have at least one dimension")
    inner = values.shape[-1]
    rows = values.size // inner
    if inner % 128:
        raise OracleError(f"Q4S innermost dimension {inner} is not divisible by 128")
    words = np.zeros((rows, inner // 8), np.uint32)
    scales = np.zeros((rows, inner // 128), np.float32)
    rc = lib().orc_q4_quantize_nk(_p(values), rows, inner, _p(words), _p(scales))
    if rc != 0:
        raise OracleError("cannot quantize a non-finite checkpoint value")
    return words, scales


def q4_dequant(words, scales, layout: int, block: int, K: int, N: int) -> np.ndarray:
    """Bit-exact dequantisation `f32(q) * scale` (artifacts.rs:10434-10440).
    Output: [K, N] for layout 1 (Boogu), [N, K] for layout 0 (Qwen)."""
    words = _c(words, np.uint32)
    scales = _c(scales, np.float32)
    out = np.zeros((K, N) if layout == 1 else (N, K), np.float32)
    lib().orc_q4_dequant(_p(words), _p(scales), layout, block, K, N, _p(out))
    return out


def q4_linear_f64(x, words, scales, layout: int, block: int, N: int, rows=None, bias=None):
    """float64 Y = X . dequant(W) for the selected rows (linear.rs:14-37; qwen linear.rs:107-140)."""
    x = _c(x, np.float32)
    M, K = x.shape
    idx = None if rows is None else _c(rows, np.int64)
    nrows = M if idx is None else idx.size
    y = np.zeros((nrows, N), np.float64)
    b = None if bias is None else _c(bias, np.float32)
    lib().orc_q4_linear_f64(_p(x), K, None if idx is None else _p(idx), nrows, _p(_c(words, np.uint32)),
                            _p(_c(scales, np.float32)), layout, block, N,
                            None if b is None else _p(b), _p(y))
    return y


def cpu_q4_linear_f32(x, words, scales, layout: int, block: int, N: int):
    """CPU baseline: restated Burn NdArray q_matmul (dequantize, f32 matmul).  Returns (y, threads)."""
    x = _c(x, np.float32)
    M, K = x.shape
    y = np.zeros((M, N), np.float32)
    t = lib().orc_cpu_q4_linear_f32(_p(x), M, K, _p(_c(words, np.uint32)), _p(_c(scales, np.float32)),
                                    layout, block, N, _p(y))
    return y, int(t)


def effective_query_chunk(query_len: int, requested: int) -> int:
    return int(lib().orc_effective_query_chunk(query_len, requested))


def attention_f64(q, k, v, scale=None, causal=False, cu_seqlens=None, rows=None, key_valid=None,
                  fill_mean=False):
    """Exact float64 attention over [B, H, S, D] inputs (GQA when k/v have fewer heads).
    key_valid: optional [B, Skv] bool (True = the key may be attended, Qwen's attention_mask);
    rows left without a visible key get mean(V) with `fill_mean` (text.rs:177-182), else 0."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    B, Hq, Sq, D = q.shape
    _, Hkv, Skv, _ = k.shape
    Dv = v.shape[3]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    idx = None if rows is None else _c(rows, np.int64)
    nrows = Sq if idx is None else idx.size
    out = np.zeros((B, Hq, nrows, Dv), np.float64)
    cu = None if cu_seqlens is None else _c(cu_seqlens, np.int32)
    nseg = 0 if cu is None else cu.size - 1
    kv = None if key_valid is None else _c(np.asarray(key_valid).reshape(B, Skv) != 0, np.uint8)
    lib().orc_attention_f64(_p(q), _p(k), _p(v), B, Hq, Hkv, Sq, Skv, D, Dv, float(scale), int(causal),
                            None if cu is None else _p(cu), nseg, None if kv is None else _p(kv),
                            int(bool(fill_mean)), None if idx is None else _p(idx), nrows, _p(out))
    return out


def cpu_attention_f32(q, k, v, scale=None, requested_chunk=8192, q_rows=None):
    """CPU baseline: restated query-chunked f32 attention (attention.rs:875-914)."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    B, Hq, Sq, D = q.shape
    _, Hkv, Skv, _ = k.shape
    Dv = v.shape[3]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    q_rows = Sq if q_rows is None else q_rows
    out = np.zeros((B, Hq, Sq, Dv), np.float32)
    t = lib().orc_cpu_attention_f32(_p(q), _p(k), _p(v), B, Hq, Hkv, Sq, Skv, D, Dv, float(scale),
                                    requested_chunk, q_rows, _p(out))
    return out, int(t)


def rope_values(ids, axis_dims, theta: float):
    ids = _c(ids, np.uint32)
    S = ids.shape[0]
    dims = _c(axis_dims, np.int64)
    hd = int(dims.sum())
    cs = np.zeros((S, hd), np.float32)
    sn = np.zeros((S, hd), np.float32)
    lib().orc_rope_values(_p(ids), S, _p(dims), float(theta), _p(cs), _p(sn))
    return cs, sn


def rms_norm(x, gamma, eps: float):
    x = _c(x, np.float32)
    D = x.shape[-1]
    rows = x.size // D
    y = np.zeros_like(x)
    lib().orc_rms_norm_f32(_p(x), rows, D, _p(_c(gamma, np.float32)), np.float32(eps), _p(y))
    return y


def apply_rope_interleaved(x, cs, sn):
    x = _c(x, np.float32)
    D = x.shape[-1]
    rows = x.size // D
    y = np.zeros_like(x)
    lib().orc_apply_rope_interleaved(_p(x), rows, D, _p(_c(np.broadcast_to(cs, x.shape), np.float32)),
                                     _p(_c(np.broadcast_to(sn, x.shape), np.float32)), _p(y))
    return y


def apply_rope_half(x, cs, sn):
    x = _c(x, np.float32)
    D = x.shape[-1]
    rows = x.size // D
    y = np.zeros_like(x)
    lib().orc_apply_rope_half(_p(x), rows, D, _p(_c(np.broadcast_to(cs, x.shape), np.float32)),
                              _p(_c(np.broadcast_to(sn, x.shape), np.float32)), _p(y))
    return y


def round_to(x, dtype: str) -> np.ndarray:
    """Round float32 values to `dtype` ("f32", "f16", "bf16", nearest even), returned as f32."""
    x = np.asarray(x, np.float32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    u = np.ascontiguousarray(x).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def qk_norm_rope_ref(x, gamma, eps: float, cos, sin, in_dtype: str, layout: str):
    """Per-row Q/K preparation before the final cast (rows [..., D], values representable in
    in_dtype F).  The strict-F32 RMS is cast to F and the normalisation runs in F
    (crates/burn_boogu/src/model/native_flash.rs:431-451: `let rms = F::cast_from(rms)`, then
    `x / rms * gamma`; Burn's nn::RmsNorm via rms_normalized, norm.rs:28-35).  RoPE:
    "interleaved" = the Boogu fused kernel's pairs in F (native_flash.rs:452-474, tables of type
    F); "half" = Qwen's apply_text_rope in f32 then cast to F (crates/burn_qwen3_vl/src/
    text.rs:425-440).  Each F operation is one f32 operation rounded to F."""
    F = lambda a: round_to(a, in_dtype)  # noqa: E731
    x = np.asarray(x, np.float32)
    D = x.shape[-1]
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    rms = F(np.sqrt((ss.astype(np.float32) / np.float32(D)) + np.float32(eps)).astype(np.float32))
    n = F(F(x / rms) * F(np.broadcast_to(np.asarray(gamma, np.float32), x.shape)))
    cos = np.broadcast_to(np.asarray(cos, np.float32), x.shape)
    sin = np.broadcast_to(np.asarray(sin, np.float32), x.shape)
    rot = np.empty_like(n)
    if layout == "interleaved":
        rot[..., 0::2] = -n[..., 1::2]
        rot[..., 1::2] = n[..., 0::2]
        return F(F(n * F(cos)) + F(rot * F(sin)))
    h = D // 2
    rot[..., :h] = -n[..., h:]
    rot[..., h:] = n[..., :h]
    return F((n * cos).astype(np.float32) + (rot * sin).astype(np.float32))


# ----------------------------------------------------------------------------------------------
# Independent numpy restatements (cross-checks for the C oracle on small inputs)
# ----------------------------------------------------------------------------------------------

def np_round_half_away(x: np.ndarray) -> np.ndarray:
    return (np.sign(x) * np.floor(np.abs(x) + np.float32(0.5))).astype(np.float32)


def np_q4_quantize_kn(w: np.ndarray):
    """Vectorised restatement of artifacts.rs:7296-7388."""
    w = np.asarray(w, np.float32)
    K, N = w.shape
    blk = next(b for b in (128, 64, 32, 16, 8) if K % b == 0)
    alpha = np.abs(w).reshape(K // blk, blk, N).max(axis=1)
    scales = np.where(alpha == 0, FLT_MIN, (alpha / np.float32(7.0)).astype(np.float32)).astype(np.float32)
    inverse = (np.float32(1.0) / scales).astype(np.float32)
    prod = (w.reshape(K // blk, blk, N) * inverse[:, None, :]).astype(np.float32)
    q = np.clip(np_round_half_away(prod), -7, 7).astype(np.int8).reshape(K, N)
    nib = (q.astype(np.uint8) & 0x0F).astype(np.uint32).reshape(K // 8, 8, N)
    words = np.zeros((K // 8, N), np.uint32)
    for lane in range(8):
        words |= nib[:, lane, :] << np.uint32(4 * lane)
    return words, scales, blk


def np_q4_quantize_nk(values: np.ndarray):
    """Vectorised restatement of artifacts.rs:7203-7288."""
    values = np.asarray(values, np.float32)
    inner = values.shape[-1]
    rows = values.size // inner
    chunks = values.reshape(-1, 128)
    alpha = np.abs(chunks).max(axis=1)
    scales = np.where(alpha == 0, FLT_MIN, (alpha / np.float32(7.0)).astype(np.float32)).astype(np.float32)
    inverse = (np.float32(1.0) / scales).astype(np.float32)
    q = np.clip(np_round_half_away((chunks * inverse[:, None]).astype(np.float32)), -7, 7).astype(np.int8)
    nib = (q.astype(np.uint8) & 0x0F).astype(np.uint32).reshape(-1, 8)
    words = np.zeros(nib.shape[0], np.uint32)
    for lane in range(8):
        words |= nib[:, lane] << np.uint32(4 * lane)
    return words.reshape(rows, inner // 8), scales.reshape(rows, inner // 128)


def np_unpack_q4(words: np.ndarray) -> np.ndarray:
    """Signed nibbles of each word along a new trailing axis of 8 (lane l at bits 4l..4l+3)."""
    w = np.asarray(words, np.uint32)
    lanes = np.stack([(w >> np.uint32(4 * l)) & np.uint32(0xF) for l in range(8)], axis=-1).astype(np.int32)
    return np.where(lanes >= 8, lanes - 16, lanes).astype(np.int8)


def np_q4_dequant(words, scales, layout: int, block: int, K: int, N: int) -> np.ndarray:
    q = np_unpack_q4(words)
    if layout == 1:  # [K/8, N, 8] -> [K, N]
        qk = np.transpose(q, (0, 2, 1)).reshape(K, N).astype(np.float32)
        s = np.repeat(np.asarray(scales, np.float32), block, axis=0)
        return (qk * s).astype(np.float32)
    qn = q.reshape(N, K).astype(np.float32)  # [N, K/8, 8] -> [N, K]
    s = np.repeat(np.asarray(scales, np.float32), block, axis=1)
    return (qn * s).astype(np.float32)


def np_attention(q, k, v, scale=None, causal=False, cu_seqlens=None, key_valid=None,
                 fill_value=None):
    """Dense float64 softmax(Q K^T s) V with optional causal / segment / key-padding masks and
    GQA.  Masked scores become -inf, or `fill_value` when given (Qwen's mask_fill(-1e30),
    text.rs:176: a row with every key masked then averages V over all keys)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, Sq, D = q.shape
    Hkv = k.shape[1]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    k = np.repeat(k, Hq // Hkv, axis=1)
    v = np.repeat(v, Hq // Hkv, axis=1)
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
    mask = np.ones((Sq, k.shape[2]), bool)
    if causal:
        mask &= np.tril(np.ones_like(mask))
    if cu_seqlens is not None:
        seg = np.searchsorted(np.asarray(cu_seqlens), np.arange(Sq), side="right") - 1
        mask &= seg[:, None] == seg[None, :]
    mask = np.broadcast_to(mask, (B, 1) + mask.shape)
    if key_valid is not None:
        mask = mask & (np.asarray(key_valid, bool).reshape(B, 1, 1, -1))
    s = np.where(mask, s, -np.inf if fill_value is None else float(fill_value))
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p, v)


# ----------------------------------------------------------------------------------------------
# Parity metrics (the reference's compare() set: boogu_denoiser_parity.rs:765-813)
# ----------------------------------------------------------------------------------------------

def parity_metrics(actual, expected) -> dict:
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    diff = a - e
    mean_abs_ref = float(np.mean(np.abs(e))) if e.size else 0.0
    rmse = float(np.sqrt(np.mean(diff * diff))) if e.size else 0.0
    ref_rms = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    denom = float(np.linalg.norm(a) * np.linalg.norm(e))
    return {
        "max_abs": float(np.max(np.abs(diff))) if e.size else 0.0,
        "mean_abs": float(np.mean(np.abs(diff))) if e.size else 0.0,
        "mean_rel": float(np.mean(np.abs(diff)) / mean_abs_ref) if mean_abs_ref > 0 else 0.0,
        "rmse": rmse,
        "rel_rmse": rmse / ref_rms if ref_rms > 0 else 0.0,
        "cosine": float(np.dot(a, e) / denom) if denom > 0 else 1.0,
        "finite": bool(np.all(np.isfinite(a))),
    }
