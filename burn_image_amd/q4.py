"""Packed signed-Q4 (Q4S, f32 block scales) weights on the GPU.

Mirrors the reference's Q4S storage contract and quantizers
(crates/burn_boogu/src/artifacts.rs:513-536, 7203-7288, 7296-7388); quantisation, dequantisation
and every matmul run in libbiq's HIP kernels.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

# Owners of model matrices (artifacts.rs `TensorOwner`).
QWEN3_VL = "qwen3_vl"
BOOGU_DENOISER = "boogu_denoiser"
FLUX_VAE = "flux_vae"

_LAYOUT_OF_OWNER = {QWEN3_VL: _lib.Q4_NK_AXIS0, BOOGU_DENOISER: _lib.Q4_KN_AXIS1}


def q4s_storage_block_and_axis(owner: str, shape: Sequence[int]) -> Optional[Tuple[int, int]]:
    """Exact Q4S storage block and packed axis of a rank-two matrix, or None
    (artifacts.rs:513-525).  Qwen packs its last axis (axis 0 of PackedU32) with block 128;
    Boogu packs the input axis (PackedU32(1)) with the largest of 128, 64, 32, 16, 8 dividing it."""
    if len(shape) != 2 or owner not in _LAYOUT_OF_OWNER:
        return None
    layout = _LAYOUT_OF_OWNER[owner]
    block = _lib.load().biq_q4_storage_block(layout, int(shape[0]), int(shape[1]))
    if block == 0:
        return None
    return block, (0 if layout == _lib.Q4_NK_AXIS0 else 1)


def q4s_stored_dtype(owner: str, shape: Sequence[int]) -> Optional[str]:
    """Inventory dtype spelling of the storage contract (artifacts.rs:527-536)."""
    if len(shape) != 2 or owner not in _LAYOUT_OF_OWNER:
        return None
    buf = ctypes.create_string_buffer(64)
    rc = _lib.load().biq_q4_stored_dtype(_LAYOUT_OF_OWNER[owner], int(shape[0]), int(shape[1]),
                                         buf, 64)
    if rc != _lib.OK:
        return None
    return buf.value.decode()


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")


@dataclass
class Q4Weight:
    """A packed signed-Q4 matrix resident on the GPU.

    layout Q4_KN_AXIS1 (Boogu): logical shape (K, N); words int32 view of u32 [K/8, N];
        scales f32 [K/block, N].
    layout Q4_NK_AXIS0 (Qwen): logical shape (N, K); words [N, K/8]; scales [N, K/block];
        the GEMM consumes W^T (crates/burn_qwen3_vl/src/linear.rs:58-62).
    """

    words: torch.Tensor
    scales: torch.Tensor
    layout: int
    block: int
    shape: Tuple[int, int]

    @property
    def K(self) -> int:
        return self.shape[0] if self.layout == _lib.Q4_KN_AXIS1 else self.shape[1]

    @property
    def N(self) -> int:
        return self.shape[1] if self.layout == _lib.Q4_KN_AXIS1 else self.shape[0]

    @property
    def device(self) -> torch.device:
        return self.words.device

    def nbytes(self) -> int:
        return self.words.numel() * 4 + self.scales.numel() * 4

    def stored_dtype(self) -> str:
        if self.layout == _lib.Q4_NK_AXIS0:
            return f"q4s-block{self.block}-f32-packed-axis0"
        return f"q4s-block{self.block}x1-f32-packed-axis1"

    def dequantize(self) -> torch.Tensor:
        """Bit-exact f32 dequantisation `f32(q) * scale` in the logical shape."""
        out = torch.empty(self.shape, dtype=torch.float32, device=self.device)
        _lib.check(_lib.load().biq_q4_dequant_f32(
            _stream_ptr(self.device), self.words.data_ptr(), self.scales.data_ptr(), self.layout,
            self.block, self.K, self.N, out.data_ptr()))
        return out


def from_packed(words: torch.Tensor, scales: torch.Tensor, layout: int, block: int,
                shape: Tuple[int, int]) -> Q4Weight:
    """Wrap already-packed Q4S buffers (e.g. loaded from an artifact: values then scales,
    artifacts.rs:7364-7377) without copying."""
    _require_cuda(words, "words")
    _require_cuda(scales, "scales")
    rows, cols = int(shape[0]), int(shape[1])
    K, N = (rows, cols) if layout == _lib.Q4_KN_AXIS1 else (cols, rows)
    exp_words = (K // 8, N) if layout == _lib.Q4_KN_AXIS1 else (N, K // 8)
    exp_scales = (K // block, N) if layout == _lib.Q4_KN_AXIS1 else (N, K // block)
    if tuple(words.shape) != exp_words or tuple(scales.shape) != exp_scales:
        raise ValueError(f"packed Q4S buffers {tuple(words.shape)}/{tuple(scales.shape)} do not "
                         f"match shape {shape} block {block} layout {layout}")
    if words.dtype not in (torch.int32, torch.uint32) or scales.dtype != torch.float32:
        raise ValueError("packed Q4S words must be 32-bit and scales float32")
    return Q4Weight(words.contiguous(), scales.contiguous(), layout, block, (rows, cols))


def payload_layout(stored_dtype: str, shape: Sequence[int], payload_bytes: int):
    """(layout, block, words_bytes, scales_bytes) of a Q4S payload for a logical [rows, cols]
    weight stored as `stored_dtype`, after libbiq checks the string and the size against the
    storage contract (artifacts.rs:513-536,7276-7283,7364-7377; boogu_import.rs:1693-1719)."""
    if len(shape) != 2:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "Q4S payloads hold rank-two matrices")
    lay, blk = ctypes.c_int(), ctypes.c_int()
    wb, sb = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(_lib.load().biq_q4_payload_layout(stored_dtype.encode(), int(shape[0]), int(shape[1]),
                                                 int(payload_bytes), ctypes.byref(lay), ctypes.byref(blk),
                                                 ctypes.byref(wb), ctypes.byref(sb)))
    return lay.value, blk.value, wb.value, sb.value


def split_payload(payload: torch.Tensor, stored_dtype: str, shape: Sequence[int]):
    """Views (words int32, scales float32, layout, block) into a flat uint8 payload (host or
    device) -- no copy: words [K/8, N] (axis 1) or [N, K/8] (axis 0), then scales."""
    if payload.dtype != torch.uint8 or payload.dim() != 1 or not payload.is_contiguous():
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "a Q4S payload is a contiguous flat uint8 tensor")
    lay, blk, wb, sb = payload_layout(stored_dtype, shape, payload.numel())
    if payload.data_ptr() % 16 != 0:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "Q4S payloads must be 16-byte aligned")
    rows, cols = int(shape[0]), int(shape[1])
    K, N = (rows, cols) if lay == _lib.Q4_KN_AXIS1 else (cols, rows)
    words = payload[:wb].view(torch.int32).view((K // 8, N) if lay == _lib.Q4_KN_AXIS1 else (N, K // 8))
    scales = payload[wb:wb + sb].view(torch.float32).view((K // blk, N) if lay == _lib.Q4_KN_AXIS1 else (N, K // blk))
    return words, scales, lay, blk


def from_payload(payload: torch.Tensor, stored_dtype: str, shape: Tuple[int, int]) -> Q4Weight:
    """A Q4Weight over a Q4S tensor payload resident on the GPU (the importer's values-then-scales
    bytes, e.g. read from an artifact), without copying; the contract is checked first."""
    _require_cuda(payload, "payload")
    words, scales, lay, blk = split_payload(payload, stored_dtype, shape)
    return Q4Weight(words, scales, lay, blk, (int(shape[0]), int(shape[1])))


def quantize_row_layout_q4s_block_up_to128_f32(weight: torch.Tensor) -> Q4Weight:
    """GPU restatement of artifacts.rs:7296-7388 for a Boogu [input, output] matrix.
    F16 input is widened to F32 first, as the reference does."""
    _require_cuda(weight, "weight")
    if weight.dtype not in (torch.float16, torch.float32):
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                   f"runtime Q4S denoiser quantization requires F16/F32, found {weight.dtype}")
    if weight.dim() != 2:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                   "runtime Q4S denoiser quantization requires a rank-two matrix")
    w = weight.to(torch.float32).contiguous()
    K, N = w.shape
    block = _lib.load().biq_q4_storage_block(_lib.Q4_KN_AXIS1, K, N)
    if block == 0:
        # let the library produce the reference's error message
        block = 8
    words = torch.empty((max(K // 8, 1), max(N, 1)), dtype=torch.int32, device=w.device)
    scales = torch.empty((max(K // block, 1), max(N, 1)), dtype=torch.float32, device=w.device)
    _lib.check(_lib.load().biq_q4_quantize(_stream_ptr(w.device), w.data_ptr(), _lib.Q4_KN_AXIS1,
                                           K, N, words.data_ptr(), scales.data_ptr()))
    return Q4Weight(words, scales, _lib.Q4_KN_AXIS1, block, (K, N))


def quantize_q4s_block128_f32(values: torch.Tensor) -> Q4Weight:
    """GPU restatement of artifacts.rs:7203-7288 for a Qwen [out, in] = [N, K] matrix."""
    _require_cuda(values, "values")
    if values.dim() != 2:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "Q4S block tensor must be a matrix here")
    v = values.to(torch.float32).contiguous()
    N, K = v.shape
    words = torch.empty((max(N, 1), max(K // 8, 1)), dtype=torch.int32, device=v.device)
    scales = torch.empty((max(N, 1), max(K // 128, 1)), dtype=torch.float32, device=v.device)
    _lib.check(_lib.load().biq_q4_quantize(_stream_ptr(v.device), v.data_ptr(), _lib.Q4_NK_AXIS0,
                                           K, N, words.data_ptr(), scales.data_ptr()))
    return Q4Weight(words, scales, _lib.Q4_NK_AXIS0, 128, (N, K))
