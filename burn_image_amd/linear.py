"""Q4-preserving linear projections on libbiq's packed-Q4 GEMM.

Host-side mirror of the reference operator surface:
  * ``q_matmul``            <- QTensorOps::q_matmul (patches/burn-cubecl-0.21.0/src/ops/qtensor.rs:303-368)
  * ``linear_forward``      <- crates/burn_boogu/src/model/linear.rs:14-37
  * ``qwen_linear_forward`` <- crates/burn_qwen3_vl/src/linear.rs:107-140
Only packed-Q4 weights are accelerated; there is no dequantising or float fallback.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Union

import torch

from . import _lib
from .q4 import Q4Weight

_DTYPE_CODE = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16,
               torch.bfloat16: _lib.DTYPE_BF16}
SUPPORTED_BLOCKS = (8, 16, 32, 64, 128)


@dataclass
class Linear:
    """nn::Linear with a packed-Q4 weight.  Boogu weights are [d_input, d_output]
    (layout Q4_KN_AXIS1); Qwen weights keep the checkpoint [d_output, d_input] (Q4_NK_AXIS0)."""

    weight: Q4Weight
    bias: Optional[torch.Tensor] = None


def q_matmul(lhs: torch.Tensor, rhs: Q4Weight, out: Optional[torch.Tensor] = None,
             out_dtype: Optional[torch.dtype] = None, bias: Optional[torch.Tensor] = None,
             stream: Optional[int] = None) -> torch.Tensor:
    """lhs[..., K] . W -> [..., N] with W packed Q4S.

    The gate of the reference's packed route (symmetric Q4S, f32 scales, PackedU32(0|1),
    block in {8, 16, 32, 64, 128}) is checked; anything else raises instead of falling back.
    The output dtype defaults to float32 (the reference's lhs dtype on this route)."""
    if not isinstance(rhs, Q4Weight):
        raise _lib.Unsupported(_lib.ERR_UNSUPPORTED, "q_matmul accelerates packed-Q4 weights only")
    if rhs.block not in SUPPORTED_BLOCKS:
        raise _lib.Unsupported(_lib.ERR_UNSUPPORTED, f"Q4 block {rhs.block} is not supported")
    if lhs.dtype not in _DTYPE_CODE:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"lhs dtype {lhs.dtype} is not supported")
    if not lhs.is_cuda:
        raise ValueError("lhs must be a GPU tensor")
    K, N = rhs.K, rhs.N
    if lhs.shape[-1] != K:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                   f"lhs width {lhs.shape[-1]} does not match weight input {K}")
    lead = lhs.shape[:-1]
    x = lhs.reshape(-1, K)
    # The packed route makes lhs contiguous (qtensor.rs:329-336); a row-strided view is fine.
    if x.stride(-1) != 1 or (x.shape[0] > 1 and x.stride(0) < K):
        x = x.contiguous()
    M = x.shape[0]
    ldx = x.stride(0) if M > 1 else K
    odt = out_dtype or (out.dtype if out is not None else torch.float32)
    if out is None:
        out = torch.empty((M, N), dtype=odt, device=lhs.device)
    else:
        if out.dtype != odt or out.numel() != M * N or not out.is_contiguous():
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "out must be a contiguous [M, N] tensor")
    if bias is not None:
        bias = bias.to(torch.float32).contiguous()
    s = torch.cuda.current_stream(lhs.device).cuda_stream if stream is None else stream
    _lib.check(_lib.load().biq_q4_linear(
        s, x.data_ptr(), _DTYPE_CODE[x.dtype], M, K, ldx, rhs.words.data_ptr(),
        rhs.scales.data_ptr(), rhs.layout, rhs.block, N,
        None if bias is None else bias.data_ptr(), out.data_ptr(), _DTYPE_CODE[odt]))
    return out.reshape(*lead, N)


def linear_forward(linear: Linear, input: torch.Tensor, **kw) -> torch.Tensor:
    """Boogu projection keeping the packed weight intact (linear.rs:14-37): rank >= 2 input,
    weight [K, N] (Q4_KN_AXIS1), optional bias broadcast over the last axis."""
    if input.dim() < 2:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "Boogu linear projections require rank >= 2")
    if linear.weight.layout != _lib.Q4_KN_AXIS1:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "Boogu linear weights use the [K, N] row layout")
    return q_matmul(input, linear.weight, bias=linear.bias, **kw)


def qwen_linear_forward(linear: Linear, input: torch.Tensor, **kw) -> torch.Tensor:
    """Qwen projection over the checkpoint [N, K] weight consumed transposed
    (crates/burn_qwen3_vl/src/linear.rs:107-140)."""
    if input.dim() < 2:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "Qwen linear projections require rank >= 2")
    if linear.weight.layout != _lib.Q4_NK_AXIS0:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "Qwen linear weights use the [N, K] layout")
    return q_matmul(input, linear.weight, bias=linear.bias, **kw)


def q_matmul_swiglu(lhs: torch.Tensor, w1: Q4Weight, w3: Q4Weight, out: Optional[torch.Tensor] = None,
                    out_dtype: Optional[torch.dtype] = None, stream: Optional[int] = None) -> torch.Tensor:
    """silu(lhs . W1) * (lhs . W3) in one pass over lhs: the gated half of the SwiGLU
    feed-forward (crates/burn_boogu/src/model/feed_forward.rs:32-36).  Both weights must share
    layout, block and shape; the output dtype defaults to float32 (the reference's lhs dtype)."""
    for w in (w1, w3):
        if not isinstance(w, Q4Weight):
            raise _lib.Unsupported(_lib.ERR_UNSUPPORTED, "q_matmul_swiglu accelerates packed-Q4 weights only")
        if w.block not in SUPPORTED_BLOCKS:
            raise _lib.Unsupported(_lib.ERR_UNSUPPORTED, f"Q4 block {w.block} is not supported")
    if (w1.layout, w1.block, w1.shape) != (w3.layout, w3.block, w3.shape):
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "the two gated projections must share layout, block and shape")
    if lhs.dtype not in _DTYPE_CODE:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"lhs dtype {lhs.dtype} is not supported")
    if not lhs.is_cuda:
        raise ValueError("lhs must be a GPU tensor")
    K, N = w1.K, w1.N
    if lhs.shape[-1] != K:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                   f"lhs width {lhs.shape[-1]} does not match weight input {K}")
    lead = lhs.shape[:-1]
    x = lhs.reshape(-1, K)
    if x.stride(-1) != 1 or (x.shape[0] > 1 and x.stride(0) < K):
        x = x.contiguous()
    M = x.shape[0]
    ldx = x.stride(0) if M > 1 else K
    odt = out_dtype or (out.dtype if out is not None else torch.float32)
    if out is None:
        out = torch.empty((M, N), dtype=odt, device=lhs.device)
    elif out.dtype != odt or out.numel() != M * N or not out.is_contiguous():
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "out must be a contiguous [M, N] tensor")
    s = torch.cuda.current_stream(lhs.device).cuda_stream if stream is None else stream
    _lib.check(_lib.load().biq_q4_linear_swiglu(
        s, x.data_ptr(), _DTYPE_CODE[x.dtype], M, K, ldx, w1.words.data_ptr(), w1.scales.data_ptr(),
        w3.words.data_ptr(), w3.scales.data_ptr(), w1.layout, w1.block, N, out.data_ptr(),
        _DTYPE_CODE[odt]))
    return out.reshape(*lead, N)


@dataclass
class LuminaFeedForward:
    """SwiGLU feed-forward (crates/burn_boogu/src/model/feed_forward.rs:5-37): bias-free
    linear_1 / linear_3 (width -> inner) and linear_2 (inner -> width), all packed Q4 [K, N]."""
    linear_1: Linear
    linear_2: Linear
    linear_3: Linear

    def forward(self, x: torch.Tensor, hidden_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """linear_2(silu(linear_1(x)) * linear_3(x)); the gated hidden state is produced by one
        fused pass (f32 by default, as the reference; `hidden_dtype` may narrow it)."""
        for lin in (self.linear_1, self.linear_3):
            if lin.weight.layout != _lib.Q4_KN_AXIS1 or lin.bias is not None:
                raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                           "the feed-forward's gated projections are bias-free [K, N] weights")
        gated = q_matmul_swiglu(x, self.linear_1.weight, self.linear_3.weight, out_dtype=hidden_dtype)
        return linear_forward(self.linear_2, gated)
