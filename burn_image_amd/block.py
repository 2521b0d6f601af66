"""The modulated Boogu DiT block on libbiq: projections, attention, feed-forward and the fused
row-wise glue, composed as the reference composes them.

Mirrors crates/burn_boogu/src/model/block.rs:84-134 (SingleStreamBlock, modulated branch),
norm.rs:101-153 (RmsNormZero), attention.rs:700-833 (GqaAttention) and feed_forward.rs:5-37
(LuminaFeedForward).  Every product and reduction runs in a libbiq kernel; torch only holds the
buffers (and applies the one-row silu of the conditioning vector, norm.rs:147).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib
from .attention import NativeQ4FlashAttention, RmsNorm
from .linear import Linear, LuminaFeedForward, linear_forward

_DTYPE_CODE = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16,
               torch.bfloat16: _lib.DTYPE_BF16}


def block_glue(branch: torch.Tensor, *, residual: Optional[torch.Tensor] = None,
               branch_norm: Optional[RmsNorm] = None, gate: Optional[torch.Tensor] = None,
               residual_out: Optional[torch.Tensor] = None, next_norm: Optional[RmsNorm] = None,
               next_scale: Optional[torch.Tensor] = None, next_dtype: Optional[torch.dtype] = None,
               stream: Optional[int] = None) -> Optional[torch.Tensor]:
    """One fused glue pass over [B, S, W] rows (block.rs:91-111):
    r = residual + rmsnorm(branch) * tanh(gate) (or r = branch without a residual), written to
    `residual_out` (may be `residual`); with `next_dtype`, returns
    rmsnorm(r) * (1 + next_scale) in that dtype.  gate / next_scale are [B, W] rows."""
    if branch.dim() != 3:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "block glue works on [B, S, W] tokens")
    B, S, Wd = branch.shape
    for name, t in (("branch", branch), ("residual", residual), ("residual_out", residual_out)):
        if t is not None and (not t.is_contiguous() or tuple(t.shape) != (B, S, Wd)):
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"{name} must be a contiguous [B, S, W] tensor")
    for name, t in (("residual", residual), ("residual_out", residual_out)):
        if t is not None and t.dtype != torch.float32:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"{name} is the f32 residual stream")
    for name, t in (("gate", gate), ("next_scale", next_scale)):
        if t is not None and tuple(t.shape) != (B, Wd):
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"{name} must be [B, W]")
    f32 = lambda t: None if t is None else t.to(torch.float32).contiguous()  # noqa: E731
    g_b = f32(branch_norm.gamma) if branch_norm is not None else None
    g_n = f32(next_norm.gamma) if next_norm is not None else None
    gate_c, scale_c = f32(gate), f32(next_scale)
    nxt = None
    if next_dtype is not None:
        nxt = torch.empty((B, S, Wd), dtype=next_dtype, device=branch.device)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    s = torch.cuda.current_stream(branch.device).cuda_stream if stream is None else stream
    _lib.check(_lib.load().biq_block_glue(
        s, B * S, Wd, S, ptr(residual), branch.data_ptr(), _DTYPE_CODE[branch.dtype], ptr(g_b),
        branch_norm.epsilon if branch_norm is not None else 0.0, ptr(gate_c), ptr(residual_out),
        ptr(g_n), next_norm.epsilon if next_norm is not None else 0.0, ptr(scale_c), ptr(nxt),
        _DTYPE_CODE[next_dtype] if next_dtype is not None else 0))
    return nxt


@dataclass
class RmsNormZero:
    """Adaptive RMSNorm (norm.rs:101-153): `linear` maps silu(conditioning) [B, C] to the four
    [B, W] modulation rows (scale_msa, gate_msa, scale_mlp, gate_mlp); `norm` holds gamma/eps."""
    linear: Linear
    norm: RmsNorm

    def modulation(self, conditioning: torch.Tensor, width: int):
        mod = linear_forward(self.linear, torch.nn.functional.silu(conditioning.to(torch.float32)))
        return tuple(mod[:, i * width:(i + 1) * width] for i in range(4))


@dataclass
class GqaAttention:
    """attention.rs:700-833: bias-free to_q / to_k / to_v / to_out projections, per-head
    strict-F32 RMSNorm + RoPE and grouped-query flash attention."""
    to_q: Linear
    to_k: Linear
    to_v: Linear
    to_out: Linear
    norm_q: RmsNorm
    norm_k: RmsNorm
    heads: int
    kv_heads: int
    head_dim: int
    query_chunk_size: int = 8192

    def forward(self, query_tokens: torch.Tensor, key_value_tokens: torch.Tensor,
                rope: Tuple[torch.Tensor, torch.Tensor]) -> torch.Tensor:
        B, Sq, _ = query_tokens.shape
        Sk = key_value_tokens.shape[1]
        q = linear_forward(self.to_q, query_tokens).reshape(B, Sq, self.heads, self.head_dim)
        k = linear_forward(self.to_k, key_value_tokens).reshape(B, Sk, self.kv_heads, self.head_dim)
        v = linear_forward(self.to_v, key_value_tokens).reshape(B, Sk, self.kv_heads, self.head_dim)
        out = NativeQ4FlashAttention.execute_gqa_with_qk_norm_rope(
            q, k, v, self.norm_q, self.norm_k, rope, self.query_chunk_size)
        return linear_forward(self.to_out, out.reshape(B, Sq, self.heads * self.head_dim))


@dataclass
class SingleStreamBlock:
    """Modulated single-stream block (block.rs:84-111):
        normalized, gate_attn, scale_mlp, gate_mlp = norm1(tokens, conditioning)
        tokens = tokens + norm2(attn(normalized)) * tanh(gate_attn)
        tokens = tokens + ffn_norm2(ffn(ffn_norm1(tokens) * (1 + scale_mlp))) * tanh(gate_mlp)
    with the three glue steps fused into biq_block_glue passes.  `activation_dtype` is the dtype
    the projections read (f32 as the reference; bf16 halves their input traffic)."""
    norm1: RmsNormZero
    attn: GqaAttention
    norm2: RmsNorm
    ffn_norm1: RmsNorm
    ffn_norm2: RmsNorm
    feed_forward: LuminaFeedForward
    activation_dtype: torch.dtype = torch.float32

    def forward(self, tokens: torch.Tensor, rope: Tuple[torch.Tensor, torch.Tensor],
                conditioning: torch.Tensor) -> torch.Tensor:
        tokens = tokens.to(torch.float32).contiguous()
        width = tokens.shape[-1]
        scale_msa, gate_msa, scale_mlp, gate_mlp = self.norm1.modulation(conditioning, width)
        normalized = block_glue(tokens, next_norm=self.norm1.norm, next_scale=scale_msa,
                                next_dtype=self.activation_dtype)
        attended = self.attn.forward(normalized, normalized, rope).contiguous()
        tokens1 = torch.empty_like(tokens)
        mlp_in = block_glue(attended, residual=tokens, branch_norm=self.norm2, gate=gate_msa,
                            residual_out=tokens1, next_norm=self.ffn_norm1, next_scale=scale_mlp,
                            next_dtype=self.activation_dtype)
        mlp = self.feed_forward.forward(mlp_in).contiguous()
        out = torch.empty_like(tokens)
        block_glue(mlp, residual=tokens1, branch_norm=self.ffn_norm2, gate=gate_mlp, residual_out=out)
        return out
