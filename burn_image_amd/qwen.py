"""Qwen3-VL text attention on libbiq: the encoder-prefill consumer of the same projection and
attention kernels as the Boogu denoiser block.

Mirrors ``Qwen3VlTextAttention::forward`` (crates/burn_qwen3_vl/src/text.rs:103-192): packed-Q4
q/k/v projections over checkpoint [N, K] weights (qwen_linear_forward, linear.rs:107-140),
per-head q_norm / k_norm (Burn nn::RmsNorm) and rotate-half RoPE (apply_text_rope,
text.rs:407-440) in one fused pass, causal grouped-query attention whose key-padding
``attention_mask`` is OR-ed into the causal mask (text.rs:146-185; the KV heads are indexed, not
repeated as repeat_key_value does, text.rs:390-405) and the o_proj projection.  Every product,
reduction and mask runs in libbiq.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from .attention import RmsNorm, attention, qk_norm_rope
from .linear import Linear, qwen_linear_forward

DEFAULT_QUERY_CHUNK_SIZE = 128


@dataclass
class Qwen3VlTextAttention:
    """Causal GQA self attention of one Qwen3-VL text decoder layer.  Projections are Linear
    layers with Qwen-layout (Q4_NK_AXIS0) packed weights; q_norm / k_norm carry gamma [head_dim]
    and the config's rms_norm_eps.  ``query_chunk_size`` is validated like the reference's
    (clamped to >= 1, text.rs:99-101) and does not change the result: the kernel sees every key
    of every query row in one launch."""
    q_proj: Linear
    k_proj: Linear
    v_proj: Linear
    o_proj: Linear
    q_norm: RmsNorm
    k_norm: RmsNorm
    num_heads: int
    num_key_value_heads: int
    head_dim: int
    query_chunk_size: int = DEFAULT_QUERY_CHUNK_SIZE
    operand_dtype: torch.dtype = torch.float16

    def set_query_chunk_size(self, query_chunk_size: int) -> None:
        self.query_chunk_size = max(int(query_chunk_size), 1)

    def forward(self, hidden_states: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                attention_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """hidden_states [B, S, hidden]; cos / sin [1 or B, S, head_dim] (rotate-half tables);
        attention_mask [B, S] bool (True = valid token) or None.  Rows of a left-padded prompt
        that see no valid key take the mean of V over every key, as the reference's
        mask_fill(-1e30) softmax gives them (text.rs:177-182).  Returns [B, S, hidden] f32."""
        Bn, S, _ = hidden_states.shape
        H, Hkv, D = self.num_heads, self.num_key_value_heads, self.head_dim
        if H % Hkv != 0:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                       "GQA query heads must be divisible by key/value heads")
        q = qwen_linear_forward(self.q_proj, hidden_states).view(Bn, S, H, D)
        k = qwen_linear_forward(self.k_proj, hidden_states).view(Bn, S, Hkv, D)
        v = qwen_linear_forward(self.v_proj, hidden_states).view(Bn, S, Hkv, D)
        if cos.dim() == 2:
            cos, sin = cos[None], sin[None]
        qn, kn, vn = qk_norm_rope(q, k, v, self.q_norm, self.k_norm, cos, sin,
                                  out_dtype=self.operand_dtype, rope_layout=_lib.ROPE_HALF)
        out = torch.empty((Bn, S, H, D), dtype=torch.float32, device=hidden_states.device)
        key_mask = None
        if attention_mask is not None:
            if tuple(attention_mask.shape) != (Bn, S):
                raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention_mask must be [B, S]")
            key_mask = attention_mask.to(torch.bool).contiguous()
        attention(qn.permute(0, 2, 1, 3), kn.permute(0, 2, 1, 3), vn.permute(0, 2, 1, 3), is_causal=True,
                  key_mask=key_mask, key_mask_mode=_lib.KEY_MASK_VALID_FILL_MEAN,
                  out=out.permute(0, 2, 1, 3), out_dtype=torch.float32)
        return qwen_linear_forward(self.o_proj, out.view(Bn, S, H * D))
