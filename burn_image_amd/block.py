"""The modulated Boogu DiT block on libbiq: projections, attention, feed-forward and the fused
row-wise glue, composed as the reference composes them.

Mirrors crates/burn_boogu/src/model/block.rs:84-134 (SingleStreamBlock, modulated branch) and
:138-350 (DoubleStreamBlock), norm.rs:101-153 (RmsNormZero), attention.rs:499-833
(DoubleStreamAttention, GqaAttention) and feed_forward.rs:5-37 (LuminaFeedForward).  Every
product, reduction and activation runs in a libbiq kernel; torch only allocates the buffers.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib
from .attention import NativeQ4FlashAttention, RmsNorm, attention
from .linear import Linear, LuminaFeedForward, linear_forward

_DTYPE_CODE = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16,
               torch.bfloat16: _lib.DTYPE_BF16}


def block_glue(branch: torch.Tensor, *, residual: Optional[torch.Tensor] = None,
               branch_norm: Optional[RmsNorm] = None, gate: Optional[torch.Tensor] = None,
               residual_out: Optional[torch.Tensor] = None, next_norm: Optional[RmsNorm] = None,
               next_scale: Optional[torch.Tensor] = None, next_dtype: Optional[torch.dtype] = None,
               branch_scale: Optional[torch.Tensor] = None, branch_shift: Optional[torch.Tensor] = None,
               stream: Optional[int] = None) -> Optional[torch.Tensor]:
    """One fused glue pass over [B, S, W] rows (block.rs:91-111, 248-350):
    u = branch * (1 + branch_scale) + branch_shift; r = residual + rmsnorm(u) * tanh(gate) (or
    r = u without a residual), written to `residual_out` (may be `residual`); with `next_dtype`,
    returns rmsnorm(r) * (1 + next_scale) in that dtype.  gate / scales / shift are [B, W] rows."""
    if branch.dim() != 3:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "block glue works on [B, S, W] tokens")
    B, S, Wd = branch.shape
    for name, t in (("branch", branch), ("residual", residual), ("residual_out", residual_out)):
        if t is not None and (not t.is_contiguous() or tuple(t.shape) != (B, S, Wd)):
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"{name} must be a contiguous [B, S, W] tensor")
    for name, t in (("residual", residual), ("residual_out", residual_out)):
        if t is not None and t.dtype != torch.float32:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"{name} is the f32 residual stream")
    for name, t in (("gate", gate), ("next_scale", next_scale), ("branch_scale", branch_scale),
                    ("branch_shift", branch_shift)):
        if t is not None and tuple(t.shape) != (B, Wd):
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"{name} must be [B, W]")
    f32 = lambda t: None if t is None else t.to(torch.float32).contiguous()  # noqa: E731
    g_b = f32(branch_norm.gamma) if branch_norm is not None else None
    g_n = f32(next_norm.gamma) if next_norm is not None else None
    gate_c, scale_c = f32(gate), f32(next_scale)
    bsc_c, bsh_c = f32(branch_scale), f32(branch_shift)
    nxt = None
    if next_dtype is not None:
        nxt = torch.empty((B, S, Wd), dtype=next_dtype, device=branch.device)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    s = torch.cuda.current_stream(branch.device).cuda_stream if stream is None else stream
    _lib.check(_lib.load().biq_block_glue(
        s, B * S, Wd, S, ptr(residual), branch.data_ptr(), _DTYPE_CODE[branch.dtype], ptr(bsc_c), ptr(bsh_c),
        ptr(g_b),
        branch_norm.epsilon if branch_norm is not None else 0.0, ptr(gate_c), ptr(residual_out),
        ptr(g_n), next_norm.epsilon if next_norm is not None else 0.0, ptr(scale_c), ptr(nxt),
        _DTYPE_CODE[next_dtype] if next_dtype is not None else 0))
    return nxt


def silu(x: torch.Tensor, stream: Optional[int] = None) -> torch.Tensor:
    """f32 silu(x) = x / (1 + e^-x) on the GPU (libbiq biq_silu)."""
    x = x.contiguous()
    y = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    s = torch.cuda.current_stream(x.device).cuda_stream if stream is None else stream
    _lib.check(_lib.load().biq_silu(s, x.numel(), x.data_ptr(), _DTYPE_CODE[x.dtype], y.data_ptr()))
    return y


def modulation_rows(linear: Linear, conditioning: torch.Tensor, width: int, parts: int = 4):
    """linear(silu(conditioning)) split into `parts` [B, width] views (norm.rs:144-151)."""
    mod = linear_forward(linear, silu(conditioning))
    return tuple(mod[:, i * width:(i + 1) * width] for i in range(parts))


@dataclass
class RmsNormZero:
    """Adaptive RMSNorm (norm.rs:101-153): `linear` maps silu(conditioning) [B, C] to the four
    [B, W] modulation rows (scale_msa, gate_msa, scale_mlp, gate_mlp); `norm` holds gamma/eps."""
    linear: Linear
    norm: RmsNorm

    def modulation(self, conditioning: torch.Tensor, width: int):
        """The four [B, W] rows of linear(silu(conditioning)) (norm.rs:144-151), silu in libbiq."""
        return tuple(t.contiguous() for t in
                     modulation_rows(self.linear, conditioning, width, 4))


def project_qkv_norm_rope(qkv: Linear, tokens: torch.Tensor, norm_q: RmsNorm, norm_k: RmsNorm,
                          rope: Tuple[torch.Tensor, torch.Tensor], heads: int, kv_heads: int,
                          head_dim: int, out_dtype: torch.dtype = torch.float16,
                          head_major: bool = False, stream: Optional[int] = None):
    """One libbiq launch for self attention's inputs (biq_q4_linear_qk_norm_rope): tokens
    [B, S, K] times the packed q | k | v weight, then strict-F32 RMSNorm + interleaved RoPE of the
    q and k heads and the cast of all three, from the projection tile in registers.  The same
    results as linear_forward(qkv) followed by qk_norm_rope (attention.rs:700-833 with the
    native_flash.rs:395-583 preparation) within one rounding of ``out_dtype``.  Returns contiguous
    q [B, S, heads, D], k / v [B, S, kv_heads, D] ([B, heads, S, D] / [B, kv_heads, S, D] with
    ``head_major``); raises Unsupported where the fused launch does not apply (head width other
    than 128, f32 tokens, blocks below 32, a bias)."""
    w = qkv.weight
    if qkv.bias is not None:
        raise _lib.Unsupported(_lib.ERR_UNSUPPORTED, "fused q/k/v projection takes a bias-free weight")
    if w.layout != _lib.Q4_KN_AXIS1:
        raise _lib.Unsupported(_lib.ERR_UNSUPPORTED, "fused q/k/v projection takes the [K/8, N] layout")
    if tokens.dim() != 3 or tokens.dtype not in _DTYPE_CODE:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "fused q/k/v projection takes [B, S, K] tokens")
    B, S, K = tokens.shape
    if w.K != K or w.N != (heads + 2 * kv_heads) * head_dim:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "fused q/k/v weight shape mismatch")
    cos, sin = rope
    if cos.dim() != 3 or tuple(cos.shape[1:]) != (S, head_dim) or cos.shape != sin.shape:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "fused RoPE tables must be [1|B, S, D]")
    x = tokens.reshape(B * S, K)
    if x.stride(-1) != 1 or (x.shape[0] > 1 and x.stride(0) < K):
        x = x.contiguous()
    ldx = x.stride(0) if x.shape[0] > 1 else K
    gq = norm_q.gamma.to(torch.float32).contiguous()
    gk = norm_k.gamma.to(torch.float32).contiguous()
    cs = cos.to(torch.float32).contiguous()
    sn = sin.to(torch.float32).contiguous()
    shape = (lambda h: (B, h, S, head_dim)) if head_major else (lambda h: (B, S, h, head_dim))
    q = torch.empty(shape(heads), dtype=out_dtype, device=tokens.device)
    k = torch.empty(shape(kv_heads), dtype=out_dtype, device=tokens.device)
    v = torch.empty(shape(kv_heads), dtype=out_dtype, device=tokens.device)
    st = torch.cuda.current_stream(tokens.device).cuda_stream if stream is None else stream
    _lib.check(_lib.load().biq_q4_linear_qk_norm_rope(
        st, x.data_ptr(), _DTYPE_CODE[x.dtype], B, S, K, ldx, w.words.data_ptr(), w.scales.data_ptr(),
        w.block, heads, kv_heads, head_dim, gq.data_ptr(), gk.data_ptr(), norm_q.epsilon,
        norm_k.epsilon, cs.data_ptr(), sn.data_ptr(), cs.shape[0], _DTYPE_CODE[out_dtype],
        int(head_major), q.data_ptr(), k.data_ptr(), v.data_ptr()))
    return q, k, v


def _fused_qkv_applies(qkv: Linear, tokens: torch.Tensor, head_dim: int) -> bool:
    """The conditions under which biq_q4_linear_qk_norm_rope accepts the call."""
    w = qkv.weight
    return (qkv.bias is None and w.layout == _lib.Q4_KN_AXIS1 and w.block >= 32 and head_dim == 128
            and tokens.dtype in (torch.float16, torch.bfloat16) and tokens.dim() == 3)


@dataclass
class GqaAttention:
    """attention.rs:700-833: bias-free to_q / to_k / to_v / to_out projections, per-head
    strict-F32 RMSNorm + RoPE and grouped-query flash attention.  to_q / to_k / to_v may be None
    when the packed `qkv` weight is given (self attention only)."""
    to_q: Optional[Linear]
    to_k: Optional[Linear]
    to_v: Optional[Linear]
    to_out: Linear
    norm_q: RmsNorm
    norm_k: RmsNorm
    heads: int
    kv_heads: int
    head_dim: int
    query_chunk_size: int = 8192
    # Optional packed [K, (heads + 2 kv_heads) * head_dim] weight holding to_q | to_k | to_v
    # column-wise: self attention then runs one projection GEMM and hands the prep kernel strided
    # Q / K / V views of its output (the same products as the three projections).
    qkv: Optional[Linear] = None

    def forward(self, query_tokens: torch.Tensor, key_value_tokens: torch.Tensor,
                rope: Tuple[torch.Tensor, torch.Tensor],
                out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """to_out(attention(norm+RoPE(q), norm+RoPE(k), v)); `out_dtype` is the dtype of the
        attention output that feeds to_out (f32 by default, as the reference)."""
        B, Sq, _ = query_tokens.shape
        Sk = key_value_tokens.shape[1]
        H, Hkv, D = self.heads, self.kv_heads, self.head_dim
        if (self.qkv is not None and query_tokens is key_value_tokens and rope is not None
                and _fused_qkv_applies(self.qkv, query_tokens, D)):
            # projection and Q/K preparation in one launch (the f32 projection is never stored);
            # head-major operands: each head's keys are one contiguous run for the attention
            # kernel (attention alone 2.5-4.5% faster than on token-major views at 4608 tokens;
            # the whole block within noise of it)
            q, k, v = project_qkv_norm_rope(self.qkv, query_tokens, self.norm_q, self.norm_k, rope,
                                            H, Hkv, D, head_major=True)
            if self.query_chunk_size <= 0:
                raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention query chunk must be non-zero")
            odt = out_dtype or torch.float32
            out = torch.empty((B, Sq, H, D), dtype=odt, device=q.device)
            attention(q, k, v, out=out.permute(0, 2, 1, 3), out_dtype=odt)
            return linear_forward(self.to_out, out.reshape(B, Sq, self.heads * self.head_dim))
        if self.qkv is not None and query_tokens is key_value_tokens:
            fused = linear_forward(self.qkv, query_tokens).view(B, Sq, H + 2 * Hkv, D)
            q, k, v = fused[:, :, :H], fused[:, :, H:H + Hkv], fused[:, :, H + Hkv:]
        else:
            q = linear_forward(self.to_q, query_tokens).reshape(B, Sq, H, D)
            k = linear_forward(self.to_k, key_value_tokens).reshape(B, Sk, Hkv, D)
            v = linear_forward(self.to_v, key_value_tokens).reshape(B, Sk, Hkv, D)
        out = NativeQ4FlashAttention.execute_gqa_with_qk_norm_rope(
            q, k, v, self.norm_q, self.norm_k, rope, self.query_chunk_size,
            out_dtype=out_dtype or torch.float32)
        return linear_forward(self.to_out, out.reshape(B, Sq, self.heads * self.head_dim))


@dataclass
class SingleStreamBlock:
    """Modulated single-stream block (block.rs:84-111):
        normalized, gate_attn, scale_mlp, gate_mlp = norm1(tokens, conditioning)
        tokens = tokens + norm2(attn(normalized)) * tanh(gate_attn)
        tokens = tokens + ffn_norm2(ffn(ffn_norm1(tokens) * (1 + scale_mlp))) * tanh(gate_mlp)
    with the three glue steps fused into biq_block_glue passes.  `activation_dtype` is the dtype
    the projections read -- the normalised tokens, the attention output and the FFN's gated
    hidden state (f32 as the reference; bf16 halves their traffic and keeps the projections on
    single-pass 16-bit matrix-core operands)."""
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
        attended = self.attn.forward(normalized, normalized, rope, out_dtype=self.activation_dtype).contiguous()
        tokens1 = torch.empty_like(tokens)
        mlp_in = block_glue(attended, residual=tokens, branch_norm=self.norm2, gate=gate_msa,
                            residual_out=tokens1, next_norm=self.ffn_norm1, next_scale=scale_mlp,
                            next_dtype=self.activation_dtype)
        mlp = self.feed_forward.forward(mlp_in, hidden_dtype=self.activation_dtype).contiguous()
        out = torch.empty_like(tokens)
        block_glue(mlp, residual=tokens1, branch_norm=self.ffn_norm2, gate=gate_mlp, residual_out=out)
        return out


# ---------------------------------------------------------------------------------------------
# dual-stream attention and block (the released model's leading layers)
# ---------------------------------------------------------------------------------------------

def _project_rows_into(lin: Linear, x: torch.Tensor, out: torch.Tensor, row0: int) -> None:
    """out[b, row0:row0 + S_x] = linear(x[b]) for every batch element, written in place (the
    reference's Tensor::cat along tokens, attention.rs:646-668, without a concatenation copy)."""
    Bn, Sx, _ = x.shape
    N = out.shape[-1]
    if Bn == 1 or out.shape[1] == Sx:
        dst = out[:, row0:row0 + Sx]
        if dst.is_contiguous():
            linear_forward(lin, x, out=dst.view(Bn * Sx, N))
            return
    for b in range(Bn):
        linear_forward(lin, x[b], out=out[b, row0:row0 + Sx])


def _rows(x: torch.Tensor, row0: int, n: int):
    """[B, n, W] token range of x as GEMM inputs: one strided view when B == 1, else per batch."""
    return [x[b, row0:row0 + n] for b in range(x.shape[0])]


@dataclass
class DoubleStreamAttention:
    """Joint instruction/image attention with per-stream projections (attention.rs:499-720):
    instruct_to_{q,k,v} and img_to_{q,k,v} project the two streams, the projections are joined
    along tokens as [instruction, image], normalised and rotated per head, attended jointly
    (grouped-query), split back, projected by instruct_out / img_out and finally by the shared
    to_out -- per stream (split) or jointly, as the kernel's SPLIT_DOUBLE_STREAM_SHARED_PROJECTION
    says (project_shared_output, attention.rs:700-720).  Returns (image, instruction)."""
    img_to_q: Linear
    img_to_k: Linear
    img_to_v: Linear
    instruct_to_q: Linear
    instruct_to_k: Linear
    instruct_to_v: Linear
    img_out: Linear
    instruct_out: Linear
    to_out: Linear
    norm_q: RmsNorm
    norm_k: RmsNorm
    heads: int
    kv_heads: int
    head_dim: int
    query_chunk_size: int = 8192
    kernel: type = NativeQ4FlashAttention

    def forward(self, image: torch.Tensor, instruction: torch.Tensor,
                rope: Tuple[torch.Tensor, torch.Tensor]):
        Bn, Si, _ = image.shape
        St = instruction.shape[1]
        S = St + Si
        dev = image.device
        q = torch.empty((Bn, S, self.heads * self.head_dim), dtype=torch.float32, device=dev)
        k = torch.empty((Bn, S, self.kv_heads * self.head_dim), dtype=torch.float32, device=dev)
        v = torch.empty_like(k)
        for dst, lin_t, lin_i in ((q, self.instruct_to_q, self.img_to_q), (k, self.instruct_to_k, self.img_to_k),
                                  (v, self.instruct_to_v, self.img_to_v)):
            _project_rows_into(lin_t, instruction, dst, 0)
            _project_rows_into(lin_i, image, dst, St)
        attended = self.kernel.execute_gqa_with_qk_norm_rope(
            q.view(Bn, S, self.heads, self.head_dim), k.view(Bn, S, self.kv_heads, self.head_dim),
            v.view(Bn, S, self.kv_heads, self.head_dim), self.norm_q, self.norm_k, rope,
            self.query_chunk_size).reshape(Bn, S, self.heads * self.head_dim)
        width = self.img_out.weight.N
        instr = torch.empty((Bn, St, width), dtype=torch.float32, device=dev)
        img = torch.empty((Bn, Si, width), dtype=torch.float32, device=dev)
        for b, rows in enumerate(_rows(attended, 0, St)):
            linear_forward(self.instruct_out, rows, out=instr[b])
        for b, rows in enumerate(_rows(attended, St, Si)):
            linear_forward(self.img_out, rows, out=img[b])
        return self.project_shared_output(instr, img, self.kernel.SPLIT_DOUBLE_STREAM_SHARED_PROJECTION)

    def project_shared_output(self, instruction: torch.Tensor, image: torch.Tensor, split_streams: bool):
        """to_out per stream (split) or on the token-joined streams; both return (image,
        instruction) and are equal, to_out being row-wise (attention.rs:700-720)."""
        if split_streams:
            return linear_forward(self.to_out, image), linear_forward(self.to_out, instruction)
        Bn, St, W = instruction.shape
        Si = image.shape[1]
        joined = torch.empty((Bn, St + Si, W), dtype=instruction.dtype, device=instruction.device)
        joined[:, :St].copy_(instruction)
        joined[:, St:].copy_(image)
        merged = linear_forward(self.to_out, joined)
        return merged[:, St:], merged[:, :St]


@dataclass
class DoubleStreamBlock:
    """The leading dual-stream block (block.rs:138-350) on libbiq kernels.  Image and
    instruction keep separate residual streams: joint attention over [instruction, image],
    image-only self attention, and a feed-forward per stream whose input is the first-norm base
    modulated by (1 + scale_mlp) plus a shift (the second adaptive norm's gate slot).  The three
    image adaptive norms share one RMS reduction of the image tokens (as do the two instruction
    ones); every residual update is one biq_block_glue pass."""
    joint_attn: DoubleStreamAttention
    image_self_attn: GqaAttention
    image_ffn: LuminaFeedForward
    instruction_ffn: LuminaFeedForward
    image_norm1: RmsNormZero
    image_norm2: RmsNormZero
    image_norm3: RmsNormZero
    instruction_norm1: RmsNormZero
    instruction_norm2: RmsNormZero
    image_attn_norm: RmsNorm
    image_self_norm: RmsNorm
    image_ffn_norm1: RmsNorm
    image_ffn_norm2: RmsNorm
    instruction_attn_norm: RmsNorm
    instruction_ffn_norm1: RmsNorm
    instruction_ffn_norm2: RmsNorm
    activation_dtype: torch.dtype = torch.float32

    def forward(self, image: torch.Tensor, instruction: torch.Tensor,
                image_rope: Tuple[torch.Tensor, torch.Tensor], joint_rope: Tuple[torch.Tensor, torch.Tensor],
                conditioning: torch.Tensor):
        for a, b in ((self.image_norm1, self.image_norm2), (self.image_norm1, self.image_norm3),
                     (self.instruction_norm1, self.instruction_norm2)):
            if a.norm.epsilon != b.norm.epsilon:
                raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                           "shared RMS normalization requires equal epsilons")
        image = image.to(torch.float32).contiguous()
        instruction = instruction.to(torch.float32).contiguous()
        W = image.shape[-1]
        adt = self.activation_dtype

        def adaptive(norm: RmsNormZero, tokens: torch.Tensor, dtype: torch.dtype):
            # forward_from_rms_normalized (norm.rs:138-152) on rms_normalized(tokens)
            scale, g1, g2, g3 = (t.contiguous() for t in modulation_rows(norm.linear, conditioning, W, 4))
            base = block_glue(tokens, next_norm=norm.norm, next_scale=scale, next_dtype=dtype)
            return base, g1, g2, g3

        img_joint, img_gate_attn, img_scale_mlp, img_gate_mlp = adaptive(self.image_norm1, image, adt)
        img_mlp_base, img_shift_mlp, _, _ = adaptive(self.image_norm2, image, torch.float32)
        img_self, img_gate_self, _, _ = adaptive(self.image_norm3, image, adt)
        ins_joint, ins_gate_attn, ins_scale_mlp, ins_gate_mlp = adaptive(self.instruction_norm1, instruction, adt)
        ins_mlp_base, ins_shift_mlp, _, _ = adaptive(self.instruction_norm2, instruction, torch.float32)

        img_attn, ins_attn = self.joint_attn.forward(img_joint, ins_joint, joint_rope)
        img_self_out = self.image_self_attn.forward(img_self, img_self, image_rope)

        img1 = torch.empty_like(image)
        block_glue(img_attn.contiguous(), residual=image, branch_norm=self.image_attn_norm,
                   gate=img_gate_attn, residual_out=img1)
        block_glue(img_self_out.contiguous(), residual=img1, branch_norm=self.image_self_norm,
                   gate=img_gate_self, residual_out=img1)
        img_ffn_in = block_glue(img_mlp_base, branch_scale=img_scale_mlp, branch_shift=img_shift_mlp,
                                next_norm=self.image_ffn_norm1, next_dtype=adt)
        img_mlp = self.image_ffn.forward(img_ffn_in).contiguous()
        block_glue(img_mlp, residual=img1, branch_norm=self.image_ffn_norm2, gate=img_gate_mlp, residual_out=img1)

        ins1 = torch.empty_like(instruction)
        block_glue(ins_attn.contiguous(), residual=instruction, branch_norm=self.instruction_attn_norm,
                   gate=ins_gate_attn, residual_out=ins1)
        ins_ffn_in = block_glue(ins_mlp_base, branch_scale=ins_scale_mlp, branch_shift=ins_shift_mlp,
                                next_norm=self.instruction_ffn_norm1, next_dtype=adt)
        ins_mlp = self.instruction_ffn.forward(ins_ffn_in).contiguous()
        block_glue(ins_mlp, residual=ins1, branch_norm=self.instruction_ffn_norm2, gate=ins_gate_mlp,
                   residual_out=ins1)
        return img1, ins1
