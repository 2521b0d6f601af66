"""Flash attention on libbiq's HIP kernel, behind the reference's AttentionKernel seam.

Mirrors crates/burn_boogu/src/model/attention.rs:47-135 (``AttentionKernel``: ``execute``,
``execute_gqa``, ``execute_gqa_with_qk_norm_rope``, ``SPLIT_DOUBLE_STREAM_SHARED_PROJECTION``)
and Burn's attention op (patches/burn-cubecl-0.21.0/src/ops/module.rs:342-367).  All arithmetic
runs in libbiq; a missing library raises.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

ctypes_i64 = ctypes.c_int64

_DTYPE_CODE = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16,
               torch.bfloat16: _lib.DTYPE_BF16}

DEFAULT_QUERY_CHUNK_SIZE = 128
PORTABLE_ATTENTION_MINIMUM_IMAGE_QUERY_PARTITIONS = 4


def effective_portable_query_chunk_size(query_len: int, requested: int) -> int:
    """attention.rs:36-45: cap a requested portable tile so image-scale queries stay partitioned."""
    if requested <= 0:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention query chunk must be non-zero")
    if query_len <= 0:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention query sequence must be non-empty")
    if query_len <= DEFAULT_QUERY_CHUNK_SIZE:
        return min(requested, query_len)
    cap = -(-query_len // PORTABLE_ATTENTION_MINIMUM_IMAGE_QUERY_PARTITIONS)
    return min(requested, max(cap, DEFAULT_QUERY_CHUNK_SIZE))


def _strides_bhsd(t: torch.Tensor, name: str):
    if t.dim() != 4:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"attention {name} must be rank 4")
    if t.stride(3) != 1:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"attention {name} head width must be contiguous")
    return _lib.strides3((t.stride(0), t.stride(1), t.stride(2)))


def check_cu_seqlens(cu_seqlens, seq_len: int) -> None:
    """Host-side validation of a segment table (libbiq's biq_check_cu_seqlens): starts at 0,
    strictly ascending, ends at `seq_len`.  Raises InvalidArgument otherwise."""
    import numpy as np
    cu = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int64))
    if cu.ndim != 1 or cu.size < 2:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "cu_seqlens must list at least one segment")
    if cu.min() < -2**31 or cu.max() >= 2**31:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "cu_seqlens values must fit int32")
    cu32 = cu.astype(np.int32)
    _lib.check(_lib.load().biq_check_cu_seqlens(cu32.ctypes.data, cu32.size - 1, int(seq_len)))


def frame_ranges_to_cu_seqlens(frame_ranges, seq_len: int):
    """Qwen vision frame ranges [(start, end), ...] (crates/burn_qwen3_vl/src/vision.rs:319-386)
    -> int32 segment table, validated on the host (frames tile [0, seq_len) in order)."""
    import numpy as np
    r = np.ascontiguousarray(np.asarray(frame_ranges, dtype=np.int64).reshape(-1, 2))
    cu = np.zeros(r.shape[0] + 1, np.int32)
    _lib.check(_lib.load().biq_frame_ranges_to_cu_seqlens(r.ctypes.data, r.shape[0], int(seq_len),
                                                          cu.ctypes.data))
    return cu


def _device_cu(cu_seqlens, seq_len: int, device) -> torch.Tensor:
    """A host segment table is validated and copied; a device int32 table is used as given (the
    kernel clamps every bound it reads)."""
    if isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.is_cuda:
        if cu_seqlens.dtype != torch.int32:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "cu_seqlens must be int32")
        return cu_seqlens.contiguous()
    host = cu_seqlens.cpu().numpy() if isinstance(cu_seqlens, torch.Tensor) else cu_seqlens
    check_cu_seqlens(host, seq_len)
    import numpy as np
    return torch.from_numpy(np.asarray(host, dtype=np.int32)).to(device)


def attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *,
              is_causal: bool = False, scale: Optional[float] = None,
              cu_seqlens=None, key_mask: Optional[torch.Tensor] = None,
              key_mask_mode: int = _lib.KEY_MASK_VALID, out: Optional[torch.Tensor] = None,
              out_dtype: Optional[torch.dtype] = None, stream: Optional[int] = None) -> torch.Tensor:
    """softmax(Q K^T * scale) V over [B, H, S, D] views (any batch/head/seq strides, D
    contiguous).  K/V may carry fewer heads (GQA: query head h reads h / (Hq / Hkv)).
    ``cu_seqlens`` (int32 [nseg + 1]; a host table is validated first) adds the block-diagonal
    segment mask of a packed sequence; ``is_causal`` masks key j > query i; ``key_mask``
    ([B, Skv] bool/uint8 on the GPU) masks keys per batch, read by ``key_mask_mode``
    (KEY_MASK_VALID: True = attend; KEY_MASK_VALID_FILL_MEAN: also rows with no visible key get
    mean(V), Qwen's -1e30 fill; KEY_MASK_MASKED: True = masked).  Default scale 1/sqrt(D);
    default output dtype is the input dtype."""
    for name, t in (("query", query), ("key", key), ("value", value)):
        if not t.is_cuda:
            raise ValueError(f"attention {name} must be a GPU tensor")
    if not (query.dtype == key.dtype == value.dtype) or query.dtype not in _DTYPE_CODE:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention Q/K/V must share an F32/F16/BF16 dtype")
    B, Hq, Sq, D = query.shape
    Bk, Hkv, Skv, Dk = key.shape
    Bv, Hv, Sv, Dv = value.shape
    if Bk != B or Bv != B:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention query/key batch mismatch")
    if Hv != Hkv:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention key/value head mismatch")
    if Sv != Skv:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention key/value length mismatch")
    if Dk != D or Dv != D:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention query/key/value width mismatch")
    odt = out_dtype or (out.dtype if out is not None else query.dtype)
    if out is None:
        out = torch.empty((B, Hq, Sq, D), dtype=odt, device=query.device)
    elif tuple(out.shape) != (B, Hq, Sq, D) or out.dtype != odt:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention out has the wrong shape or dtype")
    cu_ptr, nseg = None, 0
    if cu_seqlens is not None:
        cu_seqlens = _device_cu(cu_seqlens, Sq, query.device)
        cu_ptr, nseg = cu_seqlens.data_ptr(), cu_seqlens.numel() - 1
    km_ptr, km_stride = None, 0
    if key_mask is not None:
        if not key_mask.is_cuda or key_mask.dtype not in (torch.bool, torch.uint8, torch.int8):
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "key_mask must be a bool/uint8 GPU tensor")
        if key_mask.dim() != 2 or key_mask.shape[1] != Skv or key_mask.shape[0] not in (1, B):
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "key_mask must be [B or 1, Skv]")
        if key_mask.stride(1) != 1:
            key_mask = key_mask.contiguous()
        km_ptr = key_mask.data_ptr()
        km_stride = key_mask.stride(0) if key_mask.shape[0] == B and B > 1 else 0
    s = torch.cuda.current_stream(query.device).cuda_stream if stream is None else stream
    _lib.check(_lib.load().biq_attention(
        s, query.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr(),
        _DTYPE_CODE[query.dtype], _DTYPE_CODE[odt], B, Hq, Hkv, Sq, Skv, D,
        _strides_bhsd(query, "query"), _strides_bhsd(key, "key"), _strides_bhsd(value, "value"),
        _strides_bhsd(out, "output"), float(scale) if scale else 0.0, int(bool(is_causal)),
        cu_ptr, nseg, km_ptr, km_stride, int(key_mask_mode)))
    return out


def burn_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   mask: Optional[torch.Tensor] = None, attn_bias: Optional[torch.Tensor] = None, *,
                   is_causal: bool = False, scale: Optional[float] = None,
                   softcap: Optional[float] = None, stream: Optional[int] = None) -> torch.Tensor:
    """Burn's ModuleOps::attention (patches/burn-cubecl-0.21.0/src/ops/module.rs:342-367) on
    libbiq: [B, H, S, D] tensors of one dtype, output in that dtype.  `mask` is a bool tensor
    broadcastable to [B, H, Sq, Skv] with True = masked; only key-padding masks (broadcast over
    heads and queries) run, any other mask, an attn_bias or a softcap raises Unsupported."""
    B, Hq, Sq, D = query.shape
    Hkv, Skv = key.shape[1], key.shape[2]
    if not (query.dtype == key.dtype == value.dtype) or query.dtype not in _DTYPE_CODE:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention Q/K/V must share an F32/F16/BF16 dtype")
    out = torch.empty((B, Hq, Sq, D), dtype=query.dtype, device=query.device)
    m_ptr, m_str = None, None
    if mask is not None:
        if mask.dtype not in (torch.bool, torch.uint8) or not mask.is_cuda:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention mask must be a bool GPU tensor")
        m4 = mask
        while m4.dim() < 4:
            m4 = m4.unsqueeze(0)
        m4 = m4.expand(B, Hq, Sq, Skv)
        m_ptr = m4.data_ptr()
        m_str = (ctypes_i64 * 4)(*[int(x) for x in m4.stride()])
    s = torch.cuda.current_stream(query.device).cuda_stream if stream is None else stream
    _lib.check(_lib.load().biq_attention_burn(
        s, query.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr(),
        _DTYPE_CODE[query.dtype], B, Hq, Hkv, Sq, Skv, D, _strides_bhsd(query, "query"),
        _strides_bhsd(key, "key"), _strides_bhsd(value, "value"), _strides_bhsd(out, "output"),
        m_ptr, m_str, None if attn_bias is None else attn_bias.data_ptr(), int(bool(is_causal)),
        int(scale is not None), float(scale or 0.0), int(softcap is not None), float(softcap or 0.0)))
    return out


class AttentionKernel:
    """The reference's kernel seam (attention.rs:47-135), implemented on libbiq.

    ``execute``: Q, K, V [B, H, S, D] -> [B, H, Sq, D].
    ``execute_gqa``: token-major Q [B, S, Hq, D], K/V [B, S, Hkv, D] -> [B, S, Hq, D]; the
    head expansion is an index map inside the kernel, never a materialised repeat.
    The query chunk is validated like the reference's (non-zero) but does not change the result:
    every query tile of the kernel already sees the complete key/value sequence.
    """

    SPLIT_DOUBLE_STREAM_SHARED_PROJECTION = False

    @classmethod
    def execute(cls, query, key, value, query_chunk_size: int, **kw) -> torch.Tensor:
        if query_chunk_size <= 0:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention query chunk must be non-zero")
        if key.shape[1] != query.shape[1]:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention query/key head mismatch")
        return attention(query, key, value, **kw)

    @classmethod
    def execute_gqa(cls, query, key, value, query_chunk_size: int, **kw) -> torch.Tensor:
        if query_chunk_size <= 0:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "attention query chunk must be non-zero")
        B, S, Hq, D = query.shape
        _, Sk, Hkv, _ = key.shape
        if Hq % Hkv != 0:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                       "GQA query heads must be divisible by key/value heads")
        out_dtype = kw.pop("out_dtype", None) or query.dtype
        out = torch.empty((B, S, Hq, D), dtype=out_dtype, device=query.device)
        attention(query.permute(0, 2, 1, 3), key.permute(0, 2, 1, 3), value.permute(0, 2, 1, 3),
                  out=out.permute(0, 2, 1, 3), out_dtype=out_dtype, **kw)
        return out


class NativeQ4FlashAttention(AttentionKernel):
    """Drop-in for NativeF32ToF16PaddedBlackboxAttention<4, 1, 1> (attention.rs:220-230,406-497):
    F32 projections in, the HIP flash kernel (f16 matrix-core operands, f32 accumulation), F32 out,
    with the dual-stream shared projection split (SplitDoubleStreamSharedProjection)."""

    SPLIT_DOUBLE_STREAM_SHARED_PROJECTION = True


# ---------------------------------------------------------------------------------------------
# Q/K RMSNorm + RoPE preparation (the seam's third method)
# ---------------------------------------------------------------------------------------------

STRICT_F32 = "strict_f32"
F16_STORAGE_F32_ACCUM = "f16_storage_f32_accum"


class RmsNorm:
    """nn::RmsNorm parameters: gamma [D] and epsilon (crates/burn_boogu/src/model/norm.rs)."""

    def __init__(self, gamma: torch.Tensor, epsilon: float = 1e-5):
        self.gamma = gamma
        self.epsilon = float(epsilon)


def qk_norm_rope(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, norm_q: RmsNorm,
                 norm_k: RmsNorm, cos: torch.Tensor, sin: torch.Tensor,
                 out_dtype: torch.dtype = torch.float16, rope_layout: int = _lib.ROPE_INTERLEAVED,
                 stream: Optional[int] = None):
    """One fused HIP pass over token-major Q [B, S, Hq, D], K/V [B, S, Hkv, D]: RMSNorm (f32
    reduction, then in the input dtype) + RoPE on Q and K, cast of all three to ``out_dtype``.
    ROPE_INTERLEAVED: Boogu's fused prep (native_flash.rs:395-583); ROPE_HALF: Qwen's q/k norm +
    apply_text_rope (text.rs:112-125,407-440).  cos/sin: [1 or B, S, D].  Returns contiguous
    (q, k, v)."""
    B, S, Hq, D = query.shape
    _, Sk, Hkv, _ = key.shape
    if Sk != S or value.shape[1] != S:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                   "fused strict Q/K norm+RoPE preparation requires equal Q/K sequence lengths")
    if tuple(norm_q.gamma.shape) != (D,) or tuple(norm_k.gamma.shape) != (D,):
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "fused RMSNorm gamma width mismatch")
    if cos.dim() != 3 or tuple(cos.shape[1:]) != (S, D) or cos.shape != sin.shape:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "fused RoPE tables must be [1|B, S, D]")
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.stride(3) != 1:
            raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, f"fused {name} head width must be contiguous")
    if not (query.dtype == key.dtype == value.dtype) or query.dtype not in _DTYPE_CODE:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG, "fused Q/K/V dtype mismatch")
    gq = norm_q.gamma.to(torch.float32).contiguous()
    gk = norm_k.gamma.to(torch.float32).contiguous()
    cs = cos.to(torch.float32).contiguous()
    sn = sin.to(torch.float32).contiguous()
    qo = torch.empty((B, S, Hq, D), dtype=out_dtype, device=query.device)
    ko = torch.empty((B, S, Hkv, D), dtype=out_dtype, device=query.device)
    vo = torch.empty((B, S, Hkv, D), dtype=out_dtype, device=query.device)
    st = lambda t: _lib.strides3((t.stride(0), t.stride(1), t.stride(2)))
    s = torch.cuda.current_stream(query.device).cuda_stream if stream is None else stream
    _lib.check(_lib.load().biq_qk_norm_rope(
        s, query.data_ptr(), key.data_ptr(), value.data_ptr(), _DTYPE_CODE[query.dtype],
        B, S, Hq, Hkv, D, st(query), st(key), st(value), gq.data_ptr(), gk.data_ptr(),
        norm_q.epsilon, norm_k.epsilon, cs.data_ptr(), sn.data_ptr(), cs.shape[0], int(rope_layout),
        _DTYPE_CODE[out_dtype], qo.data_ptr(), ko.data_ptr(), vo.data_ptr()))
    return qo, ko, vo


def _execute_gqa_with_qk_norm_rope(cls, query, key, value, norm_q: RmsNorm, norm_k: RmsNorm,
                                   rope, query_chunk_size: int,
                                   rms_norm_policy: str = STRICT_F32,
                                   operand_dtype: torch.dtype = torch.float16,
                                   out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Normalise and rotate token-major Q/K, then grouped-query attention (attention.rs:107-134
    seam; the packed-Q4 route of attention.rs:447-496).  Requires strict-F32 RMSNorm and RoPE
    tables, as the reference's fused route asserts.  Output dtype defaults to the input dtype
    (F32 projections in, F32 out)."""
    if rms_norm_policy != STRICT_F32:
        raise _lib.Unsupported(_lib.ERR_UNSUPPORTED,
                               "packed-Q4 fused attention preparation requires strict-F32 RMSNorm")
    if rope is None:
        raise _lib.InvalidArgument(_lib.ERR_INVALID_ARG,
                                   "packed-Q4 fused attention preparation requires RoPE")
    cos, sin = rope
    q, k, v = qk_norm_rope(query, key, value, norm_q, norm_k, cos, sin, out_dtype=operand_dtype)
    return cls.execute_gqa(q, k, v, query_chunk_size, out_dtype=out_dtype or query.dtype)


AttentionKernel.execute_gqa_with_qk_norm_rope = classmethod(_execute_gqa_with_qk_norm_rope)
