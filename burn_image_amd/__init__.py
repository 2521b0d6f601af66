"""MI355X-native (gfx950) denoiser attention block of burn_image: packed signed-Q4 projection
GEMMs and exact flash attention, as hand-written HIP kernels behind a C ABI (include/biq.h,
libbiq.so), with a host-side mirror of the reference's Burn-facing operator surface."""
from . import _lib
from ._lib import BiqError, InvalidArgument, Unsupported, version
from .attention import (F16_STORAGE_F32_ACCUM, STRICT_F32, AttentionKernel, burn_attention,
                        check_cu_seqlens, frame_ranges_to_cu_seqlens,
                        NativeQ4FlashAttention, RmsNorm, attention,
                        effective_portable_query_chunk_size, qk_norm_rope)
from .block import (DoubleStreamAttention, DoubleStreamBlock, GqaAttention, RmsNormZero,
                    SingleStreamBlock, block_glue, project_qkv_norm_rope)
from .linear import (Linear, LuminaFeedForward, linear_forward, q_matmul, q_matmul_swiglu,
                     qwen_linear_forward)
from .qwen import Qwen3VlTextAttention
from .q4 import (BOOGU_DENOISER, FLUX_VAE, QWEN3_VL, Q4Weight, from_packed, from_payload,
                 payload_layout, split_payload,
                 q4s_storage_block_and_axis, q4s_stored_dtype, quantize_q4s_block128_f32,
                 quantize_row_layout_q4s_block_up_to128_f32)

Q4_KN_AXIS1 = _lib.Q4_KN_AXIS1
Q4_NK_AXIS0 = _lib.Q4_NK_AXIS0

__all__ = [
    "AttentionKernel", "NativeQ4FlashAttention", "attention", "effective_portable_query_chunk_size",
    "burn_attention", "check_cu_seqlens", "frame_ranges_to_cu_seqlens",
    "RmsNorm", "qk_norm_rope", "STRICT_F32", "F16_STORAGE_F32_ACCUM",
    "Linear", "LuminaFeedForward", "linear_forward", "q_matmul", "q_matmul_swiglu",
    "qwen_linear_forward", "Q4Weight", "from_packed", "from_payload", "payload_layout", "split_payload",
    "q4s_storage_block_and_axis", "q4s_stored_dtype", "quantize_q4s_block128_f32",
    "quantize_row_layout_q4s_block_up_to128_f32", "BiqError", "InvalidArgument", "Unsupported",
    "block_glue", "project_qkv_norm_rope", "RmsNormZero", "GqaAttention", "SingleStreamBlock", "DoubleStreamAttention",
    "DoubleStreamBlock", "Qwen3VlTextAttention",
    "version", "BOOGU_DENOISER", "QWEN3_VL", "FLUX_VAE", "Q4_KN_AXIS1", "Q4_NK_AXIS0",
]
