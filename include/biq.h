/*
 * biq.h - C ABI of the MI355X (gfx950) denoiser attention block library (libbiq.so).
 *
 * The library replaces the Burn/CubeCL operators below burn_boogu's attention and linear seams
 * with hand-written HIP kernels: packed signed-Q4 projection GEMMs (f32 block scales), Q4S
 * quantisation / dequantisation, and exact flash attention (non-causal, causal, segment-masked,
 * GQA).  Every entry point:
 *   - takes plain device pointers, element counts and an optional HIP stream (`stream` is a
 *     hipStream_t; NULL selects the default stream) and is asynchronous on that stream unless
 *     stated otherwise;
 *   - returns BIQ_OK or an error status and never falls back to another implementation; the
 *     message of the last failure on the calling thread is available from biq_last_error();
 *   - never frees caller memory; the caller owns every input and output buffer.
 * Calls are reentrant and thread-safe.  Reference citations are file:line in mosure/burn_image.
 */
#ifndef BIQ_H
#define BIQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  INVALID_ARG mirrors the reference's fail-closed shape/dtype/divisibility asserts
 * (crates/burn_boogu/src/model/native_flash.rs:1713-1727,1913-1955; attention.rs:78-90) and the
 * quantizers' `Err` results (crates/burn_boogu/src/artifacts.rs:7213-7236,7306-7340). */
#define BIQ_OK 0
#define BIQ_ERR_INVALID_ARG 1
#define BIQ_ERR_UNSUPPORTED 2
#define BIQ_ERR_HIP 3

/* Element types of activations and outputs. */
#define BIQ_DTYPE_F32 0
#define BIQ_DTYPE_F16 1
#define BIQ_DTYPE_BF16 2

/* Packed signed-Q4 layouts (eight signed nibbles per little-endian u32, lane l at bits 4l..4l+3).
 * BIQ_Q4_NK_AXIS0: Qwen `PackedU32(0)`, block [blk]: weight [N, K] (checkpoint [out, in]); words
 *   [N, K/8], scales f32 [N, K/blk]; the GEMM consumes W^T (artifacts.rs:7203-7288,518;
 *   crates/burn_qwen3_vl/src/linear.rs:58-62).
 * BIQ_Q4_KN_AXIS1: Boogu `PackedU32(1)`, block [blk, 1]: weight [K, N] ([input, output]); words
 *   [K/8, N], word (kw, n) holds k = 8*kw + l; scales f32 [K/blk, N] (artifacts.rs:7296-7388). */
#define BIQ_Q4_NK_AXIS0 0
#define BIQ_Q4_KN_AXIS1 1

/* Library version string, e.g. "biq 0.1.0 gfx950". */
const char *biq_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *biq_last_error(void);

/* Storage block of a Q4S weight of logical shape [rows, cols] for `layout`, or 0 if the
 * reference would not store it as Q4S.  Replaces q4s_storage_block_and_axis
 * (crates/burn_boogu/src/artifacts.rs:513-525): Qwen ([N, K], layout 0) needs K % 128 == 0 and
 * uses 128; Boogu ([K, N], layout 1) needs N % 8 == 0 and uses the largest of 128, 64, 32, 16, 8
 * dividing K.  Host-only; no GPU needed. */
int biq_q4_storage_block(int layout, int64_t rows, int64_t cols);

/* Tensor-inventory dtype string of that storage contract, written to buf (NUL-terminated):
 * "q4s-block{b}-f32-packed-axis0" or "q4s-block{b}x1-f32-packed-axis1" (artifacts.rs:527-536).
 * Returns BIQ_ERR_INVALID_ARG if the shape has no Q4S contract or buf is too small. Host-only. */
int biq_q4_stored_dtype(int layout, int64_t rows, int64_t cols, char *buf, size_t buf_len);

/* Host-only: layout, block and byte split of a Q4S tensor payload -- the importer's single byte
 * buffer of packed words followed by f32 scales (crates/burn_boogu/src/artifacts.rs:7276-7283,
 * 7364-7377) -- for a logical [rows, cols] weight stored as `stored_dtype`
 * ("q4s-block{b}-f32-packed-axis0" or "q4s-block{b}x1-f32-packed-axis1").  Checks the string
 * and payload_bytes against the storage contract of the shape (biq_q4_stored_dtype; the
 * importer's size contract, crates/burn_boogu/src/bin/boogu_import.rs:1693-1719) and returns
 * BIQ_ERR_INVALID_ARG on any mismatch.  The words are the first words_bytes of the payload and
 * the scales the next scales_bytes (4-byte aligned whenever the payload is): pass payload and
 * payload + words_bytes to biq_q4_linear without copying. */
int biq_q4_payload_layout(const char *stored_dtype, int64_t rows, int64_t cols,
                          int64_t payload_bytes, int *layout, int *block, int64_t *words_bytes,
                          int64_t *scales_bytes);

/* Quantise an f32 weight on the GPU, byte-for-byte as the reference importer does.
 * layout BIQ_Q4_KN_AXIS1: w is [K, N] -> quantize_row_layout_q4s_block_up_to128_f32
 *   (artifacts.rs:7296-7388), block = biq_q4_storage_block(1, K, N).
 * layout BIQ_Q4_NK_AXIS0: w is [N, K] -> quantize_q4s_block128_f32 (artifacts.rs:7203-7288),
 *   block 128 along K.
 * words/scales receive the layout's buffers.  Synchronous: it waits for the stream so that a
 * non-finite input can be reported as BIQ_ERR_INVALID_ARG, as the reference returns Err. */
int biq_q4_quantize(void *stream, const float *w, int layout, int64_t K, int64_t N,
                    uint32_t *words, float *scales);

/* Dequantise to f32, bit-exact `f32(q) * scale` (artifacts.rs:10434-10440; the GPU dequant
 * call patches/burn-cubecl-0.21.0/src/kernel/quantization/dequantize.rs:6-34).  Output is the
 * tensor's logical shape: [K, N] for BIQ_Q4_KN_AXIS1, [N, K] for BIQ_Q4_NK_AXIS0. */
int biq_q4_dequant_f32(void *stream, const uint32_t *words, const float *scales, int layout,
                       int block, int64_t K, int64_t N, float *w);

/* y[M, N] = x[M, K] . W (+ bias[N]) with W the packed-Q4 weight in `layout`.
 * Replaces QTensorOps::q_matmul's packed route (patches/burn-cubecl-0.21.0/src/ops/qtensor.rs:
 * 303-368: f32 lhs, Q4S symmetric, f32 scales, PackedU32(0|1), block in {8,16,32,64,128}) and
 * therefore linear_forward (crates/burn_boogu/src/model/linear.rs:14-37) and qwen_linear_forward
 * (crates/burn_qwen3_vl/src/linear.rs:107-140).  x: row-major with row stride ldx elements
 * (ldx >= K), dtype x_dtype in {F32, F16, BF16}; y: row-major, row stride N, y_dtype in
 * {F32, F16, BF16}; bias may be NULL.  Requirements: K % 8 == 0, K % block == 0, N % 8 == 0,
 * block in {8, 16, 32, 64, 128}.  Arithmetic: the signed nibbles are exact in f16, activations
 * enter the matrix cores as f16 (f32 inputs as an exact-to-2^-22 f16 hi+lo pair), products
 * accumulate in f32 per K-block, and each block sum is scaled by its f32 scale in f32.
 * Scratch: calls with M <= 16 and an f32 output, and calls whose last tiles are split along K,
 * use the library's grow-only scratch for (device, stream); it can only grow outside stream
 * capture (BIQ_ERR_UNSUPPORTED there: make the same call once before capturing).  Results are
 * deterministic; rows of a K-split tile are summed in another order than rows of a whole tile. */
int biq_q4_linear(void *stream, const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                  const uint32_t *words, const float *scales, int layout, int block, int64_t N,
                  const float *bias, void *y, int y_dtype);

/* Releases the grow-only scratch the library keeps for (current device, stream) -- used by the
 * small-M route and by K-split GEMM tails -- including buffers an earlier growth replaced.  It
 * waits for the stream first.  Without this call the buffers live until the process ends (one
 * set per stream that ever ran such a call); a runtime that creates and destroys streams should
 * call it before destroying one.  The caller must ensure no captured graph still names the
 * buffers (graphs record their addresses).  A later call on the stream allocates afresh. */
int biq_release_stream_workspace(void *stream);

/* Size of the static scratch biq_q4_linear_noalloc uses on each GPU (32 MiB). */
#define BIQ_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* biq_q4_linear for callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  No counterpart in the reference.  Same
 * arguments, kernels, work split and (bitwise) results as biq_q4_linear, but it calls no
 * hipMalloc / hipFree or other allocating routine: the partial sums of K-split tail tiles and of
 * the small-M route live in a static device array of BIQ_NOALLOC_SCRATCH_BYTES that each GPU
 * running the library holds until the process ends.  A call whose work split needs more scratch
 * returns BIQ_ERR_UNSUPPORTED before any GPU work (the message gives both sizes).  The array is
 * shared by every call on that GPU and keeps the last call's contents (each call writes every
 * element it reads): calls that overlap on one GPU -- on different streams, or from threads
 * without ordering -- race. */
int biq_q4_linear_noalloc(void *stream, const void *x, int x_dtype, int64_t M, int64_t K,
                          int64_t ldx, const uint32_t *words, const float *scales, int layout,
                          int block, int64_t N, const float *bias, void *y, int y_dtype);

/* y[M, N] = silu(x . W1) * (x . W3), the gated half of the SwiGLU feed-forward
 * `silu(linear_1(x)) * linear_3(x)` (crates/burn_boogu/src/model/feed_forward.rs:32-36), whose
 * output feeds linear_2.  One pass over x computes both projections (same layout, block, K and N;
 * bias-free, as the reference's FFN) and the gate in f32 before the y_dtype store; silu(a) =
 * a / (1 + e^-a).  Arguments and requirements as biq_q4_linear, per weight. */
int biq_q4_linear_swiglu(void *stream, const void *x, int x_dtype, int64_t M, int64_t K,
                         int64_t ldx, const uint32_t *words1, const float *scales1,
                         const uint32_t *words3, const float *scales3, int layout, int block,
                         int64_t N, void *y, int y_dtype);

/* Row-wise glue of the modulated DiT blocks (crates/burn_boogu/src/model/block.rs:91-111 and the
 * dual-stream block, block.rs:248-350), one pass per glue step over rows of `width`
 * (b = row / rows_per_batch selects the per-batch gate / scale / shift rows):
 *   u    = branch * (1 + branch_scale[b]) + branch_shift[b]            (NULL: factor 1 / shift 0)
 *   r    = x + (u / rms(u)) * branch_gamma * tanh(gate[b])             when x != NULL
 *   r    = u                                                           when x == NULL
 *   x_out = r (f32; may alias x), when x_out != NULL
 *   next = ((r / rms(r)) * next_gamma) * (1 + next_scale[b]) in next_dtype, when next_out != NULL
 * rms(v) = sqrt(mean(v^2) + eps) in f32 (rms_normalized, crates/burn_boogu/src/model/norm.rs:
 * 28-35; nn::RmsNorm's gamma product; RmsNormZero's modulation, norm.rs:144-152).  A NULL gamma
 * is all ones, a NULL gate drops the tanh factor (the unmodulated block, block.rs:113-131) and a
 * NULL next_scale is all zeros.  The branch modulation is the dual-stream block's MLP input,
 * base * (scale_mlp + 1) + shift_mlp (block.rs:322-324).  branch may be F32, F16 or BF16;
 * next_out must not alias x, x_out or branch. */
int biq_block_glue(void *stream, int64_t rows, int64_t width, int64_t rows_per_batch,
                   const float *x, const void *branch, int branch_dtype, const float *branch_scale,
                   const float *branch_shift, const float *branch_gamma, float branch_eps,
                   const float *gate, float *x_out, const float *next_gamma, float next_eps,
                   const float *next_scale, void *next_out, int next_dtype);

/* y[i] = silu(x[i]) = x / (1 + e^-x) in f32 for n elements: the conditioning rows entering
 * RmsNormZero's modulation projection (crates/burn_boogu/src/model/norm.rs:145). */
int biq_silu(void *stream, int64_t n, const void *x, int x_dtype, float *y);

/* Key-mask modes of biq_attention (the byte mask is [B, Skv], one byte per key).
 * BIQ_KEY_MASK_VALID: a nonzero byte marks a key that may be attended (Qwen's `attention_mask`,
 *   crates/burn_qwen3_vl/src/text.rs:163-170); a query row left with no visible key is zero.
 * BIQ_KEY_MASK_VALID_FILL_MEAN: as VALID, but a row with no visible key gets the mean of V over
 *   all Skv keys -- what the reference's `mask_fill(-1e30)` then softmax gives for such a row
 *   (text.rs:177-182: every score equal, uniform weights), e.g. the left-padding rows of a batch.
 * BIQ_KEY_MASK_MASKED: a nonzero byte masks its key out (Burn's bool attention mask polarity);
 *   a row with no visible key is zero. */
#define BIQ_KEY_MASK_VALID 0
#define BIQ_KEY_MASK_VALID_FILL_MEAN 1
#define BIQ_KEY_MASK_MASKED 2

/* Exact attention O = softmax(Q K^T * scale + mask) V, the operator behind
 * AttentionKernel::execute / execute_gqa (crates/burn_boogu/src/model/attention.rs:47-105), the
 * padded-blackbox flash kernel (native_flash.rs:1006-1090), plus Qwen's causal text attention with
 * its key-padding mask (crates/burn_qwen3_vl/src/text.rs:103-192) and per-frame vision attention
 * (vision.rs:319-388).
 *   q: [B, Hq, Sq, D] addressed by q_strides = {batch, head, seq} element strides (D contiguous),
 *   k, v: [B, Hkv, Skv, D] with their strides, o: [B, Hq, Sq, D] with o_strides.  Token-major
 *   [B, S, H, D] tensors are passed with strides {S*H*D, D, H*D}.
 *   in_dtype in {F32, F16, BF16} for q, k and v; out_dtype in {F32, F16, BF16}.
 *   Hq % Hkv == 0; query head h reads key/value head h / (Hq / Hkv).
 *   D in {64, 128} or any multiple of 8 below 128 (computed in a zero-extended 128-wide tile,
 *   e.g. the released D = 120 without a padded copy).
 *   scale: softmax scale; scale <= 0 selects 1/sqrt(D).
 *   causal != 0: key j is masked for query i when j > i (requires Sq == Skv).
 *   cu_seqlens (device int32[nseg + 1]) or NULL: block-diagonal segment mask over a packed
 *   sequence (requires Sq == Skv).  A valid table starts at 0, ascends strictly and ends at Sq
 *   (biq_check_cu_seqlens checks a host copy); the kernel clamps every bound it reads to [0, Skv],
 *   so a malformed table never reads outside K/V, but its rows are then unspecified.
 *   key_mask (device bytes; row b at key_mask + b * key_mask_stride, Skv bytes each; stride 0
 *   broadcasts one row over the batch) or NULL, interpreted by key_mask_mode (BIQ_KEY_MASK_*);
 *   combines with causal and segment masks.
 * Arithmetic: Q K^T on the matrix cores in bf16 (bf16 inputs) or f16 (f16 and f32 inputs, as the
 * reference's F32->F16 bridge, attention.rs:406-497), f32 online softmax, P and V in f16 on the
 * matrix cores, f32 accumulation. */
int biq_attention(void *stream, const void *q, const void *k, const void *v, void *o,
                  int in_dtype, int out_dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                  int64_t Skv, int64_t D, const int64_t *q_strides, const int64_t *k_strides,
                  const int64_t *v_strides, const int64_t *o_strides, float scale, int causal,
                  const int32_t *cu_seqlens, int64_t nseg, const uint8_t *key_mask,
                  int64_t key_mask_stride, int key_mask_mode);

/* Burn's attention op, ModuleOps::attention(q, k, v, mask: Option<Bool>, attn_bias,
 * AttentionModuleOptions { is_causal, scale, softcap })
 * (patches/burn-cubecl-0.21.0/src/ops/module.rs:342-367), over the same kernel.  Tensors and
 * strides as biq_attention, with q, k, v and o all of `dtype`.
 *   mask: NULL, or a bool tensor [B, H, Sq, Skv] (true = masked out) given by its element strides
 *   mask_strides[4] (0 = broadcast).  Only a key-padding mask -- broadcast over heads and query
 *   rows (strides[1] == strides[2] == 0), keys contiguous -- maps onto the kernel; any other mask
 *   returns BIQ_ERR_UNSUPPORTED.  A query row with every key masked is zero.
 *   attn_bias != NULL or has_softcap != 0: BIQ_ERR_UNSUPPORTED (the reference sends these to
 *   Burn's dense fallback; this library has none).
 *   has_scale != 0: softmax scale `scale` (> 0); otherwise 1/sqrt(D).
 *   is_causal: key j > query i masked (requires Sq == Skv).
 * The reference's callers pass no mask, bias or softcap (native_flash.rs:905-912,2745-2820). */
int biq_attention_burn(void *stream, const void *q, const void *k, const void *v, void *o,
                       int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Skv,
                       int64_t D, const int64_t *q_strides, const int64_t *k_strides,
                       const int64_t *v_strides, const int64_t *o_strides, const uint8_t *mask,
                       const int64_t *mask_strides, const void *attn_bias, int is_causal,
                       int has_scale, float scale, int has_softcap, float softcap);

/* Host-only check of a segment table: cu[0] == 0, cu strictly ascending, cu[nseg] == S
 * (BIQ_ERR_INVALID_ARG otherwise, with the reason in biq_last_error()). */
int biq_check_cu_seqlens(const int32_t *cu, int64_t nseg, int64_t S);

/* Host-only: Qwen vision frame ranges `&[(usize, usize)]` (crates/burn_qwen3_vl/src/vision.rs:
 * 319-386), given as int64 pairs ranges[2 f], ranges[2 f + 1], -> the segment table
 * cu[nframes + 1] biq_attention takes.  The frames must tile [0, S) in order, each non-empty
 * (the reference's per-frame loop concatenates the frame outputs in order). */
int biq_frame_ranges_to_cu_seqlens(const int64_t *ranges, int64_t nframes, int64_t S, int32_t *cu);

/* RoPE layouts of biq_qk_norm_rope: Boogu's interleaved pairs (2p, 2p + 1), rotated = (-x1, x0)
 * (crates/burn_boogu/src/model/attention.rs:916-928), and Qwen's rotate-half pairs (i, i + D/2),
 * rotated = cat(-x[D/2:], x[:D/2]) (crates/burn_qwen3_vl/src/text.rs:407-440). */
#define BIQ_ROPE_INTERLEAVED 0
#define BIQ_ROPE_HALF 1

/* Fused attention-input preparation: RMSNorm of Q and K rows, RoPE on both, and the cast of Q,
 * K and V to the attention operand type, in one pass.
 * With BIQ_ROPE_INTERLEAVED it replaces prepare_gqa_strict_norm_rope_padded_qkv_kernel and its
 * host function (crates/burn_boogu/src/model/native_flash.rs:395-583,747-817,2205-2332; the
 * FusedStrictF32ToF16 policy of crates/burn_boogu/src/config.rs:177-192) for an attention kernel
 * that takes the unpadded head width and unexpanded KV heads: it writes no 120 -> 128 padding,
 * no sqrt(128/120) Q prescale and no GQA copies.  With BIQ_ROPE_HALF it is Qwen's q_norm / k_norm
 * (Burn nn::RmsNorm) followed by apply_text_rope (crates/burn_qwen3_vl/src/text.rs:112-125,
 * 407-440).
 *   q: [B, S, Hq, D], k, v: [B, S, Hkv, D] token-major, addressed by {batch, seq, head} element
 *   strides (D contiguous), in_dtype F in {F32, F16, BF16};
 *   q_gamma, k_gamma: f32 [D]; cos, sin: f32 [rope_batch, S, D] contiguous, rope_batch 1 or B;
 *   q_out, k_out, v_out: contiguous [B, S, H, D] of out_dtype in {F16, BF16}.
 * Per row: rms = sqrt(sum(x^2) / D + eps) in f32, cast to F; n = x / rms * gamma in F (gamma
 * cast to F); interleaved: y = n * cos + rotated * sin in F (tables cast to F), rotate-half: in
 * f32 then cast to F; then one rounding to out_dtype.  For F32 inputs every step is f32.
 * D even and at most 128 (divisible by 4 for BIQ_ROPE_HALF); eps finite and positive;
 * Hq % Hkv == 0. */
int biq_qk_norm_rope(void *stream, const void *q, const void *k, const void *v, int in_dtype,
                     int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                     const int64_t *q_strides, const int64_t *k_strides,
                     const int64_t *v_strides, const float *q_gamma, const float *k_gamma,
                     float q_eps, float k_eps, const float *cos, const float *sin,
                     int64_t rope_batch, int rope_layout, int out_dtype, void *q_out, void *k_out,
                     void *v_out);

/* Fused self-attention input: the packed-Q4 projection of the token rows onto q | k | v heads
 * followed by the preparation biq_qk_norm_rope does (BIQ_ROPE_INTERLEAVED, f32 projections), in
 * one launch whose epilogue normalises, rotates and casts the projection tile in registers: the
 * f32 projection is never written.  Replaces, for GqaAttention's self attention with one packed
 * [K, (Hq + 2 Hkv) * D] weight (crates/burn_boogu/src/model/attention.rs:700-833: to_q / to_k /
 * to_v, then prepare_gqa_strict_norm_rope_padded_qkv_kernel, native_flash.rs:395-583), the pair
 * biq_q4_linear + biq_qk_norm_rope.  x: [B * S, K] rows (row stride ldx) in F16 or BF16; the
 * weight in BIQ_Q4_KN_AXIS1 with block 32, 64 or 128; q_gamma / k_gamma [D] f32; cos / sin
 * [rope_batch, S, D] f32 (rope_batch 1 or B); outputs contiguous q_out [B, S, Hq, D], k_out /
 * v_out [B, S, Hkv, D] in out_dtype (F16 or BF16), or with head_major = 1 [B, H, S, D] (the
 * attention kernel reads each head's keys as one contiguous run).  Gamma, tables and outputs
 * 16-byte aligned; each output and table below 2 GiB.  Arithmetic: the projection as biq_q4_linear
 * (every tile over the whole K, running block-scale rescale), then per row and head the
 * preparation's f32 steps; only the f32 sum of squares is added in another order, so results
 * equal the two-call path within one rounding of the output type.  D must be 128 and the other
 * requirements as biq_q4_linear, else BIQ_ERR_UNSUPPORTED (callers then make the two calls).
 * No scratch. */
int biq_q4_linear_qk_norm_rope(void *stream, const void *x, int x_dtype, int64_t B, int64_t S,
                               int64_t K, int64_t ldx, const uint32_t *words, const float *scales,
                               int block, int64_t Hq, int64_t Hkv, int64_t D,
                               const float *q_gamma, const float *k_gamma, float q_eps,
                               float k_eps, const float *cos, const float *sin,
                               int64_t rope_batch, int out_dtype, int head_major, void *q_out,
                               void *k_out, void *v_out);

#ifdef __cplusplus
}
#endif

#endif /* BIQ_H */
