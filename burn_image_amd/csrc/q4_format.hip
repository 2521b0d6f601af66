// Q4S weight format kernels for gfx950: GPU quantisers byte-identical to the reference importer
// and the bit-exact dequantiser.
//
// Format (both layouts): eight signed nibbles per little-endian u32, lane l at bits 4l..4l+3,
// stored as `(q as u8) & 0xf` (crates/burn_boogu/src/artifacts.rs:7273,7370); f32 scales.
#include <float.h>
#include <math.h>

#include "common.h"

namespace {

// Scale rule of both reference quantizers (artifacts.rs:7262-7270,7345-7353): alpha = max|w|,
// scale = f32::MIN_POSITIVE when alpha == 0 else alpha / 7 (IEEE division).
__device__ __forceinline__ float q4_scale(float alpha) {
  return alpha == 0.0f ? FLT_MIN : alpha / 7.0f;
}

// `(value * inverse).round().clamp(-7.0, 7.0) as i8` then `(q as u8) & 0x0f`.
__device__ __forceinline__ uint32_t q4_nibble(float value, float inverse) {
  float r = roundf(value * inverse);  // half away from zero, as f32::round
  r = fminf(fmaxf(r, -7.0f), 7.0f);
  return (uint32_t)((int)r) & 0xfu;
}

// Boogu row layout (artifacts.rs:7296-7388): one thread per (K-block b, column n).  It folds the
// block's max|w| over k, writes scale[b, n] and the blk/8 words (kw, n) of its column.  Reads and
// writes are coalesced along n.
__global__ void __launch_bounds__(256) q4_quantize_kn_kernel(const float *__restrict__ w, int64_t K,
                                                             int64_t N, int blk,
                                                             uint32_t *__restrict__ words,
                                                             float *__restrict__ scales,
                                                             int *__restrict__ nonfinite) {
  int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t b = blockIdx.y;
  if (n >= N) return;
  float alpha = 0.0f;
  bool bad = false;
  for (int64_t k = b * blk; k < (b + 1) * blk; ++k) {
    float v = w[k * N + n];
    bad |= !isfinite(v);
    alpha = fmaxf(alpha, fabsf(v));
  }
  if (bad) *nonfinite = 1;
  float scale = q4_scale(alpha);
  scales[b * N + n] = scale;
  float inverse = 1.0f / scale;
  for (int64_t kw = b * blk / 8; kw < (b + 1) * blk / 8; ++kw) {
    uint32_t word = 0;
#pragma unroll
    for (int lane = 0; lane < 8; ++lane)
      word |= q4_nibble(w[(8 * kw + lane) * N + n], inverse) << (4 * lane);
    words[kw * N + n] = word;
  }
}

// Qwen layout (artifacts.rs:7203-7288): one thread per contiguous 128-value chunk of the
// flattened [N, K] tensor; 16 words and one scale per chunk, in chunk order.
__global__ void __launch_bounds__(256) q4_quantize_nk_kernel(const float *__restrict__ values,
                                                             int64_t chunks,
                                                             uint32_t *__restrict__ words,
                                                             float *__restrict__ scales,
                                                             int *__restrict__ nonfinite) {
  int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= chunks) return;
  const float4 *src = reinterpret_cast<const float4 *>(values + c * 128);
  float alpha = 0.0f;
  bool bad = false;
#pragma unroll 4
  for (int i = 0; i < 32; ++i) {
    float4 v = src[i];
    bad |= !isfinite(v.x) || !isfinite(v.y) || !isfinite(v.z) || !isfinite(v.w);
    alpha = fmaxf(fmaxf(alpha, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
  }
  if (bad) *nonfinite = 1;
  float scale = q4_scale(alpha);
  scales[c] = scale;
  float inverse = 1.0f / scale;
  for (int wv = 0; wv < 16; ++wv) {
    float4 lo = src[2 * wv], hi = src[2 * wv + 1];
    uint32_t word = q4_nibble(lo.x, inverse) | (q4_nibble(lo.y, inverse) << 4) |
                    (q4_nibble(lo.z, inverse) << 8) | (q4_nibble(lo.w, inverse) << 12) |
                    (q4_nibble(hi.x, inverse) << 16) | (q4_nibble(hi.y, inverse) << 20) |
                    (q4_nibble(hi.z, inverse) << 24) | (q4_nibble(hi.w, inverse) << 28);
    words[c * 16 + wv] = word;
  }
}

__device__ __forceinline__ float q4_value(uint32_t word, int lane) {
  return (float)((int)(((word >> (4 * lane)) ^ 8u) & 15u) - 8);
}

// Dequantisation `f32(q) * scale` (artifacts.rs:10434-10440), one thread per packed word.
// Layout 1: word (kw, n) -> out[(8kw + l) * N + n]; layout 0: word (n, kw) -> out[n * K + 8kw + l].
__global__ void __launch_bounds__(256) q4_dequant_kernel(const uint32_t *__restrict__ words,
                                                         const float *__restrict__ scales,
                                                         int layout, int blk, int64_t K, int64_t N,
                                                         float *__restrict__ out) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t total = (K / 8) * N;
  if (t >= total) return;
  uint32_t word = words[t];
  if (layout == BIQ_Q4_KN_AXIS1) {
    int64_t kw = t / N, n = t % N;
    float s = scales[(8 * kw / blk) * N + n];
#pragma unroll
    for (int l = 0; l < 8; ++l) out[(8 * kw + l) * N + n] = q4_value(word, l) * s;
  } else {
    int64_t n = t / (K / 8), kw = t % (K / 8);
    float s = scales[n * (K / blk) + 8 * kw / blk];
    float4 a = make_float4(q4_value(word, 0) * s, q4_value(word, 1) * s, q4_value(word, 2) * s,
                           q4_value(word, 3) * s);
    float4 b = make_float4(q4_value(word, 4) * s, q4_value(word, 5) * s, q4_value(word, 6) * s,
                           q4_value(word, 7) * s);
    float4 *dst = reinterpret_cast<float4 *>(out + n * K + 8 * kw);
    dst[0] = a;
    dst[1] = b;
  }
}

}  // namespace

extern "C" int biq_q4_quantize(void *stream, const float *w, int layout, int64_t K, int64_t N,
                               uint32_t *words, float *scales) {
  biq::clear_error();
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!w || !words || !scales) return biq::fail(BIQ_ERR_INVALID_ARG, "null pointer argument");
  if (K <= 0 || N <= 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "Q4S quantization requires a non-empty matrix");
  int blk = 0;
  if (layout == BIQ_Q4_KN_AXIS1) {
    if (N % 8 != 0)
      return biq::fail(BIQ_ERR_INVALID_ARG, "runtime Q4S denoiser output width " +
                                                std::to_string(N) + " is not divisible by 8");
    blk = biq_q4_storage_block(BIQ_Q4_KN_AXIS1, K, N);
    if (blk == 0)
      return biq::fail(BIQ_ERR_INVALID_ARG, "runtime Q4S denoiser input width " +
                                                std::to_string(K) + " has no supported exact block");
  } else if (layout == BIQ_Q4_NK_AXIS0) {
    if (K % 128 != 0)
      return biq::fail(BIQ_ERR_INVALID_ARG, "Q4S innermost dimension " + std::to_string(K) +
                                                " is not divisible by 128");
    blk = 128;
  } else {
    return biq::fail(BIQ_ERR_INVALID_ARG, "unknown Q4 layout");
  }
  int *flag = nullptr;
  if (hipMalloc(&flag, sizeof(int)) != hipSuccess)
    return biq::fail(BIQ_ERR_HIP, "hipMalloc of the non-finite flag failed");
  int host_flag = 0;
  int rc = BIQ_OK;
  if (hipMemcpyAsync(flag, &host_flag, sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess) {
    rc = biq::fail(BIQ_ERR_HIP, "flag upload failed");
  } else {
    if (layout == BIQ_Q4_KN_AXIS1) {
      dim3 grid((unsigned)((N + 255) / 256), (unsigned)(K / blk));
      hipLaunchKernelGGL(q4_quantize_kn_kernel, grid, dim3(256), 0, s, w, K, N, blk, words, scales,
                         flag);
    } else {
      int64_t chunks = N * K / 128;
      hipLaunchKernelGGL(q4_quantize_nk_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256),
                         0, s, w, chunks, words, scales, flag);
    }
    rc = biq::check_launch("q4 quantize");
    if (rc == BIQ_OK) {
      if (hipMemcpyAsync(&host_flag, flag, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess ||
          hipStreamSynchronize(s) != hipSuccess)
        rc = biq::fail(BIQ_ERR_HIP, "quantize synchronisation failed");
      else if (host_flag)
        rc = biq::fail(BIQ_ERR_INVALID_ARG, "cannot quantize a non-finite checkpoint value");
    }
  }
  hipStreamSynchronize(s);
  hipFree(flag);
  return rc;
}

extern "C" int biq_q4_dequant_f32(void *stream, const uint32_t *words, const float *scales,
                                  int layout, int block, int64_t K, int64_t N, float *w) {
  biq::clear_error();
  if (!words || !scales || !w) return biq::fail(BIQ_ERR_INVALID_ARG, "null pointer argument");
  if (layout != BIQ_Q4_KN_AXIS1 && layout != BIQ_Q4_NK_AXIS0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "unknown Q4 layout");
  if (block != 8 && block != 16 && block != 32 && block != 64 && block != 128)
    return biq::fail(BIQ_ERR_INVALID_ARG, "Q4 block must be one of 8, 16, 32, 64, 128");
  if (K <= 0 || N <= 0 || K % 8 != 0 || K % block != 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "Q4 dequant requires K % 8 == 0 and K % block == 0");
  int64_t total = (K / 8) * N;
  hipLaunchKernelGGL(q4_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), words, scales, layout, block, K, N, w);
  return biq::check_launch("q4 dequant");
}
