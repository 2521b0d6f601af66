// Fused Q/K preparation before attention for gfx950: strict-F32 RMSNorm, Boogu interleaved-pair
// RoPE and the cast to the attention operand type, plus the V cast, in one HBM pass.
//
// Restates prepare_gqa_strict_norm_rope_padded_qkv_kernel (crates/burn_boogu/src/model/
// native_flash.rs:395-583; host side :2205-2332) for a kernel that consumes the unpadded head
// width and unexpanded KV heads directly: no 120 -> 128 zero padding, no sqrt(128/120) Q prescale
// and no GQA head copies are written (the attention kernel indexes KV heads and masks the width).
//
// Per row (one wave; lane p owns the pair d = 2p, 2p + 1):
//   rms = sqrt(sum_d x_d^2 / D + eps)            f32 (x widened to f32)
//   n_d = x_d / rms * gamma_d                    f32
//   y_2p   = n_2p * cos_2p - n_2p+1 * sin_2p     f32 (rotated = (-x1, x0), attention.rs:916-928)
//   y_2p+1 = n_2p+1 * cos_2p+1 + n_2p * sin_2p+1
//   out_d = cast(y_d)                            f16 or bf16 (round to nearest even)
#include <math.h>

#include "common.h"

namespace {

struct PrepArgs {
  const void *q, *k, *v;
  int64_t qs[3], ks[3], vs[3];  // batch, seq, head element strides (token-major [B, S, H, D])
  const float *q_gamma, *k_gamma, *cos, *sin;
  int64_t rope_bs;  // batch stride of the cos/sin tables (0 when shared by the batch)
  float q_eps, k_eps;
  int64_t B, S, Hq, Hkv, D;
  void *qo, *ko, *vo;  // contiguous [B, S, H, D]
};

template <typename T>
__device__ __forceinline__ float2 load_pair(const T *p);
template <>
__device__ __forceinline__ float2 load_pair<float>(const float *p) {
  return *reinterpret_cast<const float2 *>(p);
}
template <>
__device__ __forceinline__ float2 load_pair<f16_t>(const f16_t *p) {
  const uint32_t w = *reinterpret_cast<const uint32_t *>(p);
  return make_float2(biq::f16_bits_to_f32((uint16_t)(w & 0xffffu)),
                     biq::f16_bits_to_f32((uint16_t)(w >> 16)));
}
template <>
__device__ __forceinline__ float2 load_pair<bf16_t>(const bf16_t *p) {
  const uint32_t w = *reinterpret_cast<const uint32_t *>(p);
  return make_float2(biq::bf16_lo_to_f32(w), biq::bf16_hi_to_f32(w));
}

__device__ __forceinline__ uint32_t store_bits(float a, float b, bool bf16) {
  return bf16 ? (biq::f32_to_bf16_bits(a) | (biq::f32_to_bf16_bits(b) << 16)) : biq::pack_f16x2(a, b);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <typename InT>
__global__ void __launch_bounds__(256) qk_prep_kernel(PrepArgs p, int out_bf16) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t q_rows = p.B * p.S * p.Hq, kv_rows = p.B * p.S * p.Hkv;
  const int64_t pairs = p.D / 2;
  const bool active = lane < pairs;
  const int d = 2 * lane;

  int kind;      // 0 = Q, 1 = K, 2 = V
  int64_t r, H;
  if (row < q_rows) { kind = 0; r = row; H = p.Hq; }
  else if (row < q_rows + kv_rows) { kind = 1; r = row - q_rows; H = p.Hkv; }
  else if (row < q_rows + 2 * kv_rows) { kind = 2; r = row - q_rows - kv_rows; H = p.Hkv; }
  else return;
  const int64_t h = r % H, s = (r / H) % p.S, b = r / (H * p.S);
  const int64_t *st = kind == 0 ? p.qs : (kind == 1 ? p.ks : p.vs);
  const InT *src = reinterpret_cast<const InT *>(kind == 0 ? p.q : (kind == 1 ? p.k : p.v)) +
                   b * st[0] + s * st[1] + h * st[2];
  uint16_t *dst = reinterpret_cast<uint16_t *>(kind == 0 ? p.qo : (kind == 1 ? p.ko : p.vo)) +
                  r * p.D;

  float2 x = active ? load_pair<InT>(src + d) : make_float2(0.0f, 0.0f);
  if (kind == 2) {
    if (active) *reinterpret_cast<uint32_t *>(dst + d) = store_bits(x.x, x.y, out_bf16);
    return;
  }
  const float sum_sq = wave_sum(x.x * x.x + x.y * x.y);  // wave-uniform
  const float eps = kind == 0 ? p.q_eps : p.k_eps;
  const float rms = sqrtf(sum_sq / (float)p.D + eps);
  if (!active) return;
  const float *g = kind == 0 ? p.q_gamma : p.k_gamma;
  const float n0 = x.x / rms * g[d];
  const float n1 = x.y / rms * g[d + 1];
  const float *cs = p.cos + b * p.rope_bs + s * p.D;
  const float *sn = p.sin + b * p.rope_bs + s * p.D;
  const float y0 = n0 * cs[d] + (-n1) * sn[d];
  const float y1 = n1 * cs[d + 1] + n0 * sn[d + 1];
  *reinterpret_cast<uint32_t *>(dst + d) = store_bits(y0, y1, out_bf16);
}

}  // namespace

extern "C" int biq_qk_norm_rope(void *stream, const void *q, const void *k, const void *v,
                                int in_dtype, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                                int64_t D, const int64_t *q_strides, const int64_t *k_strides,
                                const int64_t *v_strides, const float *q_gamma,
                                const float *k_gamma, float q_eps, float k_eps, const float *cos,
                                const float *sin, int64_t rope_batch, int out_dtype, void *q_out,
                                void *k_out, void *v_out) {
  biq::clear_error();
  if (!q || !k || !v || !q_gamma || !k_gamma || !cos || !sin || !q_out || !k_out || !v_out ||
      !q_strides || !k_strides || !v_strides)
    return biq::fail(BIQ_ERR_INVALID_ARG, "null pointer argument");
  if (in_dtype != BIQ_DTYPE_F32 && in_dtype != BIQ_DTYPE_F16 && in_dtype != BIQ_DTYPE_BF16)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused strict Q/K norm+RoPE input must be F32, F16 or BF16");
  if (out_dtype != BIQ_DTYPE_F16 && out_dtype != BIQ_DTYPE_BF16)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused preparation output must be F16 or BF16");
  if (B <= 0 || S <= 0 || Hq <= 0 || Hkv <= 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused preparation requires non-empty Q/K/V");
  if (Hq % Hkv != 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "GQA query heads must be divisible by key/value heads");
  if (D <= 0 || D > 128 || D % 2 != 0)
    return biq::fail(BIQ_ERR_UNSUPPORTED, "fused preparation head width must be even and at most 128");
  if (rope_batch != 1 && rope_batch != B)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused RoPE batch must be one or match Q/K batch");
  if (!(q_eps > 0.0f) || !(k_eps > 0.0f) || q_eps == INFINITY || k_eps == INFINITY)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused RMSNorm epsilon must be finite and positive");
  const int esz = in_dtype == BIQ_DTYPE_F32 ? 4 : 2;
  const int64_t *st[3] = {q_strides, k_strides, v_strides};
  const void *ptr[3] = {q, k, v};
  for (int t = 0; t < 3; ++t) {
    if (reinterpret_cast<uintptr_t>(ptr[t]) & (2 * esz - 1))
      return biq::fail(BIQ_ERR_INVALID_ARG, "fused preparation inputs must be pair-aligned");
    for (int j = 0; j < 3; ++j)
      if ((st[t][j] * esz) % (2 * esz) != 0)
        return biq::fail(BIQ_ERR_INVALID_ARG, "fused preparation strides must be even");
  }
  PrepArgs a;
  a.q = q; a.k = k; a.v = v;
  for (int j = 0; j < 3; ++j) { a.qs[j] = q_strides[j]; a.ks[j] = k_strides[j]; a.vs[j] = v_strides[j]; }
  a.q_gamma = q_gamma; a.k_gamma = k_gamma; a.cos = cos; a.sin = sin;
  a.rope_bs = rope_batch == 1 ? 0 : S * D;
  a.q_eps = q_eps; a.k_eps = k_eps;
  a.B = B; a.S = S; a.Hq = Hq; a.Hkv = Hkv; a.D = D;
  a.qo = q_out; a.ko = k_out; a.vo = v_out;
  const int64_t rows = B * S * (Hq + 2 * Hkv);
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffff) return biq::fail(BIQ_ERR_UNSUPPORTED, "fused preparation grid too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int ob = out_dtype == BIQ_DTYPE_BF16;
  if (in_dtype == BIQ_DTYPE_F32)
    hipLaunchKernelGGL(qk_prep_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, s, a, ob);
  else if (in_dtype == BIQ_DTYPE_F16)
    hipLaunchKernelGGL(qk_prep_kernel<f16_t>, dim3((unsigned)blocks), dim3(256), 0, s, a, ob);
  else
    hipLaunchKernelGGL(qk_prep_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, s, a, ob);
  return biq::check_launch("qk norm rope");
}
