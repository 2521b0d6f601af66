// Fused Q/K preparation before attention for gfx950: strict RMSNorm, RoPE and the cast to the
// attention operand type, plus the V cast, in one HBM pass.
//
// Restates prepare_gqa_strict_norm_rope_padded_qkv_kernel (crates/burn_boogu/src/model/
// native_flash.rs:395-583; host side :2205-2332) for a kernel that consumes the unpadded head
// width and unexpanded KV heads directly: no 120 -> 128 zero padding, no sqrt(128/120) Q prescale
// and no GQA head copies are written (the attention kernel indexes KV heads and masks the width).
// The rotate-half layout restates Qwen's q_norm / k_norm (Burn nn::RmsNorm) followed by
// apply_text_rope (crates/burn_qwen3_vl/src/text.rs:112-125,407-440).
//
// Per row (one wave holds PREP_ROWS consecutive rows; lane p owns the elements d = 2p, 2p + 1 of
// each), F = the input type, rnd = rounding
// to F (identity for F32 inputs):
//   rms   = sqrt(sum_d x_d^2 / D + eps)                  f32 (x widened to f32)
//   n_d   = rnd(rnd(x_d / rnd(rms)) * rnd(gamma_d))      in F: the f32 rms is cast to F first
//                                                        (native_flash.rs:446-449; norm.rs:28-35)
//   interleaved pairs (Boogu, attention.rs:916-928), rotated = (-n_2p+1, n_2p), in F:
//     y_d = rnd(rnd(n_d * rnd(cos_d)) + rnd(rot_d * rnd(sin_d)))
//   rotate-half (Qwen), rotated = cat(-n[h:], n[:h]), in f32 then cast to F:
//     y_d = rnd(n_d * cos_d + rot_d * sin_d)
//   out_d = cast(y_d)                                    f16 or bf16 (round to nearest even)
// Products of two 16-bit values and sums of two are exact in f32, so each f32 operation rounded
// to F is F's own rounded operation; the division may differ from a correctly rounded F division
// by one unit of F in rare midpoint cases.  Contraction into FMA is off for these steps.
#include <math.h>

#include <type_traits>

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

// Round an f32 value to the input type InT, returned as f32.
template <typename InT>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (sizeof(InT) == 4) {
    return v;
  } else if constexpr (std::is_same<InT, f16_t>::value) {
    return (float)(_Float16)v;
  } else {
    return biq::bitcast<float>(biq::f32_to_bf16_bits(v) << 16);
  }
}

__device__ __forceinline__ float2 load_pair(const float *p) {
  return *reinterpret_cast<const float2 *>(p);
}
// Two 16-bit elements (one 32-bit word, low half first) widened to f32.
template <typename T>
__device__ __forceinline__ float2 widen_pair(uint32_t w) {
  if constexpr (std::is_same<T, f16_t>::value)
    return make_float2(biq::f16_bits_to_f32((uint16_t)(w & 0xffffu)),
                       biq::f16_bits_to_f32((uint16_t)(w >> 16)));
  else
    return make_float2(biq::bf16_lo_to_f32(w), biq::bf16_hi_to_f32(w));
}

__device__ __forceinline__ uint32_t store_bits(float a, float b, bool bf16) {
  return bf16 ? biq::pack_bf16x2(a, b) : biq::pack_f16x2(a, b);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Position of a row of the fused index space (Q rows, then K rows, then V rows; each [B, S, H]
// with the head fastest), stepped along a wave's rows without a division.
struct RowLoc {
  int kind;  // 0 = Q, 1 = K, 2 = V, 3 = past the end
  int64_t r, h, s, b, H;
};

__device__ __forceinline__ RowLoc locate(const PrepArgs &p, int64_t row) {
  const int64_t q_rows = p.B * p.S * p.Hq, kv_rows = p.B * p.S * p.Hkv;
  RowLoc L;
  if (row < q_rows) { L.kind = 0; L.r = row; L.H = p.Hq; }
  else if (row < q_rows + kv_rows) { L.kind = 1; L.r = row - q_rows; L.H = p.Hkv; }
  else if (row < q_rows + 2 * kv_rows) { L.kind = 2; L.r = row - q_rows - kv_rows; L.H = p.Hkv; }
  else { L.kind = 3; L.r = 0; L.H = 1; }
  L.h = L.r % L.H;
  L.s = (L.r / L.H) % p.S;
  L.b = L.r / (L.H * p.S);
  return L;
}

__device__ __forceinline__ void advance(const PrepArgs &p, RowLoc &L) {
  if (L.kind == 3) return;
  ++L.r;
  if (++L.h < L.H) return;
  L.h = 0;
  if (++L.s < p.S) return;
  L.s = 0;
  if (++L.b < p.B) return;
  L = RowLoc{L.kind + 1, 0, 0, 0, 0, p.Hkv};  // next kind (K and V both have Hkv heads)
}

constexpr int PREP_ROWS = 8;  // rows per wave: their loads are all in flight before the first use

template <typename InT, bool HALF>
__global__ void __launch_bounds__(256) qk_prep_kernel(PrepArgs p, int out_bf16) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t pairs = p.D / 2;
  const bool active = lane < pairs;
  const int d = 2 * lane;

  RowLoc L0 = locate(p, wave * PREP_ROWS);
  RowLoc L = L0;
  // 16-bit inputs are loaded as raw words and widened after the loop: with the widening inside
  // the conditional load the compiler waited for each row's load in turn (8 serial round trips)
  constexpr bool WIDE = sizeof(InT) == 4;
  float2 x[PREP_ROWS];
  [[maybe_unused]] uint32_t w[PREP_ROWS];
#pragma unroll
  for (int i = 0; i < PREP_ROWS; ++i) {
    x[i] = make_float2(0.0f, 0.0f);
    if constexpr (!WIDE) w[i] = 0u;
    if (L.kind < 3) {
      const int64_t *st = L.kind == 0 ? p.qs : (L.kind == 1 ? p.ks : p.vs);
      const InT *src = reinterpret_cast<const InT *>(L.kind == 0 ? p.q : (L.kind == 1 ? p.k : p.v)) +
                       L.b * st[0] + L.s * st[1] + L.h * st[2];
      if (active) {
        if constexpr (WIDE) x[i] = load_pair(src + d);
        else w[i] = *reinterpret_cast<const uint32_t *>(src + d);
      }
    }
    advance(p, L);
  }
  if constexpr (!WIDE) {
#pragma unroll
    for (int i = 0; i < PREP_ROWS; ++i) x[i] = widen_pair<InT>(w[i]);
  }

  L = L0;
#pragma unroll
  for (int i = 0; i < PREP_ROWS; ++i, advance(p, L)) {
    if (L.kind == 3) break;
    uint16_t *dst = reinterpret_cast<uint16_t *>(L.kind == 0 ? p.qo : (L.kind == 1 ? p.ko : p.vo)) +
                    L.r * p.D;
    if (L.kind == 2) {
      if (active) *reinterpret_cast<uint32_t *>(dst + d) = store_bits(x[i].x, x[i].y, out_bf16);
      continue;
    }
    const float sum_sq = wave_sum(x[i].x * x[i].x + x[i].y * x[i].y);  // wave-uniform
    const float eps = L.kind == 0 ? p.q_eps : p.k_eps;
    const float2 dv = biq::rn_divisor(rnd<InT>(sqrtf(sum_sq / (float)p.D + eps)));
    const float *g = L.kind == 0 ? p.q_gamma : p.k_gamma;
    const float n0 = active ? rnd<InT>(rnd<InT>(biq::div_rn(x[i].x, dv.x, dv.y)) * rnd<InT>(g[d])) : 0.0f;
    const float n1 = active ? rnd<InT>(rnd<InT>(biq::div_rn(x[i].y, dv.x, dv.y)) * rnd<InT>(g[d + 1])) : 0.0f;
    const float *cs = p.cos + L.b * p.rope_bs + L.s * p.D;
    const float *sn = p.sin + L.b * p.rope_bs + L.s * p.D;
    float y0 = 0.0f, y1 = 0.0f;
    if constexpr (HALF) {
      // partner elements d + h (first half) or d - h (second half) sit in lane p +- h / 2; every
      // lane takes part in the shuffles (D % 4 == 0, host check)
      const int hp = (int)(p.D / 4);
      const int src = d < 2 * hp ? lane + hp : lane - hp;
      const float m0 = __shfl(n0, src), m1 = __shfl(n1, src);
      if (active) {
        const float r0 = d < 2 * hp ? -m0 : m0, r1 = d < 2 * hp ? -m1 : m1;
        y0 = rnd<InT>(n0 * cs[d] + r0 * sn[d]);
        y1 = rnd<InT>(n1 * cs[d + 1] + r1 * sn[d + 1]);
      }
    } else if (active) {
      y0 = rnd<InT>(rnd<InT>(n0 * rnd<InT>(cs[d])) + rnd<InT>(-n1 * rnd<InT>(sn[d])));
      y1 = rnd<InT>(rnd<InT>(n1 * rnd<InT>(cs[d + 1])) + rnd<InT>(n0 * rnd<InT>(sn[d + 1])));
    }
    if (active) *reinterpret_cast<uint32_t *>(dst + d) = store_bits(y0, y1, out_bf16);
  }
}

}  // namespace

extern "C" int biq_qk_norm_rope(void *stream, const void *q, const void *k, const void *v,
                                int in_dtype, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                                int64_t D, const int64_t *q_strides, const int64_t *k_strides,
                                const int64_t *v_strides, const float *q_gamma,
                                const float *k_gamma, float q_eps, float k_eps, const float *cos,
                                const float *sin, int64_t rope_batch, int rope_layout,
                                int out_dtype, void *q_out, void *k_out, void *v_out) {
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
  if (rope_layout != BIQ_ROPE_INTERLEAVED && rope_layout != BIQ_ROPE_HALF)
    return biq::fail(BIQ_ERR_INVALID_ARG, "unknown RoPE layout");
  if (rope_layout == BIQ_ROPE_HALF && D % 4 != 0)
    return biq::fail(BIQ_ERR_UNSUPPORTED, "rotate-half RoPE needs a head width divisible by 4");
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
  const int64_t blocks = (rows + 4 * PREP_ROWS - 1) / (4 * PREP_ROWS);
  if (blocks > 0x7fffffff) return biq::fail(BIQ_ERR_UNSUPPORTED, "fused preparation grid too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int ob = out_dtype == BIQ_DTYPE_BF16;
  const dim3 grid((unsigned)blocks);
#define BIQ_PREP(T)                                                                      \
  do {                                                                                   \
    if (rope_layout == BIQ_ROPE_HALF)                                                    \
      hipLaunchKernelGGL((qk_prep_kernel<T, true>), grid, dim3(256), 0, s, a, ob);       \
    else                                                                                 \
      hipLaunchKernelGGL((qk_prep_kernel<T, false>), grid, dim3(256), 0, s, a, ob);      \
  } while (0)
  if (in_dtype == BIQ_DTYPE_F32) BIQ_PREP(float);
  else if (in_dtype == BIQ_DTYPE_F16) BIQ_PREP(f16_t);
  else BIQ_PREP(bf16_t);
#undef BIQ_PREP
  return biq::check_launch("qk norm rope");
}
