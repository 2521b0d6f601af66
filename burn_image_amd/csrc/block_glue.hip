// Row-wise glue of the modulated DiT block (crates/burn_boogu/src/model/block.rs:91-111) for
// gfx950: strict-f32 RMS normalisation, tanh-gated residual update and (1 + scale) modulation,
// fused so that each glue step reads and writes every activation row once.
//
//   u    = branch * (1 + branch_scale[b]) + branch_shift[b]          (either may be NULL)
//   r    = x + (u / rms(u)) * gamma_b * tanh(gate[b])                 (x given: residual update)
//   r    = u                                                          (x NULL)
//   next = ((r / rms(r)) * gamma_n) * (1 + scale[b])                  (next_out given)
// The branch modulation u is the dual-stream block's MLP input, base * (scale_mlp + 1) +
// shift_mlp (block.rs:322-324,341-344).
//
// rms(v) = sqrt(mean(v^2) + eps) over the row, reduced in f32 (rms_normalized, norm.rs:28-35;
// Burn's nn::RmsNorm for the gamma product; RmsNormZero's modulation order, norm.rs:144-152).
// Each v / rms is the correctly rounded quotient, from 1 / rms and one residual step (biq::div_rn;
// exact while values, rms and quotients stay within 2^-100 .. 2^100 in magnitude), measured
// 45 -> 38 us on the 4608 x 3072 middle pass.
// b = row / rows_per_batch picks the batch element's gate / scale row.  One 256-thread workgroup
// per row: rows of up to 4096 elements are held in registers (block_glue_row_kernel); wider rows
// are read once per pass (block_glue_kernel; the re-reads mostly hit L2).
#include <math.h>

#include "common.h"

namespace {

constexpr int GT = 256;

__device__ __forceinline__ float load_elem(const void *p, int dt, int64_t i) {
  if (dt == BIQ_DTYPE_F32) return reinterpret_cast<const float *>(p)[i];
  const uint16_t h = reinterpret_cast<const uint16_t *>(p)[i];
  if (dt == BIQ_DTYPE_BF16) return biq::bitcast<float>((uint32_t)h << 16);
  return biq::f16_bits_to_f32(h);
}

__device__ __forceinline__ void store_elem(void *p, int dt, int64_t i, float v) {
  if (dt == BIQ_DTYPE_F32) reinterpret_cast<float *>(p)[i] = v;
  else if (dt == BIQ_DTYPE_F16) reinterpret_cast<_Float16 *>(p)[i] = (_Float16)v;
  else reinterpret_cast<uint16_t *>(p)[i] = (uint16_t)biq::f32_to_bf16_bits(v);
}

// Sum over the workgroup (all threads receive the result).
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red may still be read by the previous reduction
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < GT / 64; ++i) t += red[i];
  return t;
}

struct GlueArgs {
  int64_t rows, width, rows_per_batch;
  const float *x;
  const void *branch;
  int branch_dtype;
  const float *branch_scale, *branch_shift;
  const float *branch_gamma;
  float branch_eps;
  const float *gate;
  float *x_out;
  const float *next_gamma;
  float next_eps;
  const float *next_scale;
  void *next_out;
  int next_dtype;
};

__global__ void __launch_bounds__(GT) block_glue_kernel(GlueArgs a) {
  __shared__ float red[GT / 64];
  const int64_t row = blockIdx.x;
  const int64_t b = row / a.rows_per_batch;
  const int64_t W = a.width, base = row * W;
  const float inv_w = 1.0f / (float)W;
  // the (optionally modulated) branch element i of this row
  auto branch_at = [&](int64_t i) {
    float v = load_elem(a.branch, a.branch_dtype, base + i);
    if (a.branch_scale) v *= a.branch_scale[b * W + i] + 1.0f;
    if (a.branch_shift) v += a.branch_shift[b * W + i];
    return v;
  };

  // residual branch: r = x + branch / rms(branch) * gamma * tanh(gate), or r = branch
  float rms_b = 1.0f;
  if (a.x) {
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < W; i += GT) {
      const float v = branch_at(i);
      ss += v * v;
    }
    rms_b = sqrtf(block_sum(ss, red) * inv_w + a.branch_eps);
  }
  const float2 db = biq::rn_divisor(rms_b);
  float ss_r = 0.0f;
  for (int64_t i = threadIdx.x; i < W; i += GT) {
    const float v = branch_at(i);
    float r = v;
    if (a.x) {
      float nb = biq::div_rn(v, db.x, db.y);
      if (a.branch_gamma) nb *= a.branch_gamma[i];
      if (a.gate) nb *= tanhf(a.gate[b * W + i]);
      r = a.x[base + i] + nb;
      if (a.x_out) a.x_out[base + i] = r;
    }
    ss_r += r * r;
  }
  if (!a.next_out) return;
  const float rms_r = sqrtf(block_sum(ss_r, red) * inv_w + a.next_eps);
  const float2 dr = biq::rn_divisor(rms_r);
  // The residual row was written above by this same thread for the same i, so reading it back
  // (or recomputing from the inputs when x_out is absent) gives the identical f32 value.
  for (int64_t i = threadIdx.x; i < W; i += GT) {
    float r;
    if (a.x) {
      if (a.x_out) {
        r = a.x_out[base + i];
      } else {
        float nb = biq::div_rn(branch_at(i), db.x, db.y);
        if (a.branch_gamma) nb *= a.branch_gamma[i];
        if (a.gate) nb *= tanhf(a.gate[b * W + i]);
        r = a.x[base + i] + nb;
      }
    } else {
      r = branch_at(i);
    }
    float n = biq::div_rn(r, dr.x, dr.y);
    if (a.next_gamma) n *= a.next_gamma[i];
    if (a.next_scale) n *= a.next_scale[b * W + i] + 1.0f;
    store_elem(a.next_out, a.next_dtype, base + i, n);
  }
}

// ---------------------------------------------------------------------------------------------
// The same pass with the row held in registers (rows of up to 4096 elements, W % 4 == 0, 16-byte
// aligned rows): one 256-thread workgroup per row, thread t holding the 4-vectors t, t + 256, ...
// Every load goes through a buffer descriptor at the row (or batch element) with no branch around
// it -- vectors past the row and absent inputs read zero, and the null checks guard only the
// arithmetic -- so each phase's loads (branch + residual + branch modulation; gamma + gate during
// the first row sum; next gamma + scale during the second) are in flight together.  With the
// loads under per-vector branches the compiler had waited after each residual load: three
// serial memory round trips per row instead of one.  The residual row r stays in registers for
// the second norm.  Per element the arithmetic is the order of
// block_glue_kernel; only the f32 summation order of the two row sums differs.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int GR_MAXK = 4;  // vectors of 4 per thread: rows up to 256 * 4 * 4 = 4096 elements
// The kernel is instantiated per vector count GK = ceil(W / 1024): a 3072-wide row holds 3 vectors
// per thread in 92 registers (5 waves per SIMD) where the 4-vector form took 137-140 (3 waves);
// measured on the 4608 x 3072 middle pass: 57 -> 48 us.

// Buffer descriptor over `bytes` from base (a wave-uniform base): loads at offsets past the range
// (or any offset, for a zero range) read as zero without a branch.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// Elements 4v .. 4v + 3 of a row in dtype DT at byte offset o (one 16- or 8-byte load).
template <int DT>
__device__ __forceinline__ f32x4_t load4(rsrc_t r, uint32_t o) {
  if constexpr (DT == BIQ_DTYPE_F32) {
    const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0);
    return f32x4_t{biq::bitcast<float>(d[0]), biq::bitcast<float>(d[1]), biq::bitcast<float>(d[2]),
                   biq::bitcast<float>(d[3])};
  } else {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t d = __builtin_amdgcn_raw_buffer_load_b64(r, o, 0, 0);
    if constexpr (DT == BIQ_DTYPE_BF16)
      return f32x4_t{biq::bf16_lo_to_f32(d[0]), biq::bf16_hi_to_f32(d[0]), biq::bf16_lo_to_f32(d[1]),
                     biq::bf16_hi_to_f32(d[1])};
    else
      return f32x4_t{biq::f16_bits_to_f32((uint16_t)(d[0] & 0xffffu)), biq::f16_bits_to_f32((uint16_t)(d[0] >> 16)),
                     biq::f16_bits_to_f32((uint16_t)(d[1] & 0xffffu)), biq::f16_bits_to_f32((uint16_t)(d[1] >> 16))};
  }
}

template <int DT>
__device__ __forceinline__ void store4(void *p, int64_t v, const f32x4_t &x) {
  if constexpr (DT == BIQ_DTYPE_F32) {
    reinterpret_cast<f32x4_t *>(p)[v] = x;
  } else if constexpr (DT == BIQ_DTYPE_BF16) {
    uint2 d;
    d.x = biq::pack_bf16x2(x[0], x[1]);
    d.y = biq::pack_bf16x2(x[2], x[3]);
    reinterpret_cast<uint2 *>(p)[v] = d;
  } else {
    uint2 d;
    d.x = biq::pack_f16x2(x[0], x[1]);
    d.y = biq::pack_f16x2(x[2], x[3]);
    reinterpret_cast<uint2 *>(p)[v] = d;
  }
}

// branch dtype; next dtype (-1: no next output); vectors per thread; residual given (a.x): the
// first norm of a block has none, and its instantiation without the residual's registers runs
// more waves per SIMD
template <int BDT, int NDT, int GK, bool RES>
__global__ void __launch_bounds__(GT) block_glue_row_kernel(GlueArgs a) {
  __shared__ float red[GT / 64];
  // rows < 2^31 (host check); a batch longer than the tensor holds every row
  const uint32_t row = blockIdx.x;
  const uint32_t rpb = (uint32_t)(a.rows_per_batch < a.rows ? a.rows_per_batch : a.rows);
  const uint32_t b = row / rpb;
  const uint32_t W = (uint32_t)a.width, nv = W / 4;  // W <= 4096: offsets within a row are small
  const float inv_w = 1.0f / (float)W;
  constexpr uint32_t BSZ = BDT == BIQ_DTYPE_F32 ? 16u : 8u;  // bytes per branch 4-vector
  constexpr uint32_t OOB = 0x80000000u;
  // descriptors at this row / this batch element (64-bit bases, wave-uniform); an absent input
  // gets an empty range, so its loads read zero and only the arithmetic below is skipped
  const int64_t rowW = (int64_t)row * W, bW = (int64_t)b * W;
  const rsrc_t r_br = rsrc(static_cast<const char *>(a.branch) + rowW * (BSZ / 4), nv * BSZ);
  auto vec_rsrc = [&](const float *p, int64_t first) { return rsrc(p ? p + first : a.x, p ? nv * 16u : 0u); };
  const rsrc_t r_x = vec_rsrc(a.x, rowW);
  const rsrc_t r_bsc = vec_rsrc(a.branch_scale, bW), r_bsh = vec_rsrc(a.branch_shift, bW);
  const rsrc_t r_bg = vec_rsrc(a.branch_gamma, 0), r_gate = vec_rsrc(a.gate, bW);
  const rsrc_t r_ng = vec_rsrc(a.next_gamma, 0), r_nsc = vec_rsrc(a.next_scale, bW);
  auto vo = [&](int k) {  // byte offset of this thread's k-th 4-vector in an f32 row (OOB past W)
    const uint32_t v = threadIdx.x + GT * k;
    return v < nv ? v * 16u : OOB;
  };

  // every load of the first phase in flight before the first use: the row's branch and residual
  // vectors, then the branch modulation rows
  f32x4_t u[GK], xr[GK], m0[GK], m1[GK];  // the modulated branch (then r); residual; scale; shift
#pragma unroll
  for (int k = 0; k < GK; ++k) {
    const uint32_t v = threadIdx.x + GT * k;
    u[k] = load4<BDT>(r_br, v < nv ? v * BSZ : OOB);
    if constexpr (RES) xr[k] = load4<BIQ_DTYPE_F32>(r_x, vo(k));
  }
#pragma unroll
  for (int k = 0; k < GK; ++k) {
    m0[k] = load4<BIQ_DTYPE_F32>(r_bsc, vo(k));
    m1[k] = load4<BIQ_DTYPE_F32>(r_bsh, vo(k));
  }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < GK; ++k) {
    if (threadIdx.x + GT * k < nv) {
      if (a.branch_scale) u[k] *= m0[k] + 1.0f;
      if (a.branch_shift) u[k] += m1[k];
      ss += u[k][0] * u[k][0] + u[k][1] * u[k][1] + u[k][2] * u[k][2] + u[k][3] * u[k][3];
    }
  }
  float ss_r = ss;
  if constexpr (RES) {
    // gamma and gate rows in flight during the row sum
#pragma unroll
    for (int k = 0; k < GK; ++k) {
      m0[k] = load4<BIQ_DTYPE_F32>(r_bg, vo(k));
      m1[k] = load4<BIQ_DTYPE_F32>(r_gate, vo(k));
    }
    const float2 db = biq::rn_divisor(sqrtf(block_sum(ss, red) * inv_w + a.branch_eps));
    ss_r = 0.0f;
#pragma unroll
    for (int k = 0; k < GK; ++k) {
      const uint32_t v = threadIdx.x + GT * k;
      if (v < nv) {
        f32x4_t nb;
#pragma unroll
        for (int e = 0; e < 4; ++e) nb[e] = biq::div_rn(u[k][e], db.x, db.y);
        if (a.branch_gamma) nb *= m0[k];
        if (a.gate) {
          const f32x4_t gt = m1[k];
          nb *= f32x4_t{tanhf(gt[0]), tanhf(gt[1]), tanhf(gt[2]), tanhf(gt[3])};
        }
        const f32x4_t r = xr[k] + nb;
        if (a.x_out) reinterpret_cast<f32x4_t *>(a.x_out)[rowW / 4 + v] = r;
        u[k] = r;
        ss_r += r[0] * r[0] + r[1] * r[1] + r[2] * r[2] + r[3] * r[3];
      }
    }
  }
  if constexpr (NDT >= 0) {
    // next gamma and scale rows in flight during the second row sum
#pragma unroll
    for (int k = 0; k < GK; ++k) {
      m0[k] = load4<BIQ_DTYPE_F32>(r_ng, vo(k));
      m1[k] = load4<BIQ_DTYPE_F32>(r_nsc, vo(k));
    }
    const float2 dr = biq::rn_divisor(sqrtf(block_sum(ss_r, red) * inv_w + a.next_eps));
#pragma unroll
    for (int k = 0; k < GK; ++k) {
      const uint32_t v = threadIdx.x + GT * k;
      if (v < nv) {
        f32x4_t n;
#pragma unroll
        for (int e = 0; e < 4; ++e) n[e] = biq::div_rn(u[k][e], dr.x, dr.y);
        if (a.next_gamma) n *= m0[k];
        if (a.next_scale) n *= m1[k] + 1.0f;
        store4<NDT>(a.next_out, rowW / 4 + v, n);
      }
    }
  }
}

}  // namespace

extern "C" int biq_block_glue(void *stream, int64_t rows, int64_t width, int64_t rows_per_batch,
                              const float *x, const void *branch, int branch_dtype,
                              const float *branch_scale, const float *branch_shift,
                              const float *branch_gamma, float branch_eps, const float *gate,
                              float *x_out, const float *next_gamma, float next_eps,
                              const float *next_scale, void *next_out, int next_dtype) {
  biq::clear_error();
  if (!branch) return biq::fail(BIQ_ERR_INVALID_ARG, "null branch");
  if (rows <= 0 || width <= 0 || rows_per_batch <= 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "block glue requires non-empty rows, width and rows per batch");
  if (rows > 0x7fffffffLL) return biq::fail(BIQ_ERR_UNSUPPORTED, "block glue: too many rows");
  auto dt_ok = [](int d) { return d == BIQ_DTYPE_F32 || d == BIQ_DTYPE_F16 || d == BIQ_DTYPE_BF16; };
  if (!dt_ok(branch_dtype) || (next_out && !dt_ok(next_dtype)))
    return biq::fail(BIQ_ERR_INVALID_ARG, "block glue dtypes must be F32, F16 or BF16");
  if (!x && !next_out) return biq::fail(BIQ_ERR_INVALID_ARG, "block glue has nothing to write");
  if (x && !x_out && !next_out) return biq::fail(BIQ_ERR_INVALID_ARG, "block glue has nothing to write");
  if (!(branch_eps >= 0.0f) || !(next_eps >= 0.0f))
    return biq::fail(BIQ_ERR_INVALID_ARG, "block glue epsilons must be non-negative");
  GlueArgs a{rows, width, rows_per_batch, x, branch, branch_dtype, branch_scale, branch_shift, branch_gamma, branch_eps, gate,
             x_out, next_gamma, next_eps, next_scale, next_out, next_dtype};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // wave-per-row form: rows of <= 4096 elements in whole 16-byte vectors, every row 16-byte aligned
  auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  auto al8 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; };
  const bool vec = width % 4 == 0 && width <= GT * 4 * GR_MAXK &&
                   (branch_dtype == BIQ_DTYPE_F32 ? al16(branch) : al8(branch)) && al16(x) && al16(x_out) &&
                   al16(branch_scale) && al16(branch_shift) && al16(branch_gamma) && al16(gate) &&
                   al16(next_gamma) && al16(next_scale) &&
                   (!next_out || (next_dtype == BIQ_DTYPE_F32 ? al16(next_out) : al8(next_out)));
  if (vec) {
    const dim3 grid((unsigned)rows);
    const int gk = (int)((width / 4 + GT - 1) / GT);
#define BIQ_GLUE_K(BD, ND, RES)                                                                    \
  do {                                                                                             \
    if (gk == 1) hipLaunchKernelGGL((block_glue_row_kernel<BD, ND, 1, RES>), grid, dim3(GT), 0, s, a); \
    else if (gk == 2) hipLaunchKernelGGL((block_glue_row_kernel<BD, ND, 2, RES>), grid, dim3(GT), 0, s, a); \
    else if (gk == 3) hipLaunchKernelGGL((block_glue_row_kernel<BD, ND, 3, RES>), grid, dim3(GT), 0, s, a); \
    else hipLaunchKernelGGL((block_glue_row_kernel<BD, ND, 4, RES>), grid, dim3(GT), 0, s, a);     \
  } while (0)
#define BIQ_GLUE(BD, ND)                                                                           \
  do {                                                                                             \
    if (x) BIQ_GLUE_K(BD, ND, true);                                                               \
    else BIQ_GLUE_K(BD, ND, false);                                                                \
  } while (0)
#define BIQ_GLUE_N(BD)                                                                             \
  do {                                                                                             \
    if (!next_out) BIQ_GLUE_K(BD, -1, true);  /* (x is given: checked above) */                    \
    else if (next_dtype == BIQ_DTYPE_F32) BIQ_GLUE(BD, BIQ_DTYPE_F32);                             \
    else if (next_dtype == BIQ_DTYPE_F16) BIQ_GLUE(BD, BIQ_DTYPE_F16);                             \
    else BIQ_GLUE(BD, BIQ_DTYPE_BF16);                                                             \
  } while (0)
    if (branch_dtype == BIQ_DTYPE_F32) BIQ_GLUE_N(BIQ_DTYPE_F32);
    else if (branch_dtype == BIQ_DTYPE_F16) BIQ_GLUE_N(BIQ_DTYPE_F16);
    else BIQ_GLUE_N(BIQ_DTYPE_BF16);
#undef BIQ_GLUE_N
#undef BIQ_GLUE
#undef BIQ_GLUE_K
    return biq::check_launch("block glue");
  }
  hipLaunchKernelGGL(block_glue_kernel, dim3((unsigned)rows), dim3(GT), 0, s, a);
  return biq::check_launch("block glue");
}

// ---------------------------------------------------------------------------------------------
// silu of the conditioning rows before the modulation projection (RmsNormZero,
// crates/burn_boogu/src/model/norm.rs:145: linear_forward(&self.linear, silu(conditioning))).
// silu(a) = a / (1 + e^-a) in f32; output f32.
// ---------------------------------------------------------------------------------------------
namespace {
__global__ void __launch_bounds__(256) silu_kernel(int64_t n, const void *x, int dt, float *y) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float a = load_elem(x, dt, i);
  y[i] = a / (1.0f + expf(-a));
}
}  // namespace

extern "C" int biq_silu(void *stream, int64_t n, const void *x, int x_dtype, float *y) {
  biq::clear_error();
  if (!x || !y) return biq::fail(BIQ_ERR_INVALID_ARG, "null pointer argument");
  if (n <= 0) return biq::fail(BIQ_ERR_INVALID_ARG, "silu requires a non-empty input");
  if (x_dtype != BIQ_DTYPE_F32 && x_dtype != BIQ_DTYPE_F16 && x_dtype != BIQ_DTYPE_BF16)
    return biq::fail(BIQ_ERR_INVALID_ARG, "silu input dtype must be F32, F16 or BF16");
  if ((n + 255) / 256 > 0x7fffffffLL) return biq::fail(BIQ_ERR_UNSUPPORTED, "silu input too large");
  hipLaunchKernelGGL(silu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), n, x, x_dtype, y);
  return biq::check_launch("silu");
}
