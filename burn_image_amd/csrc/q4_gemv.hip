// Small-M packed-Q4 projection (M <= 16) for gfx950: an HBM-bound streaming kernel.
//
// The same operator as q4_gemm.hip (y = x . W + bias, exact nibbles, f32 block scales) for the
// reference's small-row callers: the RmsNormZero modulation projection (one conditioning row,
// crates/burn_boogu/src/model/norm.rs:138-153) and short instruction streams.  With a 128-row
// tile those calls would waste the matrix cores and launch only N / 256 workgroups.
//
// Work unit: one wave owns a column slab over one K chunk; a K chunk is every nchunks-th unit of
// 32 * KN_BATCH (or 128 * NK_BATCH) k, so the chunks of a slab interleave and the waves of the
// chip read one band of packed rows at a time.  Three kernels:
//  * q4_gemv_kn_lds_kernel ([K/8, N], M <= 8, the modulation row): one workgroup per slab stages
//    the activations once in LDS and its waves double-buffer packed words and scales in registers
//    (the loads of the next unit in flight while the current one computes).
//  * q4_gemv_kn_kernel / q4_gemv_nk_kernel (M <= 16, either layout): a wave issues the loads of a
//    whole batch (words, activations and scales) before its first MFMA; nothing is staged.
// Every load goes through a buffer descriptor with a wave-uniform base, so a word, scale or
// activation outside the matrix reads as zero without a branch.
//
// MFMA: v_mfma_f32_16x16x32_f16.  A = the (<= 16) activation rows, converted to f16 in the
// nibble slot order [k0,k4,k1,k5,k2,k6,k3,k7] (f32 activations as hi + lo: two MFMAs, or in the
// staged kernel one MFMA with the lo parts in rows 8..15); B = the
// packed words decoded exactly to f16 (the q4_gemm.hip decode).  The k order inside one MFMA is
// free as long as A and B agree; the two layouts use that freedom differently:
//  * [K/8, N] words: lane (c16 = l % 16, g = l / 16) loads 16 bytes = the words of columns
//    4 c16 .. 4 c16 + 3 in packed row k0/8 + g.  MFMA c contracts column 4 c16 + c over the 32 k
//    of the step, so a wave reads 64 columns x 32 k (4 x 256 contiguous bytes) per step.
//  * [N, K/8] words: lane (c16, g) loads 16 bytes = 4 consecutive words of column c16; MFMA c
//    contracts octet 4 g + c of a 128-k super-step, so a wave reads 16 columns x 128 k.
// Each K block's partial is scaled by its f32 scale in f32 (the scale is never rounded); where a
// block is shorter than one MFMA's k, the MFMA is repeated with the other blocks' lanes masked.
// Two ways to combine the K chunks of a column slab, both deterministic (a fixed summation order;
// device-wide f32 atomics were measured far slower):
//  * in-workgroup (WPS > 1, the usual case): the WPS waves of one workgroup are the K chunks of
//    one slab; they leave their partial rows in LDS and, after one barrier, each thread adds one
//    output's chunks in order plus the bias and stores y.  One launch, no scratch memory.
//  * across workgroups (WPS == 1, when there are too few slabs to fill the chip with one
//    workgroup each): each wave stores its partial rows into a per-stream workspace and a second
//    kernel adds the chunks in order plus the bias.
#include <cstdlib>
#include <string>

#include "common.h"

#ifndef BIQ_GEMV_TARGET_WAVES
#define BIQ_GEMV_TARGET_WAVES 4096
#endif

namespace {

constexpr int GV_THREADS = 256;  // 4 waves per workgroup (independent work units)
constexpr int KN_SLAB = 64;      // columns per wave, [K/8, N] layout
#ifndef BIQ_GEMV_KN_BATCH
#define BIQ_GEMV_KN_BATCH 4
#endif
constexpr int KN_BATCH = BIQ_GEMV_KN_BATCH;  // steps of 32 k per batch (>= 4: a unit of >= 128 k)
// The in-register [K/8, N] kernel takes twice that for blocks >= 32: twice the loads in flight per
// wave (16 x 3072 x 9216: 9.44 -> 9.04 us); the LDS-staged kernel keeps KN_BATCH (8 measured
// slower there: 7.4 -> 8.3 us at 1 x 3072 x 12288), and so do blocks of 8 and 16, whose scales per
// batch would grow with it.
constexpr int kn_reg_batch(int blk) { return blk >= 32 ? 2 * KN_BATCH : KN_BATCH; }
constexpr int NK_SLAB = 16;      // columns per wave, [N, K/8] layout
constexpr int NK_BATCH = 2;      // super-steps of 128 k per batch -> unit of 256 k

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Exact nibble decode, slot order [k0,k4,k1,k5,k2,k6,k3,k7] (the q4_gemm.hip decode: low
// nibbles of each half as 0x6400 | (v ^ 8), high nibbles in place scaled by 1/16 in the FMA).
__device__ __forceinline__ half8_t unpack_q4(uint32_t w) {
  const uint32_t M0 = 0x000F000Fu, C0 = 0x64086408u;
  const uint32_t M1 = 0x00F000F0u, C1 = 0x64806480u;
  const uint32_t w8 = w >> 8;
  u32x4_t d;
  d[0] = ((w ^ C0) & M0) | (C0 & ~M0);
  d[1] = ((w ^ C1) & M1) | (C1 & ~M1);
  d[2] = ((w8 ^ C0) & M0) | (C0 & ~M0);
  d[3] = ((w8 ^ C1) & M1) | (C1 & ~M1);
  const _Float16 o = (_Float16)1.0f, t = (_Float16)0.0625f;
  const _Float16 a = (_Float16)(-1032.0f), b = (_Float16)(-72.0f);
  const half8_t mul = {o, o, t, t, o, o, t, t};
  const half8_t add = {a, a, b, b, a, a, b, b};
  return __builtin_elementwise_fma(biq::bitcast<half8_t>(d), mul, add);
}

// 8 raw activations of the x dtype.
template <int XD>
struct XRaw {
  static constexpr int WORDS = XD == BIQ_DTYPE_F32 ? 8 : 4;
  uint32_t v[WORDS];
};

template <int XD>
__device__ __forceinline__ void load_x8(XRaw<XD> &r, const char *p, bool ok) {
  if constexpr (XD == BIQ_DTYPE_F32) {
    u32x4_t a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    if (ok) {
      a = reinterpret_cast<const u32x4_t *>(p)[0];
      b = reinterpret_cast<const u32x4_t *>(p)[1];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) { r.v[i] = a[i]; r.v[4 + i] = b[i]; }
  } else {
    u32x4_t a = {0u, 0u, 0u, 0u};
    if (ok) a = *reinterpret_cast<const u32x4_t *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.v[i] = a[i];
  }
}

// 8 activations -> f16 in slot order; f32 activations also give the lo remainder.
template <int XD>
__device__ __forceinline__ void x8_slots(const XRaw<XD> &r, half8_t &hi, half8_t &lo) {
  float x[8];
  if constexpr (XD == BIQ_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = biq::bitcast<float>(r.v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (XD == BIQ_DTYPE_BF16) {
        x[2 * i] = biq::bf16_lo_to_f32(r.v[i]);
        x[2 * i + 1] = biq::bf16_hi_to_f32(r.v[i]);
      } else {
        x[2 * i] = biq::f16_bits_to_f32((uint16_t)(r.v[i] & 0xffffu));
        x[2 * i + 1] = biq::f16_bits_to_f32((uint16_t)(r.v[i] >> 16));
      }
    }
  }
  u32x4_t h, l;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const _Float16 h0 = (_Float16)x[i], h1 = (_Float16)x[i + 4];
    half2_t hh = {h0, h1};
    h[i] = biq::bitcast<uint32_t>(hh);
    if constexpr (XD == BIQ_DTYPE_F32) l[i] = biq::pack_f16x2(x[i] - (float)h0, x[i + 4] - (float)h1);
  }
  hi = biq::bitcast<half8_t>(h);
  if constexpr (XD == BIQ_DTYPE_F32) lo = biq::bitcast<half8_t>(l);
}

template <int XD>
__device__ __forceinline__ f32x4_t mfma_x(const half8_t &ahi, const half8_t &alo, const half8_t &b,
                                          f32x4_t c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b, c, 0, 0, 0);
  if constexpr (XD == BIQ_DTYPE_F32) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b, c, 0, 0, 0);
  return c;
}

// y[m, n] = bias[n] + sum over K chunks of part[chunk, m, n], chunks added in order (so the
// result does not depend on scheduling).  Thread = 4 consecutive columns (N % 8 == 0).
__global__ void __launch_bounds__(256) gv_reduce_kernel(const float *__restrict__ part, int64_t nchunks,
                                                        const float *__restrict__ bias,
                                                        float *__restrict__ y, int64_t M, int64_t N) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M * N / 4) return;
  const int64_t e = 4 * t, n = e % N;
  f32x4_t s = bias ? f32x4_t{bias[n], bias[n + 1], bias[n + 2], bias[n + 3]} : f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int64_t stride = M * N;
  int64_t c = 0;
  for (; c + 4 <= nchunks; c += 4) {  // four independent loads in flight, added in chunk order
    const f32x4_t p0 = *reinterpret_cast<const f32x4_t *>(part + (c + 0) * stride + e);
    const f32x4_t p1 = *reinterpret_cast<const f32x4_t *>(part + (c + 1) * stride + e);
    const f32x4_t p2 = *reinterpret_cast<const f32x4_t *>(part + (c + 2) * stride + e);
    const f32x4_t p3 = *reinterpret_cast<const f32x4_t *>(part + (c + 3) * stride + e);
    s += p0;
    s += p1;
    s += p2;
    s += p3;
  }
  for (; c < nchunks; ++c) s += *reinterpret_cast<const f32x4_t *>(part + c * stride + e);
#pragma unroll
  for (int i = 0; i < 4; ++i) y[e + i] = s[i];
}

// ---------------------------------------------------------------- [K/8, N] words, [K/BLK, N] scales
// Work unit of wave `wave` in workgroup `blockIdx.x`: (slab, K chunk).  WPS > 1: the workgroup is
// one slab and its waves the K chunks; WPS == 1: independent waves numbered slab-fastest.
template <int WPS>
__device__ __forceinline__ void gv_unit(int64_t nslabs, int64_t &slab, int64_t &chunk) {
  // wave-uniform by construction; readfirstlane tells the compiler, so that the addresses built
  // from it stay scalar (a buffer descriptor built from a per-lane value costs a waterfall loop)
  const int64_t wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if constexpr (WPS > 1) {
    slab = blockIdx.x;
    chunk = wave;
  } else {
    const int64_t wid = (int64_t)blockIdx.x * (GV_THREADS / 64) + wave;
    slab = wid % nslabs;
    chunk = wid / nslabs;
  }
}

// In-workgroup combination (WPS > 1): wave w's partial (row m, column c of the slab) sits at
// red[(w * 16 + m) * SLAB + c]; each thread adds one output's WPS chunks in wave order.
template <int WPS, int SLAB>
__device__ __forceinline__ void gv_reduce_lds(const float *red, const float *__restrict__ bias,
                                              float *__restrict__ y, int64_t M, int64_t N, int64_t col0) {
  for (int o = threadIdx.x; o < 16 * SLAB; o += 64 * WPS) {
    const int m = o / SLAB, c = o % SLAB;
    const int64_t n = col0 + c;
    if (m >= M || n >= N) continue;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < WPS; ++w) v += red[(w * 16 + m) * SLAB + c];
    y[m * N + n] = v + (bias ? bias[n] : 0.0f);
  }
}

template <int XD, int BLK, int WPS>
__global__ void __launch_bounds__(WPS > 1 ? 64 * WPS : GV_THREADS) q4_gemv_kn_kernel(
    const void *__restrict__ xv, int64_t ldx, const uint32_t *__restrict__ words,
    const float *__restrict__ scales, const float *__restrict__ bias, float *__restrict__ y,
    float *__restrict__ part, int64_t M, int64_t N, int64_t K, int64_t nchunks, int64_t nslabs,
    int64_t nunits) {
  const int lane = threadIdx.x & 63;
  int64_t slab, chunk;
  gv_unit<WPS>(nslabs, slab, chunk);
  if (WPS == 1 && slab + chunk * nslabs >= nunits) return;
  const int c16 = lane & 15, g = lane >> 4;
  const int64_t ncol = slab * KN_SLAB + 4 * c16;  // columns ncol .. ncol + 3
  const int64_t KW = K / 8, nblk = K / BLK;
  const bool col_ok = ncol < N;
  const bool row_ok = c16 < M;
  constexpr int ESZ = XD == BIQ_DTYPE_F32 ? 4 : 2;
  constexpr int KB = kn_reg_batch(BLK);  // steps of 32 k per batch

  f32x4_t acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  constexpr int SPB = BLK >= 32 ? BLK / 32 : 1;                                        // steps per block
  constexpr int NSC = BLK >= 32 ? (KB + SPB - 1) / SPB : KB * (32 / BLK);  // blocks per batch

  // Branch-free loads through buffer descriptors (scalar: every base is wave-uniform): words and
  // scales through descriptors that start at the batch and end at the matrix, activations through
  // one descriptor over the M rows.  A word or scale outside the matrix (packed rows past K,
  // columns past N) reads as zero; an activation past K or M gets the out-of-range offset OOB and
  // reads as zero.  Without a branch per load the compiler waits for each step's data only when
  // that step computes, so a batch's loads overlap its earlier steps.  Offsets are 32-bit: inside
  // a batch below 32 packed rows of N < 2^24 words (32 N * 4 < 2^31); activations below 16 rows
  // of ldx < 2^21.
  constexpr uint32_t OOB = 0x80000000u;
  auto rsrc = [](const void *base, int64_t bytes) {
    const uint32_t n = bytes > 0x7fffffffLL ? 0x7fffffffu : (bytes < 0 ? 0u : (uint32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)n, 0x00020000);
  };
  const auto rx = rsrc(xv, ((M - 1) * ldx + K) * ESZ);
  const uint32_t w_lane = col_ok ? (uint32_t)((g * N + ncol) * 4) : OOB;
  const int64_t x_row = (int64_t)c16 * ldx + 8 * g;  // this lane's 8 activations of a step, less kb
  // K chunk c is the units of 32 * KB k numbered c, c + nchunks, c + 2 nchunks, ...: the
  // chunks of a slab interleave, so the waves of the chip read one band of packed rows at a time.
  for (int64_t kb = chunk * 32 * KB; kb < K; kb += nchunks * 32 * KB) {
    const int64_t kw0 = kb / 8;
    const auto rw = rsrc(words + kw0 * N, (KW - kw0) * N * 4);
    u32x4_t wv[KB];
    XRaw<XD> xr[KB];
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      wv[t] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_lane == OOB ? OOB : w_lane + (uint32_t)(4 * t * N * 4), 0, 0);
      const bool x_ok = row_ok && kb + 32 * t + 8 * g < K;
      const uint32_t xo = x_ok ? (uint32_t)((x_row + kb + 32 * t) * ESZ) : OOB;
      if constexpr (XD == BIQ_DTYPE_F32) {
        const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
        const u32x4_t b = __builtin_amdgcn_raw_buffer_load_b128(rx, xo == OOB ? OOB : xo + 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) { xr[t].v[i] = a[i]; xr[t].v[4 + i] = b[i]; }
      } else {
        const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) xr[t].v[i] = a[i];
      }
    }
    const auto rsc = rsrc(scales + (kb / BLK) * N, (nblk - kb / BLK) * N * 4);
    float sc[NSC][4];
#pragma unroll
    for (int j = 0; j < NSC; ++j) {
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(
          rsc, col_ok ? (uint32_t)((j * N + ncol) * 4) : OOB, 0, 0);
#pragma unroll
      for (int c = 0; c < 4; ++c) sc[j][c] = biq::bitcast<float>(v[c]);
    }

    if constexpr (BLK >= 32) {
      f32x4_t p[4];
#pragma unroll
      for (int t = 0; t < KB; ++t) {
        half8_t ahi, alo;
        x8_slots<XD>(xr[t], ahi, alo);
#pragma unroll
        for (int c = 0; c < 4; ++c)
          p[c] = mfma_x<XD>(ahi, alo, unpack_q4(wv[t][c]), t % SPB == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : p[c]);
        if (t % SPB == SPB - 1) {
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[c] += sc[t / SPB][c] * p[c];
        }
      }
    } else {
      // blocks of 8 or 16: lane group g holds octet g of the step, which is in block g / GPB
      constexpr int PER = 32 / BLK, GPB = BLK / 8;
      const half8_t zh = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < KB; ++t) {
        half8_t ahi, alo;
        x8_slots<XD>(xr[t], ahi, alo);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const half8_t bq = unpack_q4(wv[t][c]);
#pragma unroll
          for (int u = 0; u < PER; ++u) {
            const half8_t bm = (g / GPB == u) ? bq : zh;
            const f32x4_t p = mfma_x<XD>(ahi, alo, bm, f32x4_t{0.f, 0.f, 0.f, 0.f});
            acc[c] += sc[t * PER + u][c] * p;
          }
        }
      }
    }
  }

  // 16x16 accumulator of MFMA c: lane holds column ncol + c, rows 4 g + r.
  if constexpr (WPS > 1) {
    __shared__ float red[WPS * 16 * KN_SLAB];
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) red[(w * 16 + 4 * g + r) * KN_SLAB + 4 * c16 + c] = acc[c][r];
    __syncthreads();
    gv_reduce_lds<WPS, KN_SLAB>(red, bias, y, M, N, slab * KN_SLAB);
    return;
  }
  // One K chunk: y = acc + bias; several: this chunk's partial rows.
  if (col_ok) {
    float *dst = part ? part + chunk * M * N : y;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = 4 * g + r;
      if (m < M) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          dst[m * N + ncol + c] = acc[c][r] + ((!part && bias) ? bias[ncol + c] : 0.0f);
      }
    }
  }
}

// ---------------------------------------------------------------- [K/8, N], activations in LDS
// The usual form of the [K/8, N] route: one workgroup per column slab, its WPS waves the K chunks.
// The workgroup converts all M x K activations once into LDS (f16 in MFMA slot order, f32
// activations as hi and lo), so a wave's registers hold only packed words and scales, and those are
// double-buffered: the loads of a wave's next unit are in flight while it computes the current
// one.  Without that the waves of a SIMD load, then compute, in step, and HBM idles while they
// compute.  The first unit's loads are issued before the staging, which they overlap.
// M <= 8.  With f32 activations the hi parts take MFMA rows 0..7 and the lo parts rows 8..15, so
// one MFMA per step does both; y[m] = row m + row m + 8.
// LDS: the staged activations, K/8 x M slots of 16 bytes (x2 for f32), reused for the partials.
// Double buffering over 12 or 16 waves was measured, and triple buffering: both slower.
template <int XD, int BLK, int WPS>
__global__ void __launch_bounds__(64 * WPS) q4_gemv_kn_lds_kernel(
    const void *__restrict__ xv, int64_t ldx, const uint32_t *__restrict__ words,
    const float *__restrict__ scales, const float *__restrict__ bias, float *__restrict__ y, int64_t M,
    int64_t N, int64_t K) {
  extern __shared__ __attribute__((aligned(16))) unsigned char gv_lds[];
  constexpr bool F32X = XD == BIQ_DTYPE_F32;
  constexpr bool FOLD = F32X;  // lo parts in MFMA rows 8..15
  constexpr int ESZ = F32X ? 4 : 2;
  const int64_t KO = K / 8;  // octets of K
  half8_t *xs_hi = reinterpret_cast<half8_t *>(gv_lds);  // slot (octet o, row m) at o * M + m
  half8_t *xs_lo = xs_hi + KO * M;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int c16 = lane & 15, g = lane >> 4;
  const int64_t slab = blockIdx.x;
  const int64_t ncol = slab * KN_SLAB + 4 * c16;  // columns ncol .. ncol + 3
  const bool col_ok = ncol < N;
  const int64_t KW = K / 8, nblk = K / BLK;
  constexpr int UNIT = 32 * KN_BATCH;
  constexpr int SPB = BLK >= 32 ? BLK / 32 : 1;                                        // steps per block
  constexpr int NSC = BLK >= 32 ? (KN_BATCH + SPB - 1) / SPB : KN_BATCH * (32 / BLK);  // blocks per unit

  // Words and scales through buffer descriptors that start at the unit and end at the matrix: a
  // word or scale past K or N reads as zero, and so do all of a unit past K (the prefetches after
  // a wave's last unit).  Offsets inside a unit are below 16 packed rows of N < 2^24 words.
  constexpr uint32_t OOB = 0x80000000u;
  auto rsrc = [](const void *base, int64_t bytes) {
    const uint32_t n = bytes > 0x7fffffffLL ? 0x7fffffffu : (bytes < 0 ? 0u : (uint32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)n, 0x00020000);
  };
  const uint32_t w_lane = col_ok ? (uint32_t)((g * N + ncol) * 4) : OOB;
  const uint32_t s_lane = col_ok ? (uint32_t)(ncol * 4) : OOB;
  struct Unit {
    u32x4_t wv[KN_BATCH];
    u32x4_t sc[NSC];
  };
  auto load = [&](int64_t kb, Unit &u) {
    const int64_t kw0 = kb / 8, b0 = kb / BLK;
    const auto rw = rsrc(words + kw0 * N, (KW - kw0) * N * 4);
#pragma unroll
    for (int t = 0; t < KN_BATCH; ++t)
      u.wv[t] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_lane == OOB ? OOB : w_lane + (uint32_t)(4 * t * N * 4), 0, 0);
    const auto rs = rsrc(scales + b0 * N, (nblk - b0) * N * 4);
#pragma unroll
    for (int j = 0; j < NSC; ++j)
      u.sc[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, s_lane == OOB ? OOB : s_lane + (uint32_t)(j * N * 4), 0, 0);
  };

  // Units w, w + WPS, w + 2 WPS, ...: the chunks interleave, so the chip reads one band of packed
  // rows at a time.
  const int64_t kstep = (int64_t)WPS * UNIT;
  int64_t kb = (int64_t)w * UNIT;
  // Staging: thread e converts slots e, e + 64 WPS, ...  The loads of its first slot go out before
  // the weight prefetch: the vector memory counter retires in order, so the wait for those
  // activations does not also wait for the prefetched units.
  auto stage_load = [&](int64_t e, XRaw<XD> &r) {
    const int64_t o = e / M, m = e % M;
    load_x8<XD>(r, reinterpret_cast<const char *>(xv) + (m * ldx + o * 8) * ESZ, e < KO * M);
  };
  auto stage_store = [&](int64_t e, const XRaw<XD> &r) {
    half8_t hi, lo;
    x8_slots<XD>(r, hi, lo);
    if (e < KO * M) {
      xs_hi[e] = hi;
      if constexpr (F32X) xs_lo[e] = lo;
    }
  };
  XRaw<XD> x0;
  stage_load(threadIdx.x, x0);
  Unit ua, ub;
  load(kb, ua);
  stage_store(threadIdx.x, x0);
  for (int64_t e = threadIdx.x + 64 * WPS; e < KO * M; e += 64 * WPS) {
    XRaw<XD> r;
    stage_load(e, r);
    stage_store(e, r);
  }
  __syncthreads();

  // A operand source of this lane: row arow of the hi (or, FOLD rows 8..15, lo) activations
  const int arow = FOLD ? (c16 & 7) : c16;
  const bool a_row_ok = arow < M;
  const half8_t *asrc = (FOLD && c16 >= 8) ? xs_lo : xs_hi;
  f32x4_t acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const half8_t zh = {0, 0, 0, 0, 0, 0, 0, 0};
  auto mfma = [&](const half8_t &a, const half8_t &b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  };
  auto compute = [&](int64_t kb, const Unit &u) {
    half8_t a[KN_BATCH];
#pragma unroll
    for (int t = 0; t < KN_BATCH; ++t) {  // A operand of step t: octet kb / 8 + 4 t + g
      const int64_t o = kb / 8 + 4 * t + g;
      const bool ok = a_row_ok && o < KO;
      a[t] = ok ? asrc[ok ? o * M + arow : 0] : zh;
    }
    if constexpr (BLK >= 32) {
      f32x4_t p[4];
#pragma unroll
      for (int t = 0; t < KN_BATCH; ++t) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          p[c] = mfma(a[t], unpack_q4(u.wv[t][c]), t % SPB == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : p[c]);
        if (t % SPB == SPB - 1) {
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[c] += biq::bitcast<float>(u.sc[t / SPB][c]) * p[c];
        }
      }
    } else {
      // blocks of 8 or 16: lane group g holds octet g of the step, which is in block g / GPB
      constexpr int PER = 32 / BLK, GPB = BLK / 8;
#pragma unroll
      for (int t = 0; t < KN_BATCH; ++t) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const half8_t bq = unpack_q4(u.wv[t][c]);
#pragma unroll
          for (int v = 0; v < PER; ++v) {
            const half8_t bm = (g / GPB == v) ? bq : zh;
            const f32x4_t p = mfma(a[t], bm, f32x4_t{0.f, 0.f, 0.f, 0.f});
            acc[c] += biq::bitcast<float>(u.sc[t * PER + v][c]) * p;
          }
        }
      }
    }
  };

  // the two unit buffers in turn: the next unit's loads are issued before the current one computes
  while (kb < K) {
    load(kb + kstep, ub);
    compute(kb, ua);
    kb += kstep;
    if (kb >= K) break;
    load(kb + kstep, ua);
    compute(kb, ub);
    kb += kstep;
  }

  // 16x16 accumulator of MFMA c: lane holds column ncol + c, rows 4 g + r.  The partials of wave
  // w (row m of R = M rows, FOLD 2 M: hi rows then lo rows; column c of the slab) go to
  // red[(w * R + m) * 64 + c] over the staged activations.
  __syncthreads();
  float *red = reinterpret_cast<float *>(gv_lds);
  const int R = FOLD ? 2 * (int)M : (int)M;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int mr = 4 * g + r;
    const int m = FOLD ? (mr & 7) : mr;
    const int ri = FOLD ? (mr < 8 ? mr : (int)M + (mr - 8)) : mr;
    if (m < M) {
#pragma unroll
      for (int c = 0; c < 4; ++c) red[(w * R + ri) * KN_SLAB + 4 * c16 + c] = acc[c][r];
    }
  }
  __syncthreads();
  const int64_t col0 = slab * KN_SLAB;
  for (int o = threadIdx.x; o < M * KN_SLAB; o += 64 * WPS) {
    const int m = o / KN_SLAB, c = o % KN_SLAB;
    const int64_t n = col0 + c;
    if (n >= N) continue;
    float v = 0.0f;
#pragma unroll
    for (int ww = 0; ww < WPS; ++ww) {
      v += red[(ww * R + m) * KN_SLAB + c];
      if constexpr (FOLD) v += red[(ww * R + M + m) * KN_SLAB + c];
    }
    y[m * N + n] = v + (bias ? bias[n] : 0.0f);
  }
}

// Most waves per slab of q4_gemv_kn_lds_kernel whose registers fit without spilling (a 16-wave
// workgroup leaves a wave 128 VGPRs, 12 waves 168, 8 waves 256), from its compiled resource usage.
constexpr int gvl_max_wps(int blk) { return blk <= 16 ? 8 : blk == 32 ? 12 : 16; }

// ---------------------------------------------------------------- [N, K/8] words, [N, K/BLK] scales
// True when octet 4 g + c of a super-step lies in block j (blocks of opb octets) for some g.
constexpr bool nk_c_in_block(int c, int j, int opb) {
  return (c / opb == j) || ((4 + c) / opb == j) || ((8 + c) / opb == j) || ((12 + c) / opb == j);
}

template <int XD, int BLK, int WPS>
__global__ void __launch_bounds__(WPS > 1 ? 64 * WPS : GV_THREADS) q4_gemv_nk_kernel(
    const void *__restrict__ xv, int64_t ldx, const uint32_t *__restrict__ words,
    const float *__restrict__ scales, const float *__restrict__ bias, float *__restrict__ y,
    float *__restrict__ part, int64_t M, int64_t N, int64_t K, int64_t nchunks, int64_t nslabs,
    int64_t nunits) {
  const int lane = threadIdx.x & 63;
  int64_t slab, chunk;
  gv_unit<WPS>(nslabs, slab, chunk);
  if (WPS == 1 && slab + chunk * nslabs >= nunits) return;
  const int c16 = lane & 15, g = lane >> 4;
  const int64_t n = slab * NK_SLAB + c16;
  const int64_t KW = K / 8, nblk = K / BLK;
  const bool col_ok = n < N;
  const bool row_ok = c16 < M;
  const bool vec_words = (KW & 3) == 0;  // 16-byte aligned rows of words
  constexpr int ESZ = XD == BIQ_DTYPE_F32 ? 4 : 2;
  const char *xrow = reinterpret_cast<const char *>(xv) + (row_ok ? c16 : 0) * ldx * ESZ;
  const uint32_t *wrow = words + (col_ok ? n : 0) * KW;

  constexpr int OPB = BLK / 8;                     // octets per block
  constexpr int NBS = BLK >= 128 ? 1 : 128 / BLK;  // blocks per super-step
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};

  // K chunk c: the units of 128 * NK_BATCH k numbered c, c + nchunks, ... (interleaved)
  for (int64_t kb = chunk * 128 * NK_BATCH; kb < K; kb += nchunks * 128 * NK_BATCH) {
    uint32_t wv[NK_BATCH][4];
    XRaw<XD> xr[NK_BATCH][4];
    float sc[NK_BATCH][NBS];
#pragma unroll
    for (int t = 0; t < NK_BATCH; ++t) {
      const int64_t kw0 = (kb + 128 * t) / 8 + 4 * g;  // this lane's words: kw0 .. kw0 + 3
      if (col_ok && vec_words && kw0 < KW) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t *>(wrow + kw0);
#pragma unroll
        for (int c = 0; c < 4; ++c) wv[t][c] = v[c];
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) wv[t][c] = (col_ok && kw0 + c < KW) ? wrow[kw0 + c] : 0u;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
        load_x8<XD>(xr[t][c], xrow + ((kw0 + c) * 8) * ESZ, row_ok && kw0 + c < KW);
#pragma unroll
      for (int j = 0; j < NBS; ++j) {
        const int64_t b = (kb + 128 * t) / BLK + j;
        sc[t][j] = (col_ok && b < nblk) ? scales[n * nblk + b] : 0.0f;
      }
    }

#pragma unroll
    for (int t = 0; t < NK_BATCH; ++t) {
      half8_t ahi[4], alo[4], bq[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        x8_slots<XD>(xr[t][c], ahi[c], alo[c]);
        bq[c] = unpack_q4(wv[t][c]);
      }
      const half8_t zh = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < NBS; ++j) {
        f32x4_t p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (!nk_c_in_block(c, j, OPB)) continue;
          const half8_t bm = (OPB >= 16 || (4 * g + c) / OPB == j) ? bq[c] : zh;
          p = mfma_x<XD>(ahi[c], alo[c], bm, p);
        }
        acc += sc[t][j] * p;
      }
    }
  }

  // accumulator: lane holds column n, rows 4 g + r
  if constexpr (WPS > 1) {
    __shared__ float red[WPS * 16 * NK_SLAB];
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(w * 16 + 4 * g + r) * NK_SLAB + c16] = acc[r];
    __syncthreads();
    gv_reduce_lds<WPS, NK_SLAB>(red, bias, y, M, N, slab * NK_SLAB);
    return;
  }
  if (col_ok) {
    float *dst = part ? part + chunk * M * N : y;
    const float bn = (!part && bias) ? bias[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = 4 * g + r;
      if (m < M) dst[m * N + n] = acc[r] + bn;
    }
  }
}

}  // namespace

namespace biq {

// Small-M route of biq_q4_linear (f32 output).  Returns a BIQ_* status.
int q4_gemv_launch(hipStream_t s, const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                   const uint32_t *words, const float *scales, int layout, int block, int64_t N,
                   const float *bias, float *y, const Scratch *scr) {
  const bool kn = layout == BIQ_Q4_KN_AXIS1;
  const int64_t slab = kn ? KN_SLAB : NK_SLAB;
  const int64_t unit = kn ? 32 * KN_BATCH : 128 * NK_BATCH;  // a multiple of every block size
  const int64_t nslabs = (N + slab - 1) / slab;
  const int64_t kunits = (K + unit - 1) / unit;

  // [K/8, N] with up to 8 rows: activations staged in LDS, one workgroup per slab.  (With more
  // rows the staging of M x K activations per slab costs more than it saves: measured slower at
  // 16 x 3072 x 9216 than the in-register kernel below.)
  if (kn && M <= 8) {
    const int64_t xs_bytes = (K / 8) * M * (x_dtype == BIQ_DTYPE_F32 ? 32 : 16);
    const bool fold = x_dtype == BIQ_DTYPE_F32;  // lo parts in MFMA rows 8..15
    const int64_t max_wps = gvl_max_wps(block);
    // 8 waves per slab measured best (over 12 and 16: more units per wave to pipeline)
    const int64_t pref = max_wps < 8 ? max_wps : 8;
    int64_t wps = kunits >= pref ? pref : ((kunits + 3) / 4) * 4;
    // BIQ_GEMV_WPS (tuning): 4, 8, 12 or 16 waves per slab, read once per process
    static const int64_t forced_wps = [] {
      const char *e = std::getenv("BIQ_GEMV_WPS");
      return e ? (int64_t)std::atoll(e) : (int64_t)0;
    }();
    if ((forced_wps == 4 || forced_wps == 8 || forced_wps == 12 || forced_wps == 16) && forced_wps <= max_wps)
      wps = forced_wps;
    const int64_t red_bytes = wps * (fold ? 2 * M : M) * KN_SLAB * 4;
    const int64_t lds = xs_bytes > red_bytes ? xs_bytes : red_bytes;
    if (lds <= 160 * 1024 && nslabs <= 0x7fffffffLL) {
      const dim3 grid((unsigned)nslabs);
      hipError_t attr = hipSuccess;
#define BIQ_GVL_FN(fn)                                                                             \
  do {                                                                                             \
    if (lds > 64 * 1024)                                                                           \
      attr = hipFuncSetAttribute(reinterpret_cast<const void *>(fn),                               \
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);            \
    if (attr == hipSuccess)                                                                        \
      hipLaunchKernelGGL(fn, grid, dim3(64 * wps), (unsigned)lds, s, x, ldx, words, scales, bias, y, \
                         M, N, K);                                                                 \
  } while (0)
#define BIQ_GVL(XD, B, WPS)                                                                        \
  do {                                                                                             \
    if constexpr (WPS <= gvl_max_wps(B)) BIQ_GVL_FN((q4_gemv_kn_lds_kernel<XD, B, WPS>));         \
  } while (0)
#define BIQ_GVL_W(XD, B)                                                                           \
  switch (wps) {                                                                                   \
    case 4: BIQ_GVL(XD, B, 4); break;                                                              \
    case 8: BIQ_GVL(XD, B, 8); break;                                                              \
    case 12: BIQ_GVL(XD, B, 12); break;                                                            \
    default: BIQ_GVL(XD, B, 16); break;                                                            \
  }
#define BIQ_GVL_BLK(XD)                                                                           \
  switch (block) {                                                                                \
    case 8: BIQ_GVL_W(XD, 8); break;                                                               \
    case 16: BIQ_GVL_W(XD, 16); break;                                                             \
    case 32: BIQ_GVL_W(XD, 32); break;                                                             \
    case 64: BIQ_GVL_W(XD, 64); break;                                                             \
    default: BIQ_GVL_W(XD, 128); break;                                                            \
  }
      if (x_dtype == BIQ_DTYPE_BF16) { BIQ_GVL_BLK(BIQ_DTYPE_BF16) }
      else if (x_dtype == BIQ_DTYPE_F16) { BIQ_GVL_BLK(BIQ_DTYPE_F16) }
      else { BIQ_GVL_BLK(BIQ_DTYPE_F32) }
#undef BIQ_GVL_BLK
#undef BIQ_GVL_W
#undef BIQ_GVL
#undef BIQ_GVL_FN
      if (attr != hipSuccess)
        return fail(BIQ_ERR_HIP, std::string("q4 linear (small M): LDS attribute: ") + hipGetErrorString(attr));
      return check_launch("q4 linear (small M)");
    }
  }

  // In-workgroup mode: one workgroup per slab, its waves the K chunks (at most 16 -- 8 for blocks
  // of 8 or 16, whose decode needs more than the 128 registers a 1024-thread workgroup leaves --
  // and at least one unit each).  Taken when the slabs times the chunks give enough waves to
  // stream the weights.
  // (units of the in-register kernels from here on)
  const int64_t unit_r = kn ? 32 * kn_reg_batch(block) : unit;
  const int64_t kunits_r = (K + unit_r - 1) / unit_r;
  const int64_t max_wps = block <= 16 ? 8 : 16;
  int64_t wps_chunks = (kunits_r + max_wps - 1) / max_wps;      // units per chunk
  const int64_t nchunks_wg = (kunits_r + wps_chunks - 1) / wps_chunks;
  if (nslabs * nchunks_wg >= 1024 && nslabs <= 0x7fffffffLL) {
    const int wps = nchunks_wg <= 4 ? 4 : (nchunks_wg <= 8 ? 8 : (nchunks_wg <= 12 ? 12 : 16));
    const dim3 grid((unsigned)nslabs);
#define BIQ_GVW(XD, B, WPS)                                                                        \
  do {                                                                                             \
    if (kn)                                                                                        \
      hipLaunchKernelGGL((q4_gemv_kn_kernel<XD, B, WPS>), grid, dim3(64 * WPS), 0, s, x, ldx, words,\
                         scales, bias, y, nullptr, M, N, K, WPS, nslabs, nslabs * WPS);             \
    else                                                                                           \
      hipLaunchKernelGGL((q4_gemv_nk_kernel<XD, B, WPS>), grid, dim3(64 * WPS), 0, s, x, ldx, words,\
                         scales, bias, y, nullptr, M, N, K, WPS, nslabs, nslabs * WPS);             \
  } while (0)
#define BIQ_GVW_W(XD, B)                                                                           \
  switch (wps) {                                                                                   \
    case 4: BIQ_GVW(XD, B, 4); break;                                                              \
    case 8: BIQ_GVW(XD, B, 8); break;                                                              \
    case 12: if constexpr (B > 16) BIQ_GVW(XD, B, 12); break;                                      \
    default: if constexpr (B > 16) BIQ_GVW(XD, B, 16); break;                                      \
  }
#define BIQ_GVW_BLK(XD)                                                                           \
  switch (block) {                                                                                \
    case 8: BIQ_GVW_W(XD, 8); break;                                                               \
    case 16: BIQ_GVW_W(XD, 16); break;                                                             \
    case 32: BIQ_GVW_W(XD, 32); break;                                                             \
    case 64: BIQ_GVW_W(XD, 64); break;                                                             \
    default: BIQ_GVW_W(XD, 128); break;                                                            \
  }
    if (x_dtype == BIQ_DTYPE_BF16) { BIQ_GVW_BLK(BIQ_DTYPE_BF16) }
    else if (x_dtype == BIQ_DTYPE_F16) { BIQ_GVW_BLK(BIQ_DTYPE_F16) }
    else { BIQ_GVW_BLK(BIQ_DTYPE_F32) }
#undef BIQ_GVW_BLK
#undef BIQ_GVW_W
#undef BIQ_GVW
    return check_launch("q4 linear (small M)");
  }

  // Across workgroups: split K until about BIQ_GEMV_TARGET_WAVES waves stream the weights.
  int64_t ksplit = (BIQ_GEMV_TARGET_WAVES + nslabs - 1) / nslabs;
  if (ksplit > kunits_r) ksplit = kunits_r;
  if (ksplit < 1) ksplit = 1;
  // partial rows cost ksplit * M * N floats of workspace: keep them under 256 MB
  const int64_t max_split = (int64_t)(256 << 20) / (4 * M * N);
  if (ksplit > max_split) ksplit = max_split > 1 ? max_split : 1;
  const int64_t nunits = nslabs * ksplit;
  const int64_t wgs = (nunits + GV_THREADS / 64 - 1) / (GV_THREADS / 64);
  if (wgs > 0x7fffffffLL) return fail(BIQ_ERR_UNSUPPORTED, "q4 small-M route: too many work units");

  // several K chunks: partial rows into the stream's workspace, then an ordered reduction
  float *part = nullptr;
  if (ksplit > 1) {
    void *ws = nullptr;
    const int st = get_scratch(s, scr, (size_t)(ksplit * M * N) * sizeof(float), &ws);
    if (st != BIQ_OK) return st;
    part = reinterpret_cast<float *>(ws);
  }
  const dim3 grid((unsigned)wgs);
#define BIQ_GV(XD, B)                                                                              \
  do {                                                                                             \
    if (kn)                                                                                        \
      hipLaunchKernelGGL((q4_gemv_kn_kernel<XD, B, 1>), grid, dim3(GV_THREADS), 0, s, x, ldx, words,\
                         scales, bias, y, part, M, N, K, ksplit, nslabs, nunits);                  \
    else                                                                                           \
      hipLaunchKernelGGL((q4_gemv_nk_kernel<XD, B, 1>), grid, dim3(GV_THREADS), 0, s, x, ldx, words,\
                         scales, bias, y, part, M, N, K, ksplit, nslabs, nunits);                  \
  } while (0)
#define BIQ_GV_BLK(XD)                                                                            \
  switch (block) {                                                                                \
    case 8: BIQ_GV(XD, 8); break;                                                                  \
    case 16: BIQ_GV(XD, 16); break;                                                                \
    case 32: BIQ_GV(XD, 32); break;                                                                \
    case 64: BIQ_GV(XD, 64); break;                                                                \
    default: BIQ_GV(XD, 128); break;                                                               \
  }
  if (x_dtype == BIQ_DTYPE_BF16) { BIQ_GV_BLK(BIQ_DTYPE_BF16) }
  else if (x_dtype == BIQ_DTYPE_F16) { BIQ_GV_BLK(BIQ_DTYPE_F16) }
  else { BIQ_GV_BLK(BIQ_DTYPE_F32) }
  if (part) {
    const int64_t threads = M * N / 4;
    hipLaunchKernelGGL(gv_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, part,
                       ksplit, bias, y, M, N);
  }
#undef BIQ_GV_BLK
#undef BIQ_GV
  return check_launch("q4 linear (small M)");
}

}  // namespace biq
