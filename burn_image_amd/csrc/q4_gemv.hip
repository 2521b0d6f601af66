// Small-M packed-Q4 projection (M <= 16) for gfx950: an HBM-bound streaming kernel.
//
// The same operator as q4_gemm.hip (y = x . W + bias, exact nibbles, f32 block scales) for the
// reference's small-row callers: the RmsNormZero modulation projection (one conditioning row,
// crates/burn_boogu/src/model/norm.rs:138-153) and short instruction streams.  With a 128-row
// tile those calls would waste the matrix cores and launch only N / 256 workgroups.
//
// Work unit: one wave owns a column slab over one K chunk.  Waves are numbered slab-fastest, so
// neighbouring waves read neighbouring columns of the same packed rows.  Nothing is staged in
// LDS and there is no barrier: a wave issues the loads of a whole batch (words, activations and
// scales) before its first MFMA, and enough waves are resident to keep HBM busy.
//
// MFMA: v_mfma_f32_16x16x32_f16.  A = the (<= 16) activation rows, converted to f16 in the
// nibble slot order [k0,k4,k1,k5,k2,k6,k3,k7] (f32 activations as hi + lo, two MFMAs); B = the
// packed words decoded exactly to f16 (the q4_gemm.hip decode).  The k order inside one MFMA is
// free as long as A and B agree; the two layouts use that freedom differently:
//  * [K/8, N] words: lane (c16 = l % 16, g = l / 16) loads 16 bytes = the words of columns
//    4 c16 .. 4 c16 + 3 in packed row k0/8 + g.  MFMA c contracts column 4 c16 + c over the 32 k
//    of the step, so a wave reads 64 columns x 32 k (4 x 256 contiguous bytes) per step.
//  * [N, K/8] words: lane (c16, g) loads 16 bytes = 4 consecutive words of column c16; MFMA c
//    contracts octet 4 g + c of a 128-k super-step, so a wave reads 16 columns x 128 k.
// Each K block's partial is scaled by its f32 scale in f32 (the scale is never rounded); where a
// block is shorter than one MFMA's k, the MFMA is repeated with the other blocks' lanes masked.
// With several K chunks each wave stores its partial rows into a per-stream workspace and a
// second kernel adds the chunks in order plus the bias, so results are deterministic (device-wide
// f32 atomics were measured far slower than these plain stores).
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
template <int XD, int BLK>
__global__ void __launch_bounds__(GV_THREADS) q4_gemv_kn_kernel(
    const void *__restrict__ xv, int64_t ldx, const uint32_t *__restrict__ words,
    const float *__restrict__ scales, const float *__restrict__ bias, float *__restrict__ y,
    float *__restrict__ part, int64_t M, int64_t N, int64_t K, int64_t kchunk, int64_t nslabs,
    int64_t nunits) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * (GV_THREADS / 64) + (threadIdx.x >> 6);
  if (wid >= nunits) return;
  const int c16 = lane & 15, g = lane >> 4;
  const int64_t ncol = (wid % nslabs) * KN_SLAB + 4 * c16;  // columns ncol .. ncol + 3
  const int64_t kbeg = (wid / nslabs) * kchunk;              // a multiple of 128 (every block)
  const int64_t kend = kbeg + kchunk < K ? kbeg + kchunk : K;
  const int64_t KW = K / 8, nblk = K / BLK;
  const bool col_ok = ncol < N;
  const bool row_ok = c16 < M;
  constexpr int ESZ = XD == BIQ_DTYPE_F32 ? 4 : 2;
  const char *xrow = reinterpret_cast<const char *>(xv) + (row_ok ? c16 : 0) * ldx * ESZ;

  f32x4_t acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  constexpr int SPB = BLK >= 32 ? BLK / 32 : 1;                                        // steps per block
  constexpr int NSC = BLK >= 32 ? (KN_BATCH + SPB - 1) / SPB : KN_BATCH * (32 / BLK);  // blocks per batch

  for (int64_t kb = kbeg; kb < kend; kb += 32 * KN_BATCH) {
    u32x4_t wv[KN_BATCH];
    XRaw<XD> xr[KN_BATCH];
#pragma unroll
    for (int t = 0; t < KN_BATCH; ++t) {
      const int64_t kw = (kb + 32 * t) / 8 + g;  // packed row of lane group g in step t
      wv[t] = u32x4_t{0u, 0u, 0u, 0u};
      if (col_ok && kw < KW) wv[t] = *reinterpret_cast<const u32x4_t *>(words + kw * N + ncol);
      load_x8<XD>(xr[t], xrow + (kw * 8) * ESZ, row_ok && kw < KW);
    }
    float sc[NSC][4];
#pragma unroll
    for (int j = 0; j < NSC; ++j) {
      const int64_t b = kb / BLK + j;
#pragma unroll
      for (int c = 0; c < 4; ++c) sc[j][c] = (col_ok && b < nblk) ? scales[b * N + ncol + c] : 0.0f;
    }

    if constexpr (BLK >= 32) {
      f32x4_t p[4];
#pragma unroll
      for (int t = 0; t < KN_BATCH; ++t) {
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
      for (int t = 0; t < KN_BATCH; ++t) {
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

  // 16x16 accumulator of MFMA c: lane holds column ncol + c, rows 4 g + r.  One K chunk: y =
  // acc + bias; several: this chunk's partial rows.
  if (col_ok) {
    float *dst = part ? part + (wid / nslabs) * M * N : y;
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

// ---------------------------------------------------------------- [N, K/8] words, [N, K/BLK] scales
// True when octet 4 g + c of a super-step lies in block j (blocks of opb octets) for some g.
constexpr bool nk_c_in_block(int c, int j, int opb) {
  return (c / opb == j) || ((4 + c) / opb == j) || ((8 + c) / opb == j) || ((12 + c) / opb == j);
}

template <int XD, int BLK>
__global__ void __launch_bounds__(GV_THREADS) q4_gemv_nk_kernel(
    const void *__restrict__ xv, int64_t ldx, const uint32_t *__restrict__ words,
    const float *__restrict__ scales, const float *__restrict__ bias, float *__restrict__ y,
    float *__restrict__ part, int64_t M, int64_t N, int64_t K, int64_t kchunk, int64_t nslabs,
    int64_t nunits) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * (GV_THREADS / 64) + (threadIdx.x >> 6);
  if (wid >= nunits) return;
  const int c16 = lane & 15, g = lane >> 4;
  const int64_t n = (wid % nslabs) * NK_SLAB + c16;
  const int64_t kbeg = (wid / nslabs) * kchunk;  // a multiple of 256 (every block)
  const int64_t kend = kbeg + kchunk < K ? kbeg + kchunk : K;
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

  for (int64_t kb = kbeg; kb < kend; kb += 128 * NK_BATCH) {
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
  if (col_ok) {
    float *dst = part ? part + (wid / nslabs) * M * N : y;
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
  // Split K until about BIQ_GEMV_TARGET_WAVES waves stream the weights (one resident round).
  const int64_t kunits = (K + unit - 1) / unit;
  int64_t ksplit = (BIQ_GEMV_TARGET_WAVES + nslabs - 1) / nslabs;
  if (ksplit > kunits) ksplit = kunits;
  if (ksplit < 1) ksplit = 1;
  // partial rows cost ksplit * M * N floats of workspace: keep them under 256 MB
  const int64_t max_split = (int64_t)(256 << 20) / (4 * M * N);
  if (ksplit > max_split) ksplit = max_split > 1 ? max_split : 1;
  const int64_t kchunk = ((kunits + ksplit - 1) / ksplit) * unit;
  ksplit = (K + kchunk - 1) / kchunk;
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
      hipLaunchKernelGGL((q4_gemv_kn_kernel<XD, B>), grid, dim3(GV_THREADS), 0, s, x, ldx, words,  \
                         scales, bias, y, part, M, N, K, kchunk, nslabs, nunits);                  \
    else                                                                                           \
      hipLaunchKernelGGL((q4_gemv_nk_kernel<XD, B>), grid, dim3(GV_THREADS), 0, s, x, ldx, words,  \
                         scales, bias, y, part, M, N, K, kchunk, nslabs, nunits);                  \
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
