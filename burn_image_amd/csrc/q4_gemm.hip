// Packed signed-Q4 projection GEMM for gfx950: y[M, N] = x[M, K] . W (+ bias).
//
// Replaces the quantized CMMA matmul behind QTensorOps::q_matmul
// (patches/burn-cubecl-0.21.0/src/ops/qtensor.rs:303-368, kernel/matmul/quantized.rs:35-60).
//
// Arithmetic (exact where it matters for the f32-result parity gate):
//  * Each packed word holds 8 consecutive k of one column n.  A lane of v_mfma_f32_32x32x16_f16's
//    B operand holds exactly 8 consecutive k of one column, so one word feeds one lane-operand.
//  * Nibbles decode to EXACT f16 integers: (0x6400 | (v ^ 8)) is 1024 + q + 8 in f16, and one
//    v_pk_add_f16 of -1032 leaves q in [-8, 7].  The word is split as (k0,k4),(k1,k5),(k2,k6),
//    (k3,k7) pairs, so B slots carry k in the order [0,4,1,5,2,6,3,7]; the activations are written
//    to LDS in the same order, which leaves every product x[k] * q[k] paired correctly.
//  * Activations enter as f16: bf16 -> f16 is exact for |x| >= 2^-14 (the reference itself stages
//    f16, kernel/matmul/quantized.rs:172-178); f32 activations are split into f16 hi + lo
//    (x - hi rounded again), two MFMAs, leaving a 2^-22 relative residual.
//  * Products are exact in the f32 accumulator.  Each K-block's partial sum is kept in its own
//    accumulator and added to the output accumulator as acc += scale[b, n] * partial in f32,
//    so the f32 block scale is never rounded to 16 bits.
//
// Schedule: 512 threads = 8 waves (2 per SIMD) in a 2 (M) x 4 (N) grid; workgroup tile
// 128 x 256, wave tile 64 x 64 (2 x 2 MFMA 32 x 32 tiles); K advances 128 per tile (64 for f32
// activations and blocks <= 16).  While the waves run the MFMAs of tile t from one LDS buffer,
// the threads hold the global loads (activations, packed words, block scales) of the next one or
// two tiles in registers; tile t+1 is converted and stored into the other LDS buffer during
// tile t, so one barrier per tile separates the two.  Workgroups are numbered so that each XCD
// (hardware places workgroup i on XCD i % 8) walks a compact, M-grouped block of output tiles,
// keeping the shared activation and weight tiles in its L2.  When the tiles leave the last
// round of workgroups mostly idle, the tail tiles are split along K (SkPlan below).
#include <stdlib.h>

#include <type_traits>

#include "common.h"

namespace {

// M tiles per raster group (measured on the 4608-row projections against 2, 3, 6, 8 and 16: 4 and
// 2 lead 8 by 0.3-1%, 16 trails)
constexpr int GROUP_M = 4;

enum XMode { XM_F16 = 0, XM_BF16 = 1, XM_F32 = 2 };

// Eight signed nibbles -> eight exact f16 integers in slot order [k0,k4,k1,k5,k2,k6,k3,k7].
// Nibbles i and i + 4 sit at bits 4i and 16 + 4i.  The even pairs (bits 0-3 / 16-19 of w and of
// w >> 8) become 0x6400 | (v ^ 8) = 1024 + q + 8; the odd pairs are used in place, at bits 4-7 /
// 20-23, as 0x6400 | (v ^ 8) << 4 = 1024 + 16 (q + 8) and scaled by 1/16 in the same packed FMA
// that removes the offset.  Every intermediate is an exact f16, so q in [-8, 7] is exact, and
// one shift serves all eight nibbles.
__device__ __forceinline__ half8_t unpack_q4_f16(uint32_t w) {
  const uint32_t M0 = 0x000F000Fu, C0 = 0x64086408u;  // low nibble of each half, sign-flip bit 3
  const uint32_t M1 = 0x00F000F0u, C1 = 0x64806480u;  // high nibble of each half, sign-flip bit 7
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

// 8 bf16 -> 8 f16 in slot order [0,4,1,5,2,6,3,7].
__device__ __forceinline__ u32x4_t bf16x8_to_f16_slots(u32x4_t v) {
  u32x4_t r;
  r[0] = biq::pack_f16x2(biq::bf16_lo_to_f32(v[0]), biq::bf16_lo_to_f32(v[2]));
  r[1] = biq::pack_f16x2(biq::bf16_hi_to_f32(v[0]), biq::bf16_hi_to_f32(v[2]));
  r[2] = biq::pack_f16x2(biq::bf16_lo_to_f32(v[1]), biq::bf16_lo_to_f32(v[3]));
  r[3] = biq::pack_f16x2(biq::bf16_hi_to_f32(v[1]), biq::bf16_hi_to_f32(v[3]));
  return r;
}

// 8 f16 -> slot order [0,4,1,5,2,6,3,7]: one byte permute per output word (v_perm_b32 picks
// bytes 0-3 from its second operand and 4-7 from its first).
__device__ __forceinline__ u32x4_t f16x8_to_slots(u32x4_t v) {
  u32x4_t r;
  r[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);  // (v0.lo, v2.lo)
  r[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);  // (v0.hi, v2.hi)
  r[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
  r[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
  return r;
}

// 8 f32 -> (hi, lo) f16 slots, x = hi + lo to within 2^-22 relative.
__device__ __forceinline__ void f32x8_to_f16_split_slots(const float4 &a, const float4 &b,
                                                         u32x4_t &hi, u32x4_t &lo) {
  float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  _Float16 h[8];
  float l[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    h[i] = (_Float16)x[i];
    l[i] = x[i] - (float)h[i];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    half2_t hh = {h[i], h[i + 4]};
    hi[i] = biq::bitcast<uint32_t>(hh);
    lo[i] = biq::pack_f16x2(l[i], l[i + 4]);
  }
}

// Tile geometry: a wave owns WM x WN MFMA tiles of 32 x 32; the workgroup holds WAVES_M x WAVES_N
// waves.  RESCALE selects how block scales are applied (see the kernel): false keeps each block's
// partial sum in its own accumulator and adds scale * partial at the block's end; true rescales
// the running accumulator at each block boundary, which halves the accumulator registers and so
// leaves room for the 128-row wave tile.
template <int WM_, int WN_, int WAVES_M_, int WAVES_N_, int BK_, bool RESCALE_ = false>
struct Geo {
  static constexpr int WM = WM_, WN = WN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr bool RESCALE = RESCALE_;
  static constexpr int BK = BK_;        // K per LDS stage
  static constexpr int A_LD = BK + 8;   // LDS row stride of the activation tile, in halves
  static constexpr int BM = 32 * WM * WAVES_M, BN = 32 * WN * WAVES_N;
  static constexpr int NTHREADS = 64 * WAVES_M * WAVES_N;
  static constexpr int A_CHUNKS = (BM * BK / 8) / NTHREADS;  // 8-element groups per thread
  static constexpr int B_CHUNKS = (BK / 8) * (BN / 4) / NTHREADS;  // 4-word groups per thread
  static_assert(A_CHUNKS * NTHREADS == BM * BK / 8, "activation tile split");
  static_assert(B_CHUNKS * NTHREADS == (BK / 8) * (BN / 4), "word tile split");
};

// Workgroup shape: 8 waves (2 per SIMD) in a 2 x 4 grid of 64 x 64 wave tiles -> 128 x 256.
// 16-bit activations stage K 128 at a time (more bytes in flight per prefetch); the f32 hi/lo
// path keeps 64 so that its two activation planes fit the 160 KB LDS, and blocks of 8 or 16 keep
// 64 so that their per-tile scale lists stay in registers.
#ifndef BIQ_GEMM_WAVES
#define BIQ_GEMM_WAVES 2, 2, 2, 4
#endif
#ifndef BIQ_GEMM_BK
#define BIQ_GEMM_BK 128
#endif
template <int XMODE, int BLK>
using GemmGeo = Geo<BIQ_GEMM_WAVES, (XMODE == XM_F32 || BLK <= 16) ? 64 : BIQ_GEMM_BK>;
// Large workgroup tile for 16-bit activations and blocks >= 32: 8 waves in a 2 x 4 grid of
// 128 x 64 wave tiles -> 256 x 256, K staged 64 at a time (two 45 KB LDS buffers).  A decoded
// weight fragment feeds four MFMAs instead of two and each staged activation / weight byte serves
// twice the output of the 128 x 256 tile; block scales use the running rescale.  Measured
// against 128 x 256 at 4608 rows: 3072x3072 -8%, 3072x12288 -3%, 12288x3072 -5% time, 3072x9216
// level (648 tiles leave the last of three rounds half idle) -- launch_blk picks per shape.
using GemmGeoBig = Geo<4, 2, 2, 4, 64, true>;

// Register sets of the global -> LDS pipeline (see the kernel): two for 16-bit activations,
// blocks of 128 and the [K/8, N] word layout; one where a second set would not fit the 256
// registers without spilling.
// The large tile keeps one set (a second does not fit its registers).
template <class G, int LAYOUT, int XMODE, int BLK>
constexpr int PF_SETS = (!G::RESCALE && LAYOUT == BIQ_Q4_KN_AXIS1 && XMODE != XM_F32 && BLK >= 128) ? 2 : 1;
// K units a tail part starts on a multiple of (see the kernel's paired loop)
template <class G, int LAYOUT, int XMODE, int BLK>
constexpr int PART_GRANULE = (PF_SETS<G, LAYOUT, XMODE, BLK> == 2 && BLK <= G::BK) ? 2 : 1;

// Running-rescale form: block scales enter as t = s with |t| clamped to [2^-60, 2^60], so that
// the ratio of two consecutive scales stays finite.  Scales the importer writes (max|w| / 7, or
// f32::MIN_POSITIVE for an all-zero block, whose nibbles are all zero) are exact up to the clamp;
// a block of zero scale contributes q * 2^-60 * x instead of 0.  NaN stays NaN.
__device__ __forceinline__ float clamp_scale(float s) {
  const float a = fabsf(s);
  const float c = a < 0x1p-60f ? 0x1p-60f : (a > 0x1p60f ? 0x1p60f : a);
  return (a != a) ? s : (s < 0.0f ? -c : c);
}

// Per-thread register copy of one tile's global data.
template <class G, int XMODE, int NSC>
struct TileRegs {
  u32x4_t a16[XMODE == XM_F32 ? 1 : G::A_CHUNKS];
  float4 a32[XMODE == XM_F32 ? 2 * G::A_CHUNKS : 1];
  u32x4_t b[G::B_CHUNKS];
  float sc[G::WN][NSC];  // block scales of this thread's columns
};

// Work split of one launch.  Workgroups [0, dp_tiles) each own one whole output tile (in the
// XCD-aware order below).  When whole-tile rounds would leave the last round mostly idle, the
// remaining tail tiles are split along K into `parts` equal runs of K units (one unit = the K of
// one outer iteration, whole quantisation blocks): chunk c is part c / tail of tail tile
// c % tail, and tail workgroup w computes chunks w, w + sk_wgs, ...  All chunks in flight at a
// time then cover the same K range of neighbouring tiles (the activation and weight tiles they
// read are shared in L2, as for owned tiles).  A chunk writes its partial accumulators to slot c
// of `part`; a second kernel (q4_tail_reduce_kernel) adds each tile's partials in K order and
// applies the epilogue, so the result does not depend on which chunk finished first.
struct SkPlan {
  int dp_tiles;
  int sk_wgs;     // 0: every tile is owned
  int parts;      // K parts of a tail tile
  int64_t units;  // K units per tile
  float *part;    // (tiles - dp_tiles) * parts partial tiles of BM x BN f32, register-major
};

// pid -> output tile: M-grouped raster (GROUP_M M tiles per group, walked column by column).
// (32-bit: tile counts stay below 2^31, host check; 64-bit divisions are long scalar sequences
// that every wave of the workgroup would run)
__device__ __forceinline__ void tile_coords(uint32_t pid, uint32_t tiles_m, uint32_t tiles_n,
                                            int64_t &tile_m, int64_t &tile_n) {
  const uint32_t in_group = (uint32_t)GROUP_M * tiles_n;
  const uint32_t rem = pid % in_group;
  const uint32_t first_m = (pid / in_group) * GROUP_M;
  const uint32_t gsize = (tiles_m - first_m) < (uint32_t)GROUP_M ? (tiles_m - first_m) : (uint32_t)GROUP_M;
  tile_m = first_m + rem % gsize;
  tile_n = rem / gsize;
}

// Epilogue of one wave's accumulators: bias (or the SwiGLU gate), conversion, store.  Register r
// of MFMA tile (i, j) holds row 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4 and column
// 32 j + lane % 32 of the wave tile.
template <class G, bool GLU>
__device__ __forceinline__ void store_tile_out(const floatx16_t (&acc)[G::WM][G::WN], int64_t m0,
                                               int64_t n0, const float *__restrict__ bias,
                                               void *__restrict__ yv, int y_dtype, int64_t M,
                                               int64_t N) {
  constexpr int WM = G::WM, WN = G::WN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
  const int l32 = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int j = 0; j < (GLU ? 1 : WN); ++j) {
    const int64_t col = GLU ? n0 + wn * 32 + l32 : n0 + wn * (32 * WN) + 32 * j + l32;
    if (col >= N) continue;
    const float bv = (!GLU && bias) ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * (32 * WM) + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (row >= M) continue;
        float v = acc[i][j][r] + bv;
        if constexpr (GLU) {
          // silu(a) = a / (1 + e^-a), times the W3 projection of the same row and column
          v = v / (1.0f + __expf(-v)) * acc[i][1][r];
        }
        if (y_dtype == BIQ_DTYPE_F32) {
          reinterpret_cast<float *>(yv)[row * N + col] = v;
        } else if (y_dtype == BIQ_DTYPE_F16) {
          reinterpret_cast<_Float16 *>(yv)[row * N + col] = biq::f16_of_f32(v);
        } else {
          reinterpret_cast<uint16_t *>(yv)[row * N + col] = (uint16_t)biq::f32_to_bf16_bits(v);
        }
      }
  }
}

// The same epilogue without a branch per element: the output type is a template argument, and
// each store goes through a buffer descriptor based at the wave's tile corner, with the row of the
// register in the scalar offset and the lane's own row / column in the vector offset; an element
// past M or N gets an out-of-range vector offset, so the hardware drops its store.  Used when
// 32 WM rows of the output span less than 2^31 bytes (the offsets are 32-bit).
template <class G, bool GLU, typename OT>
__device__ __forceinline__ void store_tile_out_rows(const floatx16_t (&acc)[G::WM][G::WN], int64_t m0,
                                                    int64_t n0, const float *__restrict__ bias,
                                                    void *__restrict__ yv, int64_t M, int64_t N) {
  constexpr int WM = G::WM, WN = G::WN;
  constexpr uint32_t OOB = 0x80000000u;
  constexpr uint32_t OSZ = sizeof(OT);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
  const int l32 = lane & 31, lh = lane >> 5;
  const int64_t r0 = m0 + wm * (32 * WM);
  const int64_t c0 = GLU ? n0 + wn * 32 : n0 + wn * (32 * WN);
  const int64_t rows_left = M - r0, cols_left = N - c0;
  OT *base = reinterpret_cast<OT *>(yv) + (r0 < M ? r0 : 0) * N + (c0 < N ? c0 : 0);
  const int64_t bytes = (rows_left > 0 && cols_left > 0) ? ((rows_left - 1) * N + cols_left) * (int64_t)OSZ : 0;
  const uint32_t n_rec = bytes > 0x7fffffffLL ? 0x7fffffffu : (uint32_t)bytes;
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)n_rec, 0x00020000);
  const int64_t lim = rows_left - 4 * lh;  // register rows u (without 4 lh) below lim are inside M
  const uint32_t row_bytes = (uint32_t)N * OSZ;
#pragma unroll
  for (int j = 0; j < (GLU ? 1 : WN); ++j) {
    const int cl = GLU ? l32 : 32 * j + l32;  // column of the lane from c0
    const bool col_ok = cl < cols_left;
    const float bv = (!GLU && bias && col_ok) ? bias[c0 + cl] : 0.0f;
    const uint32_t vo = col_ok ? (uint32_t)(4 * lh) * row_bytes + (uint32_t)cl * OSZ : OOB;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int u = 32 * i + 8 * (r >> 2) + (r & 3);
        float v = acc[i][j][r] + bv;
        if constexpr (GLU) {
          // silu(a) = a / (1 + e^-a), times the W3 projection of the same row and column
          v = v / (1.0f + __expf(-v)) * acc[i][1][r];
        }
        const uint32_t o = u < lim ? vo : OOB;
        const uint32_t so = (uint32_t)u * row_bytes;
        if constexpr (sizeof(OT) == 4) {
          __builtin_amdgcn_raw_buffer_store_b32(biq::bitcast<uint32_t>(v), rs, o, so, 0);
        } else if constexpr (std::is_same<OT, uint16_t>::value) {  // bf16 bits
          __builtin_amdgcn_raw_buffer_store_b16((uint16_t)biq::f32_to_bf16_bits(v), rs, o, so, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b16(biq::bitcast<uint16_t>(biq::f16_of_f32(v)), rs, o, so, 0);
        }
      }
  }
}

// Fused self-attention projection epilogue (biq_q4_linear_qk_norm_rope).  The output columns are
// Hq + 2 Hkv heads of 128 (q heads, then k heads, then v heads); a 256 x 256 workgroup tile holds
// two whole heads.  Per (token, q or k head), in the order of the fused preparation kernel for
// f32 input (qk_prep.hip): rms = sqrt(sum x^2 / 128 + eps), n = (x / rms) * gamma (the quotient
// correctly rounded from 1 / rms by one residual step, biq::div_rn), interleaved RoPE
// y_2p = n_2p cos - n_2p+1 sin, y_2p+1 = n_2p+1 cos + n_2p sin, each product and sum rounded in
// f32; then the cast.  v heads are only cast.  Outputs are contiguous [B, S, H, 128] or
// [B, H, S, 128].  Only the sum of squares is added in another order than the preparation
// kernel's.
struct QkEpi {
  const float *q_gamma, *k_gamma, *cos, *sin;
  void *qo, *ko, *vo;
  int64_t S, Hq, Hkv;
  int rope_per_batch;  // 1: cos / sin rows per (batch, token) = per output row; 0: per token
  int out_bf16;
  int head_major;      // outputs [B, H, S, 128] instead of [B, S, H, 128]
  float q_eps, k_eps;
};

// Each MFMA tile row i (32 rows of every wave) passes through LDS as four (row block, head)
// groups of 32 rows x 128 columns; thread t then owns 16 consecutive columns (t % 8) of one
// (row, head) of a group: the row's sum of squares is a 16-term sum plus three lane exchanges,
// RoPE pairs sit in one thread, and cos / sin / gamma / outputs move as 16-byte vectors.  Waves
// 0-3 take the tile's first head and waves 4-7 its second, in both passes of every i.
constexpr int QK_LD = 132;  // LDS row stride of a group, in floats
template <class G>
__device__ __forceinline__ void qk_epilogue(const floatx16_t (&acc)[G::WM][G::WN], int64_t m0,
                                            int64_t n0, int64_t M, const QkEpi &e,
                                            float *__restrict__ lds) {
#pragma clang fp contract(off)
  static_assert(G::WM == 4 && G::WN == 2 && G::WAVES_M == 2 && G::WAVES_N == 4 && G::NTHREADS == 512,
                "two 128-column heads per 256 x 256 tile");
  constexpr int D = 128;
  constexpr uint32_t OOB = 0x80000000u;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
  const int l32 = lane & 31, lh = lane >> 5;
  // writer side: this wave's 32 x 64 piece of group (wm, wn / 2) at columns (wn % 2) * 64
  float *wr = lds + (wm * 2 + (wn >> 1)) * 32 * QK_LD + (wn & 1) * 64 + l32;
  // reader side: head hh of the tile, chunk k (columns 16 k .. 16 k + 15)
  const int hh = wave >> 2, k = tid & 7;
  const int64_t head = n0 / D + hh;  // wave-uniform
  const int64_t Hq = e.Hq, Hkv = e.Hkv;
  const int kind = head < Hq ? 0 : (head < Hq + Hkv ? 1 : (head < Hq + 2 * Hkv ? 2 : 3));
  const int64_t H = kind == 0 ? Hq : Hkv;
  const int64_t hk = head - (kind == 0 ? 0 : (kind == 1 ? Hq : Hq + Hkv));
  float gm[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) gm[c] = 0.0f;
  if (kind < 2) {
    const float4 *gp = reinterpret_cast<const float4 *>((kind == 0 ? e.q_gamma : e.k_gamma) + 16 * k);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 v = gp[c];
      gm[4 * c] = v.x; gm[4 * c + 1] = v.y; gm[4 * c + 2] = v.z; gm[4 * c + 3] = v.w;
    }
  }
  const float eps = kind == 0 ? e.q_eps : e.k_eps;
  const uint32_t S = (uint32_t)e.S;
  auto rsrc = [](const void *base, int64_t bytes) {
    const uint32_t n = bytes > 0x7fffffffLL ? 0x7fffffffu : (bytes < 0 ? 0u : (uint32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)n, 0x00020000);
  };
  const int64_t table_rows = e.rope_per_batch ? M : e.S;
  const auto cs_rs = rsrc(e.cos, table_rows * D * 4), sn_rs = rsrc(e.sin, table_rows * D * 4);
  u32x4_t packed[4][2][2];  // (i, pass): the thread's 16 outputs as 16-bit pairs

#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        wr[(8 * (r >> 2) + 4 * lh + (r & 3)) * QK_LD + 32 * j] = acc[i][j][r];
    __syncthreads();
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const int rr = (tid >> 3) & 31;                // row of the group
      const int g = 2 * ps + hh;                     // group: row block ps, head hh
      const int64_t row = m0 + ps * 128 + 32 * i + rr;
      float x[16];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 v = reinterpret_cast<const float4 *>(lds + (g * 32 + rr) * QK_LD + 16 * k)[c];
        x[4 * c] = v.x; x[4 * c + 1] = v.y; x[4 * c + 2] = v.z; x[4 * c + 3] = v.w;
      }
      float y[16];
      if (kind < 2) {
        const uint32_t trow = e.rope_per_batch ? (uint32_t)(row < M ? row : M - 1) : (uint32_t)(row % (int64_t)S);
        const uint32_t to = (trow * (uint32_t)D + 16u * k) * 4u;
        float cs[16], sn[16];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(cs_rs, to + 16u * c, 0, 0);
          const u32x4_t b = __builtin_amdgcn_raw_buffer_load_b128(sn_rs, to + 16u * c, 0, 0);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            cs[4 * c + t] = biq::bitcast<float>(a[t]);
            sn[4 * c + t] = biq::bitcast<float>(b[t]);
          }
        }
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < 16; ++c) ss = ss + x[c] * x[c];
        // the eight threads of the row add their sums pairwise: every one ends with the same total
        ss = ss + __shfl_xor(ss, 1);
        ss = ss + __shfl_xor(ss, 2);
        ss = ss + __shfl_xor(ss, 4);
        const float2 dv = biq::rn_divisor(sqrtf(ss / (float)D + eps));
        float n[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) n[c] = biq::div_rn(x[c], dv.x, dv.y) * gm[c];
#pragma unroll
        for (int c = 0; c < 16; c += 2) {
          y[c] = (n[c] * cs[c]) + ((-n[c + 1]) * sn[c]);
          y[c + 1] = (n[c + 1] * cs[c + 1]) + (n[c] * sn[c + 1]);
        }
      } else {
#pragma unroll
        for (int c = 0; c < 16; ++c) y[c] = x[c];
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t w = e.out_bf16 ? biq::pack_bf16x2(y[2 * c], y[2 * c + 1])
                                      : biq::pack_f16x2(y[2 * c], y[2 * c + 1]);
        packed[i][ps][c >> 2][c & 3] = w;
      }
    }
    __syncthreads();  // the next i rewrites the groups
  }
  if (kind == 3) return;  // columns past N (the last tile of an odd head count)
  // stores: (row, head hk) chunk k = 32 bytes; rows past M take an out-of-range offset.  Element
  // (row = b S + s, hk, d) sits at (row H + hk) D + d, or head-major at ((b H + hk) S + s) D + d
  // = (row + b (H - 1) S + hk S) D + d.
  uint16_t *out = reinterpret_cast<uint16_t *>(kind == 0 ? e.qo : (kind == 1 ? e.ko : e.vo)) + 16 * k;
  const auto out_rs = rsrc(out, (M * H * D - 16 * k) * 2);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const int64_t row = m0 + ps * 128 + 32 * i + ((tid >> 3) & 31);
      uint32_t el;  // element offset of the (row, head) from `out`
      if (e.head_major) {
        const uint32_t b = (uint32_t)row / S;
        el = ((uint32_t)row + b * (uint32_t)((H - 1) * e.S) + (uint32_t)(hk * e.S)) * (uint32_t)D;
      } else {
        el = ((uint32_t)row * (uint32_t)H + (uint32_t)hk) * (uint32_t)D;
      }
      const uint32_t o = row < M ? el * 2u : OOB;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        __builtin_amdgcn_raw_buffer_store_b128(packed[i][ps][h], out_rs, o + 16u * h, 0, 0);
    }
}

// Tail reduction.  One thread takes one output register q of four consecutive source threads
// of one tail tile (one 16-byte load per part, coalesced), adds the `parts` partials in K order
// and writes the four outputs: same rows and columns, bias and SwiGLU gate as the GEMM epilogue
// (store_tile_out) would have used for those registers.
constexpr int RED_THREADS = 256;
template <class G, bool GLU>
__global__ void __launch_bounds__(RED_THREADS)
    q4_tail_reduce_kernel(const float *__restrict__ part, int tail, int parts, int dp_tiles,
                          int tiles_m, int tiles_n, const float *__restrict__ bias,
                          void *__restrict__ yv, int y_dtype, int64_t M, int64_t N) {
  constexpr int WM = G::WM, WN = G::WN, NT = G::NTHREADS, PART = G::BM * G::BN;
  constexpr int BNO = GLU ? G::BN / 2 : G::BN;
  constexpr int QN = GLU ? WM * 16 : WM * WN * 16;  // output registers per source thread
  const int64_t per_tile = (int64_t)QN * (NT / 4);
  const int64_t gid = (int64_t)blockIdx.x * RED_THREADS + threadIdx.x;
  const int64_t t = gid / per_tile;
  if (t >= tail) return;
  const int rem = (int)(gid % per_tile);
  const int qo = rem / (NT / 4), ts = (rem % (NT / 4)) * 4;
  const int i = GLU ? qo / 16 : qo / (WN * 16), j = GLU ? 0 : (qo / 16) % WN, r = qo % 16;
  const int q = (i * WN + j) * 16 + r;  // GLU: W3's register of the same output is q + 16
  floatx4_t a = {0.0f, 0.0f, 0.0f, 0.0f}, g = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
  for (int p = 0; p < parts; ++p) {
    const float *src = part + ((int64_t)p * tail + t) * PART + ts;
    a += *reinterpret_cast<const floatx4_t *>(src + q * NT);
    if constexpr (GLU) g += *reinterpret_cast<const floatx4_t *>(src + (q + 16) * NT);
  }
  int64_t tile_m, tile_n;
  tile_coords((uint32_t)(dp_tiles + t), (uint32_t)tiles_m, (uint32_t)tiles_n, tile_m, tile_n);
  const int64_t m0 = tile_m * G::BM, n0 = tile_n * BNO;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int st = ts + e, lane = st & 63, wave = st >> 6;
    const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N, l32 = lane & 31, lh = lane >> 5;
    const int64_t row = m0 + wm * (32 * WM) + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
    const int64_t col = GLU ? n0 + wn * 32 + l32 : n0 + wn * (32 * WN) + 32 * j + l32;
    if (row >= M || col >= N) continue;
    float v = a[e] + ((!GLU && bias) ? bias[col] : 0.0f);
    if constexpr (GLU) v = v / (1.0f + __expf(-v)) * g[e];
    if (y_dtype == BIQ_DTYPE_F32) {
      reinterpret_cast<float *>(yv)[row * N + col] = v;
    } else if (y_dtype == BIQ_DTYPE_F16) {
      reinterpret_cast<_Float16 *>(yv)[row * N + col] = biq::f16_of_f32(v);
    } else {
      reinterpret_cast<uint16_t *>(yv)[row * N + col] = (uint16_t)biq::f32_to_bf16_bits(v);
    }
  }
}

// EPI = 1: the fused Q/K preparation epilogue (qk_epilogue; every tile owned, yv unused).
template <class G, int LAYOUT, int XMODE, int BLK, bool GLU, int EPI = 0>
__global__ void __launch_bounds__(G::NTHREADS, G::NTHREADS >= 512 ? 1 : 2)
    q4_gemm_kernel(const void *__restrict__ xv, int64_t ldx, const uint32_t *__restrict__ words,
                   const float *__restrict__ scales, const uint32_t *__restrict__ words3,
                   const float *__restrict__ scales3, const float *__restrict__ bias,
                   void *__restrict__ yv, int y_dtype, int64_t M, int64_t N, int64_t K,
                   int tiles_m, int tiles_n, SkPlan sk, QkEpi qe) {
  static_assert(EPI == 0 || (G::RESCALE && !GLU), "the fused epilogue runs on the 256 x 256 tile");
  constexpr int WM = G::WM, WN = G::WN, BM = G::BM, BN = G::BN, NT = G::NTHREADS;
  static_assert(!GLU || WN == 2, "the SwiGLU form pairs the two column tiles of a wave");
  constexpr int BNO = GLU ? BN / 2 : BN;  // output columns per workgroup
  constexpr int BK = G::BK, A_LD = G::A_LD;
  constexpr int B_LD = BN;  // LDS row stride of the word tile, in words
  constexpr int NSPLIT = XMODE == XM_F32 ? 2 : 1;
  constexpr int TILE_BLOCKS = BLK >= BK ? 1 : BK / BLK;
  constexpr int TPB = BLK >= BK ? BLK / BK : 1;  // K tiles per quantisation block
  static_assert(TPB == 1 || TPB == 2, "a pair of K tiles must cover whole blocks");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][NSPLIT][BM * A_LD];
  __shared__ __attribute__((aligned(16))) uint32_t Bs[2][(BK / 8) * B_LD];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
  const int l32 = lane & 31, lh = lane >> 5;

  // ---- this workgroup's tile segments.  Owned tiles come in the XCD-aware order: hardware
  //      places workgroup L on XCD L % 8, and the workgroups of one XCD take a compact run of
  //      pids (tail workgroups likewise take a compact run of chunk indices; dp_tiles is a
  //      multiple of 8, so tail workgroup w also runs on XCD w % 8).
  // Work indices in 32 bits (tiles, chunks and K units stay below 2^31: host checks).
  const uint32_t T = (uint32_t)tiles_m * (uint32_t)tiles_n;
  const uint32_t L = blockIdx.x;
  const uint32_t units = (uint32_t)sk.units, dp = (uint32_t)sk.dp_tiles, sk_wgs = (uint32_t)sk.sk_wgs;
  const uint32_t parts = (uint32_t)sk.parts;
  const bool tail_wg = L >= dp;
  const uint32_t tail = T - dp, chunks = tail * parts;
  auto xcd_order = [](uint32_t i, uint32_t n) {
    const uint32_t q = n / 8, r = n % 8, xcd = i % 8, slot = i / 8;
    return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
  };
  const uint32_t first = tail_wg ? xcd_order(L - dp, sk_wgs) : xcd_order(L, dp);
  // (the fused epilogue's launches own every tile: one segment, known at compile time, so no
  // value of the segment loop stays live through the epilogue)
  const uint32_t n_seg = EPI == 1 ? 1u : (tail_wg ? (chunks - first + sk_wgs - 1) / sk_wgs : 1u);

  for (uint32_t seg = 0; seg < n_seg; ++seg) {
  const uint32_t c = first + seg * sk_wgs;  // tail chunk (tail workgroups only)
  const uint32_t t_tail = tail_wg ? c % tail : 0u, k_part = tail_wg ? c / tail : 0u;
  const uint32_t pid = tail_wg ? dp + t_tail : first;
  // with two register sets, tail parts start on even K tiles, so every part but the last (which
  // ends at K) has an even number of tiles for the paired loop below
  constexpr uint32_t GRAN = PART_GRANULE<G, LAYOUT, XMODE, BLK>;
  auto part_start = [&](uint32_t kp) -> uint32_t {
    return kp >= parts ? units : GRAN * (kp * (units / GRAN) / parts);
  };
  const int64_t ku0 = tail_wg ? part_start(k_part) : 0;
  const int64_t ku1 = tail_wg ? part_start(k_part + 1) : units;
  constexpr int64_t UNIT = (int64_t)TPB * BK;
  const int64_t k_lo = ku0 * UNIT, k_hi = ku1 * UNIT < K ? ku1 * UNIT : K;

  int64_t tile_m, tile_n;
  tile_coords(pid, tiles_m, tiles_n, tile_m, tile_n);
  const int64_t m0 = tile_m * BM, n0 = tile_n * BNO;
  const int64_t nblk = K / BLK;
  const int64_t KW = K / 8;

  int64_t ncol[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j)
    ncol[j] = GLU ? n0 + wn * 32 + l32 : n0 + wn * (32 * WN) + 32 * j + l32;

  // ---- global -> registers through buffer loads.  Descriptors start at the tile (scalar
  //      registers, advanced per tile) and end at the matrix, so rows past M and packed rows past
  //      K read as zero; columns past N get an offset beyond any range, and so do activation
  //      groups / packed column groups past K in a partial last tile.  Offsets stay below 2^31
  //      (host check).
  constexpr uint32_t OOB = 0x80000000u;
  constexpr int64_t XSZ = XMODE == XM_F32 ? 4 : 2;
  uint32_t a_off[G::A_CHUNKS], b_off[G::B_CHUNKS];
  bool b_w3[G::B_CHUNKS];  // GLU: this word group comes from W3
#pragma unroll
  for (int it = 0; it < G::A_CHUNKS; ++it) {
    const int c = tid + it * NT;
    a_off[it] = (uint32_t)(((int64_t)(c / (BK / 8)) * ldx + 8 * (c % (BK / 8))) * XSZ);
  }
  // GLU with an even number of word groups per thread: groups [0, B_CHUNKS / 2) come from W1
  // and the rest from W3 (for the [N, K/8] layout the plain numbering already does this), so each
  // load names its weight at compile time.  Otherwise both weights are read with the same offset,
  // the other weight's lanes passing an out-of-range offset (zero, no memory access), and the
  // two results are OR-ed -- which makes the wave wait for them right away.
  // With an odd number (the 256 x 256 tile: one group per thread), the first half of the
  // workgroup's waves loads W1 and the second half W3, so the weight is wave-uniform: the load
  // picks its descriptor on the scalar unit (measured: the OR form made the fused SwiGLU's large
  // tile wait for every word load right after issuing it).
  constexpr bool GLU_SPLIT = GLU && G::B_CHUNKS % 2 == 0;
  constexpr bool GLU_WAVE = GLU && !GLU_SPLIT && LAYOUT == BIQ_Q4_KN_AXIS1 &&
                            (BK / 8) * (BNO / 4) == G::B_CHUNKS * (NT / 2);
  const bool half_w3 = __builtin_amdgcn_readfirstlane(tid / (NT / 2)) != 0;  // GLU_WAVE: W3 half
  auto kn_group = [&](int it, int &kwr, int &nc, bool &w3) {  // [K/8, N] word group `it`
    if constexpr (GLU_WAVE) {
      const int ch = tid % (NT / 2) + it * (NT / 2);
      w3 = half_w3;
      kwr = ch / (BNO / 4);
      nc = (ch % (BNO / 4)) * 4;
    } else if constexpr (GLU_SPLIT) {
      const int ch = tid + (it % (G::B_CHUNKS / 2)) * NT;
      w3 = it >= G::B_CHUNKS / 2;
      kwr = ch / (BNO / 4);
      nc = (ch % (BNO / 4)) * 4;
    } else {
      const int c = tid + it * NT;
      kwr = c / (BN / 4);
      nc = (c % (BN / 4)) * 4;
      w3 = GLU && nc >= BNO;
      nc -= w3 ? BNO : 0;
    }
  };
#pragma unroll
  for (int it = 0; it < G::B_CHUNKS; ++it) {
    const int c = tid + it * NT;
    if constexpr (LAYOUT == BIQ_Q4_KN_AXIS1) {
      int kwr, nc;
      bool w3;
      kn_group(it, kwr, nc, w3);
      b_w3[it] = w3;
      b_off[it] = n0 + nc < N ? (uint32_t)(((int64_t)kwr * N + nc) * 4) : OOB;
    } else {
      const int part4 = c % (BK / 32);
      int nl = c / (BK / 32);
      b_w3[it] = GLU && nl >= BNO;
      nl -= b_w3[it] ? BNO : 0;
      b_off[it] = n0 + nl < N ? (uint32_t)(((int64_t)nl * KW + 4 * part4) * 4) : OOB;
    }
  }
  auto rsrc = [](const void *base, int64_t bytes) {
    const uint32_t n = bytes > 0x7fffffffLL ? 0x7fffffffu : (bytes < 0 ? 0u : (uint32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)n, 0x00020000);
  };
  // Word rows of the [N, K/8] layout are 16-byte aligned only when K % 32 == 0.
  const bool vec_nk = (KW & 3) == 0;
  // Block scales also come in through buffer loads: a scale outside the matrix reads as zero
  // through an out-of-range offset.  (A select on the loaded value would make the wave wait for
  // the whole prefetch right after issuing it.)
  const auto rs = rsrc(scales, nblk * N * 4);
  const auto rs3 = rsrc(GLU ? scales3 : scales, nblk * N * 4);
  auto scale_off = [&](int64_t b, int j) -> uint32_t {
    const int64_t n = ncol[j];
    if (n >= N || b >= nblk) return OOB;
    return (uint32_t)((LAYOUT == BIQ_Q4_KN_AXIS1 ? b * N + n : n * nblk + b) * 4);
  };

  auto load_tile = [&](int64_t kt, TileRegs<G, XMODE, TILE_BLOCKS> &R) {
    // scales first: a wait for the tile's data then covers them too
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int t = 0; t < TILE_BLOCKS; ++t)
        R.sc[j][t] = biq::bitcast<float>(__builtin_amdgcn_raw_buffer_load_b32(
            GLU && j == 1 ? rs3 : rs, scale_off(kt / BLK + t, j), 0, 0));
    const auto ra = rsrc(reinterpret_cast<const char *>(xv) + (m0 * ldx + kt) * XSZ,
                         ((M - m0) * ldx - kt) * XSZ);
#pragma unroll
    for (int it = 0; it < G::A_CHUNKS; ++it) {
      const int kc = (tid + it * NT) % (BK / 8);
      const uint32_t off = kt + 8 * kc < K ? a_off[it] : OOB;
      if constexpr (XMODE == XM_F32) {
        R.a32[2 * it] = biq::bitcast<float4>(__builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
        R.a32[2 * it + 1] = biq::bitcast<float4>(__builtin_amdgcn_raw_buffer_load_b128(ra, off + 16, 0, 0));
      } else {
        R.a16[it] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
      }
    }
    const int64_t kw0 = kt / 8;
    auto ld128 = [&](const __amdgpu_buffer_rsrc_t &r1, const __amdgpu_buffer_rsrc_t &r3, uint32_t off,
                     bool w3, int it) -> u32x4_t {
      if constexpr (!GLU) return __builtin_amdgcn_raw_buffer_load_b128(r1, off, 0, 0);
      if constexpr (GLU_WAVE) return __builtin_amdgcn_raw_buffer_load_b128(half_w3 ? r3 : r1, off, 0, 0);
      if constexpr (GLU_SPLIT) return __builtin_amdgcn_raw_buffer_load_b128(it >= G::B_CHUNKS / 2 ? r3 : r1, off, 0, 0);
      return __builtin_amdgcn_raw_buffer_load_b128(r1, w3 ? OOB : off, 0, 0) |
             __builtin_amdgcn_raw_buffer_load_b128(r3, w3 ? off : OOB, 0, 0);
    };
    auto ld32 = [&](const __amdgpu_buffer_rsrc_t &r1, const __amdgpu_buffer_rsrc_t &r3, uint32_t off,
                    bool w3, int it) -> uint32_t {
      if constexpr (!GLU) return __builtin_amdgcn_raw_buffer_load_b32(r1, off, 0, 0);
      if constexpr (GLU_SPLIT) return __builtin_amdgcn_raw_buffer_load_b32(it >= G::B_CHUNKS / 2 ? r3 : r1, off, 0, 0);
      return __builtin_amdgcn_raw_buffer_load_b32(r1, w3 ? OOB : off, 0, 0) |
             __builtin_amdgcn_raw_buffer_load_b32(r3, w3 ? off : OOB, 0, 0);
    };
    if constexpr (LAYOUT == BIQ_Q4_KN_AXIS1) {
      const auto rb = rsrc(words + kw0 * N + n0, ((KW - kw0) * N - n0) * 4);
      const auto rb3 = rsrc((GLU ? words3 : words) + kw0 * N + n0, ((KW - kw0) * N - n0) * 4);
#pragma unroll
      for (int it = 0; it < G::B_CHUNKS; ++it) R.b[it] = ld128(rb, rb3, b_off[it], b_w3[it], it);
    } else {
      const auto rb = rsrc(words + n0 * KW + kw0, ((N - n0) * KW - kw0) * 4);
      const auto rb3 = rsrc((GLU ? words3 : words) + n0 * KW + kw0, ((N - n0) * KW - kw0) * 4);
#pragma unroll
      for (int it = 0; it < G::B_CHUNKS; ++it) {
        const int part4 = (tid + it * NT) % (BK / 32);
        const int64_t kwb = kw0 + 4 * part4;
        if (vec_nk) {
          R.b[it] = ld128(rb, rb3, kwb < KW ? b_off[it] : OOB, b_w3[it], it);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) R.b[it][j] = ld32(rb, rb3, kwb + j < KW ? b_off[it] + 4 * j : OOB, b_w3[it], it);
        }
      }
    }
  };

  // ---- registers -> LDS buffer (activation conversion to f16 slot order happens here)
  auto store_tile = [&](const TileRegs<G, XMODE, TILE_BLOCKS> &R, int buf) {
#pragma unroll
    for (int it = 0; it < G::A_CHUNKS; ++it) {
      const int c = tid + it * NT;
      const int row = c / (BK / 8), kc = c % (BK / 8);
      u32x4_t hi, lo;
      if constexpr (XMODE == XM_BF16) hi = bf16x8_to_f16_slots(R.a16[it]);
      else if constexpr (XMODE == XM_F16) hi = f16x8_to_slots(R.a16[it]);
      else f32x8_to_f16_split_slots(R.a32[2 * it], R.a32[2 * it + 1], hi, lo);
      *reinterpret_cast<u32x4_t *>(&As[buf][0][row * A_LD + 8 * kc]) = hi;
      if constexpr (NSPLIT == 2) *reinterpret_cast<u32x4_t *>(&As[buf][1][row * A_LD + 8 * kc]) = lo;
    }
#pragma unroll
    for (int it = 0; it < G::B_CHUNKS; ++it) {
      const int c = tid + it * NT;
      if constexpr (LAYOUT == BIQ_Q4_KN_AXIS1) {
        int kwr, nc;
        bool w3;
        kn_group(it, kwr, nc, w3);
        *reinterpret_cast<u32x4_t *>(&Bs[buf][kwr * B_LD + nc + (w3 ? BNO : 0)]) = R.b[it];
      } else {
        const int nl = c / (BK / 32), part4 = c % (BK / 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) Bs[buf][(4 * part4 + j) * B_LD + nl] = R.b[it][j];
      }
    }
  };

  // Block scales.  Partial form: the MFMAs of block b accumulate part = sum_k x q in their own
  // registers, then acc += s_b * part.  Rescale form (G::RESCALE): the MFMAs accumulate straight
  // into acc, which is kept relative to the current block's scale: at the first step of block b,
  // acc *= t_{b-1} / t_b, and at the end acc *= t_last, so acc = sum_b t_b * part_b.  The same one
  // VALU op per accumulator per block, half the registers; the relative rounding of the ratios and
  // multiplies is ~2^-24 per block of the partial output, far inside the f32 parity gate.
  constexpr bool RESC = G::RESCALE;
  floatx16_t acc[WM][WN], part[RESC ? 1 : WM][RESC ? 1 : WN];
  [[maybe_unused]] float t_prev[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j) t_prev[j] = 1.0f;
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = biq::zero16();

  // LDS operand reads of one K16 step: WM activation fragments and WN packed words.
  auto read_step = [&](int buf, int s, half8_t (&a)[WM][NSPLIT], uint32_t (&w)[WN]) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int x = 0; x < NSPLIT; ++x)
        a[i][x] = *reinterpret_cast<const half8_t *>(
            &As[buf][x][(wm * (32 * WM) + 32 * i + l32) * A_LD + 16 * s + 8 * lh]);
#pragma unroll
    for (int j = 0; j < WN; ++j)
      w[j] = Bs[buf][(2 * s + lh) * B_LD + (GLU ? j * BNO + wn * 32 : wn * (32 * WN) + 32 * j) + l32];
  };

  // Pipeline, PF register sets deep: while tile t computes from one LDS buffer, register set
  // t % PF holds tile t+1 (stored into the other LDS buffer during iteration t) and is then
  // refilled with tile t+1+PF, so every global load has PF whole tiles to arrive.  Iterations go
  // in pairs so that every set is named at compile time: a loaded register is never copied while
  // its load is in flight (a copy would make the wave wait for it).  Two sets where the registers
  // allow it without spilling in the loop, else one.  The block scales travel in the same sets.
  // 16-bit activations are stored (converted) after the tile's MFMAs and the refill follows:
  // stored first, the conversion ran as one VALU burst ahead of the tile's first MFMA, in step on
  // both waves of a SIMD (measured: -1 to -2% time on the 4608-row shapes, -2% fused SwiGLU).
  // f32 activations keep the store first: their two hi/lo planes stored late ran +28% slower.
  constexpr int PF = PF_SETS<G, LAYOUT, XMODE, BLK>;
  constexpr bool STAGE_LATE = XMODE != XM_F32;
  constexpr int NTT = (PF == 2 || TPB == 2) ? 2 : 1;  // K tiles per loop iteration
  TileRegs<G, XMODE, TILE_BLOCKS> RS[PF];
  float sc_hold[WN][TILE_BLOCKS];  // scales of the tile computed next, copied out of its set
  load_tile(k_lo, RS[0]);
  store_tile(RS[0], 0);
#pragma unroll
  for (int j = 0; j < WN; ++j)
#pragma unroll
    for (int t = 0; t < TILE_BLOCKS; ++t) sc_hold[j][t] = RS[0].sc[j][t];
  // issued in set order, as the loop issues them (the wave's wait counts assume it)
#pragma unroll
  for (int p = 0; p < PF; ++p) {
    load_tile(k_lo + (1 + p) * BK, RS[p]);
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();

  int buf = 0;
  // A pair of iterations covers whole quantisation blocks (TPB is 1 or 2), so the first / last
  // step of every block is known at compile time: the MFMA chain of a block starts from an inline
  // zero and no accumulator is copied or selected at run time.  With two register sets a segment
  // with an odd number of tiles (TPB 1) ends at K, and the second tile of its last pair lies
  // wholly past K: its
  // loads read zeros (activations, words and scales), so it adds exact zeros.  (Skipping it
  // would put a join in the loop, where the compiler waits for the whole prefetch.)
  for (int64_t kg = k_lo; kg < k_hi; kg += NTT * BK) {
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
      const int64_t kt = kg + tt * BK;
      TileRegs<G, XMODE, TILE_BLOCKS> &R = RS[tt % PF];

      half8_t a_cur[WM][NSPLIT], a_nxt[WM][NSPLIT];
      uint32_t w_cur[WN], w_nxt[WN];
      half8_t b_cur[WN];
      read_step(buf, 0, a_cur, w_cur);
      float sc_cur[WN][TILE_BLOCKS];
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int t = 0; t < TILE_BLOCKS; ++t) sc_cur[j][t] = sc_hold[j][t];
      // Staging and prefetch run unconditionally: past the end of K the buffer loads return
      // zeros and a store past the last tile lands in a buffer nobody reads again.  (A branch
      // here makes the compiler merge the freshly loaded registers at the join, which waits for
      // the whole prefetch before the first MFMA.)  The set's scales are copied out after the
      // store, which has waited for the set anyway.
      auto stage_next = [&]() {
        store_tile(R, buf ^ 1);
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
          for (int t = 0; t < TILE_BLOCKS; ++t) sc_hold[j][t] = R.sc[j][t];
        load_tile(kt + (1 + PF) * BK, R);
      };
      if constexpr (!STAGE_LATE) stage_next();
#pragma unroll
      for (int j = 0; j < WN; ++j) b_cur[j] = unpack_q4_f16(w_cur[j]);

      // A partial last tile (K % 64 != 0, small blocks only) runs to the end: its activations,
      // words and scales beyond K were loaded as zeros, so the extra steps add exact zeros.
#pragma unroll
      for (int s = 0; s < BK / 16; ++s) {
        if (s + 1 < BK / 16) read_step(buf, s + 1, a_nxt, w_nxt);

        if constexpr (BLK == 8) {
          // Lanes 0-31 carry block 2g, lanes 32-63 block 2g + 1: two masked MFMAs.
          const half8_t zh = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
          for (int j = 0; j < WN; ++j) {
            const half8_t b_lo = lh == 0 ? b_cur[j] : zh;
            const half8_t b_hi = lh == 0 ? zh : b_cur[j];
#pragma unroll
            for (int i = 0; i < WM; ++i) {
              floatx16_t p = biq::mfma32x32x16_f16(a_cur[i][0], b_lo, biq::zero16());
              if constexpr (NSPLIT == 2) p = biq::mfma32x32x16_f16(a_cur[i][1], b_lo, p);
              acc[i][j] += sc_cur[j][2 * s] * p;
              p = biq::mfma32x32x16_f16(a_cur[i][0], b_hi, biq::zero16());
              if constexpr (NSPLIT == 2) p = biq::mfma32x32x16_f16(a_cur[i][1], b_hi, p);
              acc[i][j] += sc_cur[j][2 * s + 1] * p;
            }
          }
        } else {
          constexpr int SPB = BLK / 16;  // K16 steps per block
          const bool first = BLK >= BK ? (tt % TPB == 0 && s == 0) : (s % SPB) == 0;
          const bool last = BLK >= BK ? (tt % TPB == TPB - 1 && s == BK / 16 - 1) : (s % SPB) == SPB - 1;
          const int tb = BLK >= BK ? 0 : s / SPB;
          if constexpr (RESC) {
            // acc starts at zero and t_prev at 1, so the first block's ratio (finite: clamped
            // scales) leaves it zero
            float r[WN];
            if (first) {
#pragma unroll
              for (int j = 0; j < WN; ++j) {
                const float t = clamp_scale(sc_cur[j][tb]);
                r[j] = t_prev[j] / t;
                t_prev[j] = t;
              }
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
              for (int j = 0; j < WN; ++j) {
                floatx16_t c = acc[i][j];
                if (first) c *= r[j];
                acc[i][j] = biq::mfma32x32x16_f16(a_cur[i][0], b_cur[j], c);
              }
          } else {
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
              for (int j = 0; j < WN; ++j) {
                floatx16_t p =
                    biq::mfma32x32x16_f16(a_cur[i][0], b_cur[j], first ? biq::zero16() : part[i][j]);
                if constexpr (NSPLIT == 2) p = biq::mfma32x32x16_f16(a_cur[i][1], b_cur[j], p);
                part[i][j] = p;
              }
            if (last) {
#pragma unroll
              for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j) acc[i][j] += sc_cur[j][tb] * part[i][j];
            }
          }
        }

        if (s + 1 < BK / 16) {
#pragma unroll
          for (int j = 0; j < WN; ++j) b_cur[j] = unpack_q4_f16(w_nxt[j]);
#pragma unroll
          for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int x = 0; x < NSPLIT; ++x) a_cur[i][x] = a_nxt[i][x];
        }
      }
      if constexpr (STAGE_LATE) stage_next();
      if constexpr (!RESC && XMODE != XM_F32 && BLK >= 32) {
        // 128 x 256 tile: one MFMA, then six VALU (the block-end flush and the decode of the next
        // fragments spread through the MFMA stream; same-box runs: ~0.6% over the shapes that
        // take this tile, up to 2%)
#pragma unroll
        for (int g = 0; g < BK / 16 * WM * WN; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
        }
      }
      if constexpr (RESC) {
        // One MFMA, then four VALU, through the tile: otherwise the block-boundary rescale (one
        // multiply per accumulator) runs as a burst before the block's first MFMA.  (Same-box
        // runs of 2-10 VALU per MFMA: 4 leads 6 by ~0.5% summed over the 4608-row projections,
        // 8 and 10 trail.)
#pragma unroll
        for (int g = 0; g < BK / 16 * WM * WN; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
        }
      }
      __syncthreads();
      buf ^= 1;
    }
  }

  // ---------------- epilogue: bias (or the SwiGLU gate), convert, store ---------------------
  if constexpr (RESC) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[i][j] *= t_prev[j];
  }
  if constexpr (EPI == 1) {  // the loop's last barrier has retired every LDS access
    qk_epilogue<G>(acc, m0, n0, M, qe, reinterpret_cast<float *>(&As[0][0][0]));
    continue;
  }
  if (ku0 == 0 && ku1 == units) {  // the whole K of the tile
    // rows of a wave tile within 32-bit offsets (else the per-element form)
    if ((int64_t)(32 * WM) * N * (y_dtype == BIQ_DTYPE_F32 ? 4 : 2) < (1LL << 31)) {
      if (y_dtype == BIQ_DTYPE_F32) store_tile_out_rows<G, GLU, float>(acc, m0, n0, bias, yv, M, N);
      else if (y_dtype == BIQ_DTYPE_F16) store_tile_out_rows<G, GLU, _Float16>(acc, m0, n0, bias, yv, M, N);
      else store_tile_out_rows<G, GLU, uint16_t>(acc, m0, n0, bias, yv, M, N);
    } else {
      store_tile_out<G, GLU>(acc, m0, n0, bias, yv, y_dtype, M, N);
    }
    continue;
  }
  // ---- tail chunk: the partial goes to slot c, register-major (element (register q, thread
  //      tid) at q * NT + tid: one coalesced 256-byte row per wave and register)
  {
    constexpr int PART = BM * BN;
    const auto dst = __builtin_amdgcn_make_buffer_rsrc(sk.part + (int64_t)c * PART, 0, PART * 4, 0x00020000);
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          __builtin_amdgcn_raw_buffer_store_b32(biq::bitcast<uint32_t>(acc[i][j][r]), dst, tid * 4,
                                                ((i * WN + j) * 16 + r) * NT * 4, 0);
  }
  }  // segments
}

// Weights of one launch: W (and W3 for the SwiGLU form).
struct Q4Args {
  const uint32_t *words, *words3;
  const float *scales, *scales3;
};

// Split of a grid of T tiles of `units` K units each over `cus` compute units (see SkPlan): the
// whole rounds are owned tiles; the tail of T % cus tiles is split into the number of K parts
// that minimises the estimated time, counted in tile times: rounds of chunks, each chunk 1 /
// parts of a tile plus the cost of writing and reading back a round of partials (~0.13 tile),
// plus the tail reduction's read of a tile's partials (~0.012 tile per part).  A tail that is
// already most of a round stays whole.
// BIQ_GEMM_STREAMK in the environment: "0" (or "1") keeps every tile whole; a number n > 1
// forces n parts (capped to what K allows) -- a tuning switch.  Measured against the model's
// choice: 1024x4096x4096 (128 tiles) 79.5 -> 57.2 us with 2 parts (chosen); 1024x4096x6144 (192
// tiles) and the 4608-row O / MLP shapes are fastest whole (chosen); 4608x3072x9216: 6 parts
// (chosen) 403 us, 8 parts 400 us, whole 423 us.
SkPlan plan_tail(int64_t T, int64_t units, int64_t granule, int cus, double *est_rounds = nullptr) {
  SkPlan p{(int)T, 0, 1, units, nullptr};
  if (est_rounds) *est_rounds = cus > 0 ? (double)((T + cus - 1) / cus) : 1.0;
  const char *env = getenv("BIQ_GEMM_STREAMK");
  const int forced = env ? atoi(env) : -1;
  if (cus <= 0 || units < 2 || forced == 0 || forced == 1) return p;
  const int64_t tail = T % cus;
  if (tail == 0) return p;
  const int64_t max_parts = units / granule < 16 ? units / granule : 16;
  double best = 1.0;
  int parts = 1;
  for (int s = 2; s <= max_parts; ++s) {
    const int64_t rounds = (tail * s + cus - 1) / cus;
    const double est = rounds * (1.0 / s + 0.13) + 0.012 * s;
    if (est < best - 0.05) {
      best = est;
      parts = s;
    }
  }
  if (forced > 1) parts = forced < max_parts ? forced : (int)max_parts;
  if (est_rounds) {
    const int64_t rounds = (tail * parts + cus - 1) / cus;
    *est_rounds = (double)(T / cus) + (parts > 1 ? rounds * (1.0 / parts + 0.13) + 0.012 * parts : 1.0);
  }
  if (parts <= 1) return p;
  p.dp_tiles = (int)(T - tail);
  p.parts = parts;
  p.sk_wgs = (int)(tail * parts < cus ? tail * parts : cus);
  return p;
}

template <class GG, int LAYOUT, int XMODE, int B, bool GLU>
int launch_geo(hipStream_t s, const void *x, int64_t ldx, const Q4Args &w, const float *bias,
               void *y, int y_dtype, int64_t M, int64_t N, int64_t K, const biq::Scratch *scr) {
  constexpr int BNO = GLU ? GG::BN / 2 : GG::BN;
  constexpr int64_t UNIT = (int64_t)(B >= GG::BK ? B : GG::BK);
  const int tiles_m = (int)((M + GG::BM - 1) / GG::BM), tiles_n = (int)((N + BNO - 1) / BNO);
  const int64_t T = (int64_t)tiles_m * tiles_n;
  SkPlan plan = plan_tail(T, (K + UNIT - 1) / UNIT, PART_GRANULE<GG, LAYOUT, XMODE, B>,
                         biq::device_cu_count());
  const int tail = (int)(T - plan.dp_tiles);
  if (plan.sk_wgs > 0) {
    void *part = nullptr;
    const size_t chunks = (size_t)tail * plan.parts;
    const int st = biq::get_scratch(s, scr, chunks * GG::BM * GG::BN * sizeof(float), &part);
    if (st != BIQ_OK) return st;
    plan.part = reinterpret_cast<float *>(part);
  }
  dim3 grid((unsigned)(plan.dp_tiles + plan.sk_wgs));
  hipLaunchKernelGGL((q4_gemm_kernel<GG, LAYOUT, XMODE, B, GLU>), grid, dim3(GG::NTHREADS), 0, s, x,
                     ldx, w.words, w.scales, w.words3, w.scales3, bias, y, y_dtype, M, N, K,
                     tiles_m, tiles_n, plan, QkEpi{});
  if (plan.sk_wgs > 0) {
    const int st = biq::check_launch(GLU ? "q4 linear swiglu" : "q4 linear");
    if (st != BIQ_OK) return st;
    constexpr int QN = GLU ? GG::WM * 16 : GG::WM * GG::WN * 16;
    const int64_t threads = (int64_t)tail * QN * (GG::NTHREADS / 4);
    hipLaunchKernelGGL((q4_tail_reduce_kernel<GG, GLU>),
                       dim3((unsigned)((threads + RED_THREADS - 1) / RED_THREADS)), dim3(RED_THREADS),
                       0, s, plan.part, tail, plan.parts, plan.dp_tiles, tiles_m, tiles_n, bias, y,
                       y_dtype, M, N);
  }
  return biq::check_launch(GLU ? "q4 linear swiglu" : "q4 linear");
}

// Estimated launch time of geometry GG in units of one 128 x 256 tile: rounds of tiles over the
// CUs (with the tail split the way launch_geo would split it) times the cost of one tile.  A
// 256 x 256 tile costs 1.86 units (measured: 7% less per output than two 128 x 256 tiles).
template <class GG, int LAYOUT, int XMODE, int B, bool GLU>
double est_launch(int64_t M, int64_t N, int64_t K) {
  constexpr int BNO = GLU ? GG::BN / 2 : GG::BN;
  constexpr int64_t UNIT = (int64_t)(B >= GG::BK ? B : GG::BK);
  const int64_t T = ((M + GG::BM - 1) / GG::BM) * ((N + BNO - 1) / BNO);
  double rounds = 1.0;
  plan_tail(T, (K + UNIT - 1) / UNIT, PART_GRANULE<GG, LAYOUT, XMODE, B>, biq::device_cu_count(), &rounds);
  return rounds * (GG::RESCALE ? 1.86 : 1.0);
}

// Geometry choice.  Where the 256 x 256 tile applies, the rows may also be split: rows
// [0, M_big) run as 256 x 256 tiles and the rest as 128 x 256 tiles, in two launches on the
// stream, with M_big (a multiple of 256, possibly 0 or M) minimising the summed est_launch.  E.g.
// 4608 x 3072 x 9216: 3584 rows of 256 x 256 tiles fill two rounds (504 tiles) and the last
// 1024 rows (288 tiles of 128 x 256) finish in a little over one round of half-size tiles,
// where either tile alone leaves most of a round idle.  Rows of the two parts are rounded in a
// different order (partial vs rescale form): equal within the parity gate, not bitwise.
// BIQ_GEMM_TILE in the environment: "small" or "big" forces one geometry for all rows (a tuning
// switch); BIQ_GEMM_STREAMK=0 ("every tile owned") also keeps the rows unsplit.
template <int LAYOUT, int XMODE, int B, bool GLU>
int launch_pick(hipStream_t s, const void *x, int64_t ldx, const Q4Args &w, const float *bias, void *y,
                int y_dtype, int64_t M, int64_t N, int64_t K, const biq::Scratch *scr) {
  using GS = GemmGeo<XMODE, B>;
  using GB = GemmGeoBig;
  if constexpr (XMODE != XM_F32 && B >= 32) {
    const char *env = getenv("BIQ_GEMM_TILE");
    const char *sk = getenv("BIQ_GEMM_STREAMK");
    const bool no_split = sk && (sk[0] == '0' || sk[0] == '1') && sk[1] == 0;
    int64_t m_big = 0;
    if (env && env[0] == 's') {
      m_big = 0;
    } else if (env && env[0] == 'b') {
      m_big = M;
    } else {
      double best = est_launch<GS, LAYOUT, XMODE, B, GLU>(M, N, K);
      const double whole_big = est_launch<GB, LAYOUT, XMODE, B, GLU>(M, N, K);
      if (whole_big < best) { best = whole_big; m_big = M; }
      if (!no_split)
        for (int64_t mb = GB::BM; mb < M; mb += GB::BM) {
          const double e = est_launch<GB, LAYOUT, XMODE, B, GLU>(mb, N, K) +
                           est_launch<GS, LAYOUT, XMODE, B, GLU>(M - mb, N, K);
          if (e < best - 0.02) { best = e; m_big = mb; }
        }
    }
    if (m_big > 0) {
      const int st = launch_geo<GB, LAYOUT, XMODE, B, GLU>(s, x, ldx, w, bias, y, y_dtype, m_big, N, K, scr);
      if (st != BIQ_OK || m_big == M) return st;
      const int esz = XMODE == XM_F32 ? 4 : 2;
      const int osz = y_dtype == BIQ_DTYPE_F32 ? 4 : 2;
      return launch_geo<GS, LAYOUT, XMODE, B, GLU>(s, reinterpret_cast<const char *>(x) + m_big * ldx * esz, ldx,
                                                   w, bias, reinterpret_cast<char *>(y) + m_big * N * osz, y_dtype,
                                                   M - m_big, N, K, scr);
    }
  }
  return launch_geo<GS, LAYOUT, XMODE, B, GLU>(s, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
}

template <int LAYOUT, int XMODE, bool GLU>
int launch_blk(hipStream_t s, int block, const void *x, int64_t ldx, const Q4Args &w,
               const float *bias, void *y, int y_dtype, int64_t M, int64_t N, int64_t K,
               const biq::Scratch *scr) {
  using G8 = GemmGeo<XMODE, 8>;
  using G16 = GemmGeo<XMODE, 16>;
  switch (block) {
    case 8: return launch_geo<G8, LAYOUT, XMODE, 8, GLU>(s, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
    case 16: return launch_geo<G16, LAYOUT, XMODE, 16, GLU>(s, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
    case 32: return launch_pick<LAYOUT, XMODE, 32, GLU>(s, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
    case 64: return launch_pick<LAYOUT, XMODE, 64, GLU>(s, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
    default: return launch_pick<LAYOUT, XMODE, 128, GLU>(s, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
  }
}

template <int LAYOUT, bool GLU>
int launch_layout(hipStream_t s, int x_dtype, int block, const void *x, int64_t ldx,
                  const Q4Args &w, const float *bias, void *y, int y_dtype, int64_t M, int64_t N,
                  int64_t K, const biq::Scratch *scr) {
  switch (x_dtype) {
    case BIQ_DTYPE_BF16:
      return launch_blk<LAYOUT, XM_BF16, GLU>(s, block, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
    case BIQ_DTYPE_F16:
      return launch_blk<LAYOUT, XM_F16, GLU>(s, block, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
    default:
      return launch_blk<LAYOUT, XM_F32, GLU>(s, block, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
  }
}

}  // namespace

namespace biq {
int q4_gemv_launch(hipStream_t s, const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                   const uint32_t *words, const float *scales, int layout, int block, int64_t N,
                   const float *bias, float *y, const Scratch *scr);
}

namespace {

// Argument checks shared by the plain and the SwiGLU entry points (BIQ_* status).
int check_linear(const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint32_t *words,
                 const float *scales, int layout, int block, int64_t N, const void *y, int y_dtype) {
  if (!x || !words || !scales || !y) return biq::fail(BIQ_ERR_INVALID_ARG, "null pointer argument");
  if (layout != BIQ_Q4_KN_AXIS1 && layout != BIQ_Q4_NK_AXIS0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "unknown Q4 layout");
  if (x_dtype != BIQ_DTYPE_F32 && x_dtype != BIQ_DTYPE_F16 && x_dtype != BIQ_DTYPE_BF16)
    return biq::fail(BIQ_ERR_INVALID_ARG, "activation dtype must be F32, F16 or BF16");
  if (y_dtype != BIQ_DTYPE_F32 && y_dtype != BIQ_DTYPE_F16 && y_dtype != BIQ_DTYPE_BF16)
    return biq::fail(BIQ_ERR_INVALID_ARG, "output dtype must be F32, F16 or BF16");
  if (block != 8 && block != 16 && block != 32 && block != 64 && block != 128)
    return biq::fail(BIQ_ERR_UNSUPPORTED, "Q4 block must be one of 8, 16, 32, 64, 128");
  if (M <= 0 || N <= 0 || K <= 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "q4 linear requires non-empty M, N and K");
  if (K % 8 != 0 || K % block != 0 || N % 8 != 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "q4 linear requires K % 8 == 0, K % block == 0, N % 8 == 0");
  if (ldx < K) return biq::fail(BIQ_ERR_INVALID_ARG, "activation row stride is smaller than K");
  // tile-relative buffer offsets are 32-bit: 256 activation rows, 16 packed rows of N words or
  // 256 packed columns of K / 8 words must span less than 2^31 bytes
  if (ldx >= (1LL << 21) || N >= (1LL << 24) || K >= (1LL << 24))
    return biq::fail(BIQ_ERR_UNSUPPORTED, "q4 linear: row stride, N or K too large for 32-bit tile offsets");
  // the scale grid is addressed through one buffer descriptor with 32-bit offsets
  if ((K / block) * N * 4 >= (1LL << 31))
    return biq::fail(BIQ_ERR_UNSUPPORTED, "q4 linear: the scale grid (K / block) * N * 4 bytes must stay below 2^31");
  const int esz = x_dtype == BIQ_DTYPE_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || ((ldx * esz) & 15) ||
      (reinterpret_cast<uintptr_t>(words) & 15) || (reinterpret_cast<uintptr_t>(scales) & 3))
    return biq::fail(BIQ_ERR_INVALID_ARG,
                     "q4 linear requires 16-byte aligned activation rows and packed words");
  using G0 = GemmGeo<XM_BF16, 128>;
  const int64_t tiles = ((M + G0::BM - 1) / G0::BM) * ((2 * N + G0::BN - 1) / G0::BN);
  if (tiles > 0x7fffffffLL)
    return biq::fail(BIQ_ERR_UNSUPPORTED, "q4 linear output has too many tiles for one launch");
  return BIQ_OK;
}

}  // namespace

namespace biq {
// biq_q4_linear with its scratch taken from `scr` (NULL: the library's per-stream workspace).
int q4_linear_launch(void *stream, const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                     const uint32_t *words, const float *scales, int layout, int block, int64_t N,
                     const float *bias, void *y, int y_dtype, const Scratch *scr) {
  const int st = check_linear(x, x_dtype, M, K, ldx, words, scales, layout, block, N, y, y_dtype);
  if (st != BIQ_OK) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Up to 16 rows with an f32 output stream the weights through the small-M kernel
  // (q4_gemv.hip): split-K over the whole chip instead of N / 256 workgroups of 128 rows.
  if (M <= 16 && y_dtype == BIQ_DTYPE_F32)
    return q4_gemv_launch(s, x, x_dtype, M, K, ldx, words, scales, layout, block, N, bias,
                          reinterpret_cast<float *>(y), scr);
  const Q4Args w{words, nullptr, scales, nullptr};
  if (layout == BIQ_Q4_KN_AXIS1)
    return launch_layout<BIQ_Q4_KN_AXIS1, false>(s, x_dtype, block, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
  return launch_layout<BIQ_Q4_NK_AXIS0, false>(s, x_dtype, block, x, ldx, w, bias, y, y_dtype, M, N, K, scr);
}
}  // namespace biq

extern "C" int biq_q4_linear(void *stream, const void *x, int x_dtype, int64_t M, int64_t K,
                             int64_t ldx, const uint32_t *words, const float *scales, int layout,
                             int block, int64_t N, const float *bias, void *y, int y_dtype) {
  biq::clear_error();
  return biq::q4_linear_launch(stream, x, x_dtype, M, K, ldx, words, scales, layout, block, N, bias, y,
                               y_dtype, nullptr);
}

extern "C" int biq_q4_linear_swiglu(void *stream, const void *x, int x_dtype, int64_t M, int64_t K,
                                    int64_t ldx, const uint32_t *words1, const float *scales1,
                                    const uint32_t *words3, const float *scales3, int layout,
                                    int block, int64_t N, void *y, int y_dtype) {
  biq::clear_error();
  int st = check_linear(x, x_dtype, M, K, ldx, words1, scales1, layout, block, N, y, y_dtype);
  if (st != BIQ_OK) return st;
  st = check_linear(x, x_dtype, M, K, ldx, words3, scales3, layout, block, N, y, y_dtype);
  if (st != BIQ_OK) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const Q4Args w{words1, words3, scales1, scales3};
  if (layout == BIQ_Q4_KN_AXIS1)
    return launch_layout<BIQ_Q4_KN_AXIS1, true>(s, x_dtype, block, x, ldx, w, nullptr, y, y_dtype, M, N, K, nullptr);
  return launch_layout<BIQ_Q4_NK_AXIS0, true>(s, x_dtype, block, x, ldx, w, nullptr, y, y_dtype, M, N, K, nullptr);
}

namespace {
// The fused projection on the 256 x 256 tile, every tile owned (the epilogue needs whole rows of
// K): one launch.
template <int XMODE, int B>
int launch_qk(hipStream_t s, const void *x, int64_t ldx, const uint32_t *words, const float *scales,
              int64_t M, int64_t N, int64_t K, const QkEpi &e) {
  using GG = GemmGeoBig;
  constexpr int64_t UNIT = (int64_t)(B >= GG::BK ? B : GG::BK);
  const int tiles_m = (int)((M + GG::BM - 1) / GG::BM), tiles_n = (int)((N + GG::BN - 1) / GG::BN);
  const int64_t T = (int64_t)tiles_m * tiles_n;
  const SkPlan plan{(int)T, 0, 1, (K + UNIT - 1) / UNIT, nullptr};
  hipLaunchKernelGGL((q4_gemm_kernel<GG, BIQ_Q4_KN_AXIS1, XMODE, B, false, 1>), dim3((unsigned)T),
                     dim3(GG::NTHREADS), 0, s, x, ldx, words, scales, nullptr, nullptr, nullptr,
                     nullptr, 0, M, N, K, tiles_m, tiles_n, plan, e);
  return biq::check_launch("q4 linear qk norm rope");
}

template <int XMODE>
int launch_qk_blk(hipStream_t s, int block, const void *x, int64_t ldx, const uint32_t *words,
                  const float *scales, int64_t M, int64_t N, int64_t K, const QkEpi &e) {
  switch (block) {
    case 32: return launch_qk<XMODE, 32>(s, x, ldx, words, scales, M, N, K, e);
    case 64: return launch_qk<XMODE, 64>(s, x, ldx, words, scales, M, N, K, e);
    default: return launch_qk<XMODE, 128>(s, x, ldx, words, scales, M, N, K, e);
  }
}
}  // namespace

extern "C" int biq_q4_linear_qk_norm_rope(void *stream, const void *x, int x_dtype, int64_t B,
                                          int64_t S, int64_t K, int64_t ldx, const uint32_t *words,
                                          const float *scales, int block, int64_t Hq, int64_t Hkv,
                                          int64_t D, const float *q_gamma, const float *k_gamma,
                                          float q_eps, float k_eps, const float *cos,
                                          const float *sin, int64_t rope_batch, int out_dtype,
                                          int head_major, void *q_out, void *k_out, void *v_out) {
  biq::clear_error();
  if (!q_gamma || !k_gamma || !cos || !sin || !q_out || !k_out || !v_out)
    return biq::fail(BIQ_ERR_INVALID_ARG, "null pointer argument");
  if (B <= 0 || S <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused projection requires non-empty batch, tokens and heads");
  if (Hq % Hkv != 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "GQA query heads must be divisible by key/value heads");
  if (out_dtype != BIQ_DTYPE_F16 && out_dtype != BIQ_DTYPE_BF16)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused preparation output must be F16 or BF16");
  if (!(q_eps > 0.0f) || !(k_eps > 0.0f) || q_eps == INFINITY || k_eps == INFINITY)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused RMSNorm epsilon must be finite and positive");
  if (rope_batch != 1 && rope_batch != B)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused RoPE batch must be one or match the token batch");
  if (head_major != 0 && head_major != 1)
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused projection output layout must be 0 ([B, S, H, D]) or 1 ([B, H, S, D])");
  // the epilogue's buffer offsets are 32-bit: each output and the cos / sin tables must span less
  // than 2^31 bytes
  if (B > (1LL << 31) / S || Hq + 2 * Hkv > 32768 || B * S * Hq * D * 2 >= (1LL << 31) ||
      (rope_batch == B ? B * S : S) * D * 4 >= (1LL << 31))
    return biq::fail(BIQ_ERR_UNSUPPORTED, "fused projection: outputs or RoPE tables of 2 GiB or more");
  auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!al16(q_gamma) || !al16(k_gamma) || !al16(cos) || !al16(sin) || !al16(q_out) || !al16(k_out) ||
      !al16(v_out))
    return biq::fail(BIQ_ERR_INVALID_ARG, "fused projection: gamma, RoPE tables and outputs must be 16-byte aligned");
  const int64_t M = B * S, N = (Hq + 2 * Hkv) * D;
  const int st = check_linear(x, x_dtype, M, K, ldx, words, scales, BIQ_Q4_KN_AXIS1, block, N, q_out,
                             out_dtype);
  if (st != BIQ_OK) return st;
  if (D != 128)
    return biq::fail(BIQ_ERR_UNSUPPORTED, "fused projection + Q/K preparation needs 128-wide heads");
  if (x_dtype == BIQ_DTYPE_F32 || block < 32)
    return biq::fail(BIQ_ERR_UNSUPPORTED,
                     "fused projection + Q/K preparation needs 16-bit activations and blocks of at least 32");
  const QkEpi e{q_gamma, k_gamma, cos, sin, q_out, k_out, v_out, S, Hq, Hkv, rope_batch == B && B > 1 ? 1 : 0,
                out_dtype == BIQ_DTYPE_BF16 ? 1 : 0, head_major, q_eps, k_eps};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (x_dtype == BIQ_DTYPE_BF16) return launch_qk_blk<XM_BF16>(s, block, x, ldx, words, scales, M, N, K, e);
  return launch_qk_blk<XM_F16>(s, block, x, ldx, words, scales, M, N, K, e);
}
