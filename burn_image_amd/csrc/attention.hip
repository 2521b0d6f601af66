// Exact flash attention for gfx950 (online softmax, LDS-tiled K/V, 64-wide wavefronts).
//
// Replaces the forced BlackboxAccelerated cubek kernel (crates/burn_boogu/src/model/
// native_flash.rs:1006-1090) and Burn's attention op (patches/burn-cubecl-0.21.0/src/ops/
// module.rs:342-367) for non-causal joint image+text attention, and Qwen's causal / per-segment
// GQA attention (crates/burn_qwen3_vl/src/text.rs:146-185, vision.rs:344-386).
//
// Mapping onto v_mfma_f32_32x32x16_{bf16,f16} (one wave = 32 query rows):
//  * S^T = K . Q^T: A = a 32-key x 16-d slice of K from LDS, B = Q^T kept in registers.  The
//    32 x 32 accumulator gives each lane ONE query column (lane & 31) and 16 keys, so the row
//    max / sum of the online softmax are per-lane register reductions plus one exchange with
//    lane ^ 32.
//  * O^T = V^T . P^T: P^T leaves the S^T accumulator already shaped as the B operand (f16).  A
//    lane's 8 B slots hold keys {0-3, 8-11} (lanes 0-31) or {4-7, 12-15} (lanes 32-63) of each
//    16-key step, so V is stored transposed in LDS with bits 2 and 3 of the key index swapped;
//    one 16-byte LDS read then yields the matching A operand.
//  * Precision: Q K^T in bf16 (bf16 inputs) or f16 (f16/f32 inputs, the reference's F32->F16
//    bridge), exact products, f32 accumulation; f32 online softmax in base 2; P and V in f16
//    (u = 2^-11); f32 output accumulation; one final 1/l in f32.
#include <math.h>

#include <type_traits>

#include "common.h"

namespace {

constexpr int BKV = 64;      // keys per LDS tile
constexpr int VT_LD = BKV + 8;  // halves per row of the transposed V tile

// Mask bits: causal (key j > query i masked), segment (block-diagonal over cu_seqlens) and keys
// (a per-batch byte mask over the key sequence: Qwen's key-padding attention_mask, Burn's
// key-broadcast bool mask).
enum MaskMode { MASK_NONE = 0, MASK_CAUSAL = 1, MASK_SEGMENT = 2, MASK_CAUSAL_SEGMENT = 3, MASK_KEYS = 4 };

// Waves per workgroup (each wave owns 32 query rows; two waves per SIMD either way).  Non-causal
// forms run 8 waves (256 query rows) on each staged K/V tile, so a tile is loaded and written to
// LDS once for twice the queries of a 4-wave block (measured 7-10% faster unmasked at 4608 and
// 18944 tokens, 6-10% with per-segment masks).  Causal forms keep 4 waves (128 rows): a taller
// block widens the band of keys that only some of its rows see, and 8 waves measured 5% slower
// there (12% slower when waves also skipped the tiles none of their rows see).
constexpr int wg_waves(int mask) { return (mask & MASK_CAUSAL) ? 4 : 8; }

struct AttnArgs {
  const void *q, *k, *v;
  void *o;
  int64_t qs[3], ks[3], vs[3], os[3];  // batch, head, seq element strides
  int64_t B, Hq, Hkv, Sq, Skv, D;
  float scale_log2;  // softmax scale * log2(e)
  int out_dtype;
  const int32_t *cu;
  int64_t nseg;
  const uint8_t *km;   // key mask bytes [B, Skv] at batch stride km_stride (MASK_KEYS)
  int64_t km_stride;
  uint32_t km_drop;    // 1: a nonzero byte masks its key out; 0: a nonzero byte keeps it
  int fill_mean;       // rows with no visible key: 1 = mean of V over all keys, 0 = zeros
};

// Load 8 consecutive elements of type InT at p and return them as 8 16-bit values of the
// compute type (bf16 stays bf16 when COMPUTE_BF16, everything else becomes f16).
template <typename InT, bool COMPUTE_BF16>
__device__ __forceinline__ u32x4_t load8_compute(const InT *p) {
  if constexpr (sizeof(InT) == 2) {
    return *reinterpret_cast<const u32x4_t *>(p);
  } else {
    const float4 *f = reinterpret_cast<const float4 *>(p);
    float4 a = f[0], b = f[1];
    u32x4_t r;
    r[0] = biq::pack_f16x2(a.x, a.y);
    r[1] = biq::pack_f16x2(a.z, a.w);
    r[2] = biq::pack_f16x2(b.x, b.y);
    r[3] = biq::pack_f16x2(b.z, b.w);
    return r;
  }
}

// Physical position of key c inside its 16-key group of the transposed V tile (swap bits 2, 3).
__device__ __forceinline__ int vt_slot(int key) {
  return (key & ~15) | (key & 3) | ((key & 4) << 1) | ((key & 8) >> 1);
}

__device__ __forceinline__ int64_t segment_of(const int32_t *cu, int64_t nseg, int64_t i) {
  int64_t lo = 0, hi = nseg - 1;
  while (lo < hi) {
    int64_t mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= i) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Per-thread register copy of one K/V tile (prefetched while the previous tile computes).
template <int DP, typename InT, int NT>
struct KVRegs {
  static constexpr int K_CHUNKS = (BKV * DP / 8) / NT;  // 8-element K groups per thread
  static constexpr int V_GROUPS = (BKV / 4) * (DP / 8);       // 4-key x 8-dim V blocks per tile
  u32x4_t k16[K_CHUNKS];  // compute-type bits (f32 inputs are narrowed to f16 at load)
  u32x4_t v16[4];         // input bits (bf16 / f16; f32 inputs narrowed to f16 at load)
  uint32_t kmb;           // key-mask byte of key tid (wave 0, MASK_KEYS)
};

// 8 f32 at p -> 8 f16 packed (f32 inputs take the reference's F32 -> F16 bridge at load).
__device__ __forceinline__ u32x4_t load8_f32_as_f16(const float *p) {
  const float4 *f = reinterpret_cast<const float4 *>(p);
  const float4 a = f[0], b = f[1];
  return u32x4_t{biq::pack_f16x2(a.x, a.y), biq::pack_f16x2(a.z, a.w), biq::pack_f16x2(b.x, b.y),
                 biq::pack_f16x2(b.z, b.w)};
}

template <int DP, typename InT, int MASK>
__global__ void __launch_bounds__(64 * wg_waves(MASK), 8 / wg_waves(MASK)) attn_fwd_kernel(AttnArgs p) {
  constexpr int NT = 64 * wg_waves(MASK);  // threads per workgroup
  constexpr int BQ = 32 * wg_waves(MASK);  // query rows per workgroup
  constexpr bool BF16 = std::is_same<InT, bf16_t>::value;
  constexpr bool F32IN = sizeof(InT) == 4;
  constexpr int KS_LD = DP + 8;  // halves per row of the K tile
  constexpr int K_CHUNKS = KVRegs<DP, InT, NT>::K_CHUNKS;
  constexpr int V_GROUPS = KVRegs<DP, InT, NT>::V_GROUPS;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BKV * KS_LD];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][DP * VT_LD];
  __shared__ uint64_t Kbits[2];  // MASK_KEYS: bit t = key t of the staged tile may be attended

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, lh = lane >> 5;
  // ---- XCD-aware order: the hardware places workgroup i on XCD i % 8; give each XCD a
  //      contiguous run of (batch, head, query block) items, query blocks fastest, so the
  //      workgroups sharing one head's K/V also share one XCD's L2.
  int64_t h, b, qblk;
  {
    const int64_t nqb = (p.Sq + BQ - 1) / BQ;
    const int64_t T = nqb * p.Hq * p.B, L = blockIdx.x;
    const int64_t q8 = T / 8, r8 = T % 8, xcd = L % 8, slot = L / 8;
    const int64_t pid = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + slot;
    qblk = (pid % nqb) * BQ;
    h = (pid / nqb) % p.Hq;
    b = pid / (nqb * p.Hq);
  }
  const int64_t hk = h / (p.Hq / p.Hkv);
  const int64_t qi = qblk + wave * 32 + l32;  // this lane's query row
  const int64_t D = p.D;

  const InT *qg = reinterpret_cast<const InT *>(p.q) + b * p.qs[0] + h * p.qs[1];
  const InT *kg = reinterpret_cast<const InT *>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const InT *vg = reinterpret_cast<const InT *>(p.v) + b * p.vs[0] + hk * p.vs[1];

  // ---- Q^T fragments (B operand of S^T = K Q^T): lane holds d = 16 s + 8 lh .. +7 of row qi
  u32x4_t qf[DP / 16];
#pragma unroll
  for (int s = 0; s < DP / 16; ++s) {
    const int d0 = 16 * s + 8 * lh;
    if (qi < p.Sq && d0 < D)
      qf[s] = load8_compute<InT, BF16>(qg + qi * p.qs[2] + d0);
    else
      qf[s] = u32x4_t{0u, 0u, 0u, 0u};
  }
  // Q is in registers before the K/V pipeline starts: otherwise the loop's first MFMA, reached
  // from here with Q's loads in flight and from the back-edge with a K/V set in flight, makes
  // the compiler wait for every outstanding load at the top of each iteration.
  __builtin_amdgcn_s_waitcnt(0);

  // ---- key range of this workgroup and visibility bounds of this lane's query
  int64_t kv_begin = 0, kv_end = p.Skv;
  int64_t seg_lo = 0, seg_hi = p.Skv;
  if constexpr (MASK & MASK_SEGMENT) {
    // Every bound read from cu_seqlens is clamped to [0, Skv] and the range to begin <= end, so
    // the K/V descriptors below never start before the head or end past it, whatever cu holds
    // (the binary search itself only ever indexes cu[0 .. nseg]).
    auto clampk = [&](int64_t x) { return x < 0 ? (int64_t)0 : (x > p.Skv ? p.Skv : x); };
    const int64_t qc = qi < p.Sq ? qi : p.Sq - 1;
    const int64_t sg = segment_of(p.cu, p.nseg, qc);
    seg_lo = clampk(p.cu[sg]);
    seg_hi = clampk(p.cu[sg + 1]);
    const int64_t qlast = (qblk + BQ - 1) < p.Sq ? (qblk + BQ - 1) : p.Sq - 1;
    kv_begin = clampk(p.cu[segment_of(p.cu, p.nseg, qblk)]);
    kv_end = clampk(p.cu[segment_of(p.cu, p.nseg, qlast) + 1]);
    kv_end = kv_end < kv_begin ? kv_begin : kv_end;
  }
  if constexpr (MASK & MASK_CAUSAL) {
    const int64_t qlast = (qblk + BQ - 1) < p.Sq ? (qblk + BQ - 1) : p.Sq - 1;
    kv_end = kv_end < qlast + 1 ? kv_end : qlast + 1;
  }
  kv_begin = (kv_begin / BKV) * BKV;
  const int64_t qmin = qblk + wave * 32;  // this wave's first query row
  // Visible keys of this lane: [vis_lo, vis_hi) (segment and causal bounds, capped at Skv).  A
  // tile needs the mask unless it lies inside every lane's range of this wave.
  int64_t vis_lo = seg_lo, vis_hi = seg_hi < p.Skv ? seg_hi : p.Skv;
  if constexpr (MASK & MASK_CAUSAL) vis_hi = vis_hi < qi + 1 ? vis_hi : qi + 1;
  int64_t wave_lo = vis_lo, wave_hi = vis_hi;
  if constexpr (MASK != MASK_NONE) {
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
      const int64_t a = __shfl_xor(wave_lo, sh), c = __shfl_xor(wave_hi, sh);
      wave_lo = a > wave_lo ? a : wave_lo;  // largest lower bound
      wave_hi = c < wave_hi ? c : wave_hi;  // smallest upper bound
    }
  }

  // ---- global -> registers for the tile at kv0, through buffer loads.  The descriptor starts
  //      at the tile's first key and ends at key Skv, so rows past the sequence read as zero
  //      without a compare; chunks past the head width D get an offset beyond any range.  The
  //      per-thread offsets stay fixed; only the (scalar) descriptor moves from tile to tile.
  constexpr uint32_t OOB = 0x80000000u;
  constexpr int64_t ESZ = sizeof(InT);
  const int64_t krow_b = p.ks[2] * ESZ, vrow_b = p.vs[2] * ESZ;
  uint32_t koff[K_CHUNKS], voff[4];
#pragma unroll
  for (int it = 0; it < K_CHUNKS; ++it) {
    const int c = tid + it * NT;
    const int row = c / (DP / 8), d0 = 8 * (c % (DP / 8));
    koff[it] = d0 < D ? (uint32_t)(row * krow_b + d0 * ESZ) : OOB;
  }
  {
    const int kb = tid % (BKV / 4), d0 = 8 * (tid / (BKV / 4));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      voff[j] = (tid < V_GROUPS && d0 < D) ? (uint32_t)((4 * kb + j) * vrow_b + d0 * ESZ) : OOB;
  }
  auto rsrc = [&](const InT *base, int64_t kv0, int64_t row_b) {
    // valid offsets stay below 2^31 (host check), so capping the range there keeps OOB
    // offsets out of range for any sequence length
    // A prefetch past the last key (kv0 >= Skv) gets an empty range: every load reads zero.
    const int64_t rem = (p.Skv - kv0) * row_b;
    const uint32_t n = rem > 0x7fffffffLL ? 0x7fffffffu : (rem < 0 ? 0u : (uint32_t)rem);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<InT *>(base + kv0 * (row_b / ESZ)), 0,
                                             (int)n, 0x00020000);
  };
  auto load16 = [&](const __amdgpu_buffer_rsrc_t &r, uint32_t off) -> u32x4_t {
    if constexpr (F32IN) {
      const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
      const u32x4_t b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0);
      return u32x4_t{biq::pack_f16x2(biq::bitcast<float>(a[0]), biq::bitcast<float>(a[1])),
                     biq::pack_f16x2(biq::bitcast<float>(a[2]), biq::bitcast<float>(a[3])),
                     biq::pack_f16x2(biq::bitcast<float>(b[0]), biq::bitcast<float>(b[1])),
                     biq::pack_f16x2(biq::bitcast<float>(b[2]), biq::bitcast<float>(b[3]))};
    } else {
      return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    }
  };
  // Key-mask bytes: lane t of wave 0 loads the byte of key kv0 + t (a byte past Skv reads 0; such
  // keys are outside every visible range anyway).
  [[maybe_unused]] const uint8_t *kmrow = (MASK & MASK_KEYS) ? p.km + b * p.km_stride : nullptr;
  auto load_tile = [&](int64_t kv0, KVRegs<DP, InT, NT> &R) {
    if constexpr (MASK & MASK_KEYS) {
      const int64_t rem = p.Skv - kv0;
      const uint32_t n = rem <= 0 ? 0u : (rem > 0x7fffffffLL ? 0x7fffffffu : (uint32_t)rem);
      const auto rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(kmrow + kv0), 0, (int)n, 0x00020000);
      R.kmb = wave == 0 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rm, (uint32_t)lane, 0, 0) : 0u;
    }
    const auto rk = rsrc(kg, kv0, krow_b);
#pragma unroll
    for (int it = 0; it < K_CHUNKS; ++it) R.k16[it] = load16(rk, koff[it]);
    // V: thread owns keys 4 kb .. 4 kb + 3 at dims d0 .. d0 + 7 (key-consecutive lanes);
    // threads past V_GROUPS hold out-of-range offsets, so the loads need no branch
    const auto rv = rsrc(vg, kv0, vrow_b);
#pragma unroll
    for (int j = 0; j < 4; ++j) R.v16[j] = load16(rv, voff[j]);
  };

  // ---- registers -> LDS buffer: K row-major in the compute type, V transposed f16
  auto store_tile = [&](const KVRegs<DP, InT, NT> &R, int buf) {
    if constexpr (MASK & MASK_KEYS) {
      if (wave == 0) {
        const uint64_t bits = __ballot((R.kmb != 0u) != (p.km_drop != 0u));
        if (lane == 0) Kbits[buf] = bits;
      }
    }
#pragma unroll
    for (int it = 0; it < K_CHUNKS; ++it) {
      const int c = tid + it * NT;
      const int row = c / (DP / 8), d0 = 8 * (c % (DP / 8));
      *reinterpret_cast<u32x4_t *>(&Ks[buf][row * KS_LD + d0]) = R.k16[it];
    }
    if (tid < V_GROUPS) {
      const int kb = tid % (BKV / 4), d0 = 8 * (tid / (BKV / 4));
      // dim d0 + e of keys (j, j + 1) as one f16 pair: bf16 pairs convert two at a time, f16
      // pairs are a byte permute of the two source words
      const int slot = vt_slot(4 * kb);  // the 4 keys keep consecutive slots
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint32_t pr[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const uint32_t w0 = R.v16[2 * h2][e / 2], w1 = R.v16[2 * h2 + 1][e / 2];
          if constexpr (BF16) {
            const float f0 = (e & 1) ? biq::bf16_hi_to_f32(w0) : biq::bf16_lo_to_f32(w0);
            const float f1 = (e & 1) ? biq::bf16_hi_to_f32(w1) : biq::bf16_lo_to_f32(w1);
            pr[h2] = biq::pack_f16x2(f0, f1);
          } else {
            // bytes of (w0, w1): the low halves are bytes 0-1 / 4-5, the high halves 2-3 / 6-7
            pr[h2] = __builtin_amdgcn_perm(w1, w0, (e & 1) ? 0x07060302u : 0x05040100u);
          }
        }
        *reinterpret_cast<uint2 *>(&Vt[buf][(d0 + e) * VT_LD + slot]) = make_uint2(pr[0], pr[1]);
      }
    }
  };

  floatx16_t oacc[DP / 32];
#pragma unroll
  for (int i = 0; i < DP / 32; ++i) oacc[i] = biq::zero16();
  // m_run: reference maximum (log2 domain) the running sums are relative to; it only moves
  // when a new score exceeds it by more than 2^8, so most tiles skip the O rescale.
  float m_run = -INFINITY, l_run = 0.0f;

  // Two register sets (16-bit inputs): while tile t computes, set t % 2 receives tile t+2 and set (t+1) % 2
  // (loaded one tile earlier) is stored into the other LDS buffer at the end, so every load has
  // two tiles of compute to land.  Iterations go in pairs so both sets are named at compile time
  // (a copy of a register whose load is still in flight would make the wave wait for it).  An
  // odd tile count runs one more tile past the key range: every key of it is masked (outside
  // every lane's visible range), so it adds exact zeros -- skipping it instead would put a join
  // in the loop, where the compiler waits for the whole prefetch.
  // f32 inputs are narrowed to f16 as they load (which waits for them), and a second set would
  // not fit their registers: one set there.
  constexpr int NS = F32IN ? 1 : 2;
  KVRegs<DP, InT, NT> RS[NS];
  int buf = 0;
  if (kv_begin < kv_end) {
    load_tile(kv_begin, RS[0]);
    store_tile(RS[0], 0);
#pragma unroll
    for (int p1 = 1; p1 < NS; ++p1) load_tile(kv_begin + p1 * BKV, RS[p1]);
  }
  __syncthreads();

  for (int64_t kv00 = kv_begin; kv00 < kv_end; kv00 += NS * BKV) {
#pragma unroll
  for (int tt = 0; tt < NS; ++tt, buf ^= 1) {
    const int64_t kv0 = kv00 + tt * BKV;
    // The loads and LDS stores run unconditionally: past the key range the buffer loads return
    // zeros and a store lands in a buffer nobody reads again.  (A branch here makes the compiler
    // merge the prefetched registers at the join, which waits for the whole prefetch before the
    // first MFMA.)
    load_tile(kv0 + NS * BKV, RS[tt]);

    // ---- S^T = K Q^T for the tile's 64 keys (2 x 32).  The two 32-key halves are independent
    //      accumulator chains; d-steps outermost alternates them, so consecutive MFMAs never
    //      wait for each other's result.
    floatx16_t sacc[2] = {biq::zero16(), biq::zero16()};
#pragma unroll
    for (int s = 0; s < DP / 16; ++s) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const u32x4_t kf = *reinterpret_cast<const u32x4_t *>(
            &Ks[buf][(32 * ks + l32) * KS_LD + 16 * s + 8 * lh]);
        if constexpr (BF16)
          sacc[ks] = biq::mfma32x32x16_bf16(biq::bitcast<bf16x8_t>(kf), biq::bitcast<bf16x8_t>(qf[s]), sacc[ks]);
        else
          sacc[ks] = biq::mfma32x32x16_f16(biq::bitcast<half8_t>(kf), biq::bitcast<half8_t>(qf[s]), sacc[ks]);
      }
    }

    // ---- mask where the tile needs it; row max of the raw scores (the positive scale commutes
    //      with max, so it is applied once to the maximum and folded into the exponent's FMA)
    uint64_t kbits = ~0ull;
    if constexpr (MASK & MASK_KEYS) kbits = Kbits[buf];
    const bool need_mask = kv0 < wave_lo || kv0 + BKV > wave_hi || kbits != ~0ull;
    float mx = -INFINITY;
    if (need_mask) {
      // key offsets inside the tile are small: compare in 32 bits against this lane's bounds,
      // shifted by the lane's own key offset 4 lh
      const int64_t lo64 = vis_lo - kv0 - 4 * lh, hi64 = vis_hi - kv0 - 4 * lh;
      const int lo = lo64 < -BKV ? -BKV : (lo64 > 2 * BKV ? 2 * BKV : (int)lo64);
      const int hi = hi64 > 2 * BKV ? 2 * BKV : (hi64 < -BKV ? -BKV : (int)hi64);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        // this lane's 16 keys of the 32-key half ks sit at bits 8 g + e of m32 (g = r / 4, e = r % 4)
        const uint32_t m32 = (uint32_t)(kbits >> (32 * ks + 4 * lh));
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kr = 32 * ks + 8 * (r >> 2) + (r & 3);  // key offset without 4 lh
          bool ok = kr >= lo && kr < hi;
          if constexpr (MASK & MASK_KEYS) ok = ok && ((m32 >> (8 * (r >> 2) + (r & 3))) & 1u);
          sacc[ks][r] = ok ? sacc[ks][r] : -INFINITY;
          mx = fmaxf(mx, sacc[ks][r]);
        }
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[ks][r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32)) * p.scale_log2;  // log2 domain
    // ---- move the reference maximum only when it grows by more than 2^8 (exact: O and l
    //      are both relative to the same reference)
    const bool grow = mx > m_run + 8.0f;
    if (__any(grow)) {
      // Lanes that do not grow keep alpha = 1 exactly (their m_run may still be -inf when all
      // keys seen so far were masked, and -inf - -inf must not reach exp2).
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - mx) : 1.0f;  // 0 if m_run = -inf
      m_run = grow ? mx : m_run;
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < DP / 32; ++i) oacc[i] *= alpha;
    }
    const float neg_m = m_run == -INFINITY ? 0.0f : -m_run;
    // p = 2^(s * scale_log2 - m) with one FMA; the row sum adds the f16-rounded p (the values
    // the P V product uses) with v_dot2 against ones, two per instruction into f32
    const half2_t ones = {(_Float16)1.0f, (_Float16)1.0f};
    float rs = 0.0f;
    u32x4_t pf[4];  // P^T as f16 B operands of the four 16-key steps
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[ks][8 * t + 2 * j], p.scale_log2, neg_m));
          const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[ks][8 * t + 2 * j + 1], p.scale_log2, neg_m));
          const uint32_t pk = biq::pack_f16x2(e0, e1);
          pf[2 * ks + t][j] = pk;
          rs = __builtin_amdgcn_fdot2(biq::bitcast<half2_t>(pk), ones, rs, false);
        }
    l_run += rs;

    // ---- O^T += V^T P^T
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const half8_t bp = biq::bitcast<half8_t>(pf[t]);
#pragma unroll
      for (int i = 0; i < DP / 32; ++i) {
        const half8_t av = *reinterpret_cast<const half8_t *>(
            &Vt[buf][(32 * i + l32) * VT_LD + 16 * t + 8 * lh]);
        oacc[i] = biq::mfma32x32x16_f16(av, bp, oacc[i]);
      }
    }

    store_tile(RS[(tt + 1) % NS], buf ^ 1);
    __syncthreads();
  }
  }

  // ---- normalise and store O[b, h, qi, d]
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  // Rows with no visible key (only a key mask can empty a row: causal and segment ranges hold the
  // query's own key).  With fill_mean they take the mean of V over all Skv keys, the softmax of a
  // row filled with one constant everywhere.  Cold path: the wave sums V cooperatively, lane L
  // owning dims 2L and 2L + 1, then each empty lane gathers its dims by lane shuffles.
  [[maybe_unused]] bool empty_row = false;
  [[maybe_unused]] float mean0 = 0.0f, mean1 = 0.0f;
  if constexpr (MASK & MASK_KEYS) {
    empty_row = p.fill_mean && qi < p.Sq && !(l_tot > 0.0f);
    if (__any(empty_row)) {
      float s0 = 0.0f, s1 = 0.0f;
      const int64_t dd = 2 * lane;
      if (dd < D) {
        const InT *vc = vg + dd;
        for (int64_t j = 0; j < p.Skv; ++j) {
          const InT *e = vc + j * p.vs[2];
          if constexpr (F32IN) {
            s0 += e[0];
            s1 += e[1];
          } else {
            const uint32_t w = *reinterpret_cast<const uint32_t *>(e);
            if constexpr (BF16) {
              s0 += biq::bf16_lo_to_f32(w);
              s1 += biq::bf16_hi_to_f32(w);
            } else {
              s0 += (float)biq::bitcast<half2_t>(w)[0];
              s1 += (float)biq::bitcast<half2_t>(w)[1];
            }
          }
        }
      }
      const float invn = 1.0f / (float)p.Skv;
      mean0 = s0 * invn;
      mean1 = s1 * invn;
    }
  }
  // Lanes past the sequence stay until the end: the empty-row fill gathers dims from every lane.
  const bool row_in = qi < p.Sq;
  if (!(MASK & MASK_KEYS) && !row_in) return;
  char *ob = reinterpret_cast<char *>(p.o);
  const int64_t obase = b * p.os[0] + h * p.os[1] + qi * p.os[2];
#pragma unroll
  for (int i = 0; i < DP / 32; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * i + 8 * g + 4 * lh;
      if (d0 >= D) continue;
      float v0 = oacc[i][4 * g] * inv, v1 = oacc[i][4 * g + 1] * inv;
      float v2 = oacc[i][4 * g + 2] * inv, v3 = oacc[i][4 * g + 3] * inv;
      if constexpr (MASK & MASK_KEYS) {
        // dims d0 .. d0 + 3 live in lanes d0 / 2 (d0, d0 + 1) and d0 / 2 + 1 (d0 + 2, d0 + 3)
        const float a0 = __shfl(mean0, d0 / 2), a1 = __shfl(mean1, d0 / 2);
        const float a2 = __shfl(mean0, d0 / 2 + 1), a3 = __shfl(mean1, d0 / 2 + 1);
        if (empty_row) { v0 = a0; v1 = a1; v2 = a2; v3 = a3; }
      }
      if (!row_in) continue;
      if (p.out_dtype == BIQ_DTYPE_F32) {
        float *dst = reinterpret_cast<float *>(ob) + obase + d0;
        *reinterpret_cast<float4 *>(dst) = make_float4(v0, v1, v2, v3);
      } else if (p.out_dtype == BIQ_DTYPE_F16) {
        uint16_t *dst = reinterpret_cast<uint16_t *>(ob) + obase + d0;
        uint2 w = make_uint2(biq::pack_f16x2(v0, v1), biq::pack_f16x2(v2, v3));
        *reinterpret_cast<uint2 *>(dst) = w;
      } else {
        uint16_t *dst = reinterpret_cast<uint16_t *>(ob) + obase + d0;
        uint2 w = make_uint2(biq::pack_bf16x2(v0, v1), biq::pack_bf16x2(v2, v3));
        *reinterpret_cast<uint2 *>(dst) = w;
      }
    }
}

template <int DP, typename InT, int MASK>
void launch_one(hipStream_t s, dim3 grid, const AttnArgs &a) {
  hipLaunchKernelGGL((attn_fwd_kernel<DP, InT, MASK>), grid, dim3(64 * wg_waves(MASK)), 0, s, a);
}

template <int DP, typename InT>
void launch_mask(hipStream_t s, dim3 grid, const AttnArgs &a, int mask) {
  switch (mask) {
    case MASK_NONE: launch_one<DP, InT, MASK_NONE>(s, grid, a); break;
    case MASK_CAUSAL: launch_one<DP, InT, MASK_CAUSAL>(s, grid, a); break;
    case MASK_SEGMENT: launch_one<DP, InT, MASK_SEGMENT>(s, grid, a); break;
    case MASK_CAUSAL_SEGMENT: launch_one<DP, InT, MASK_CAUSAL_SEGMENT>(s, grid, a); break;
    case MASK_KEYS: launch_one<DP, InT, MASK_KEYS>(s, grid, a); break;
    case MASK_KEYS | MASK_CAUSAL: launch_one<DP, InT, MASK_KEYS | MASK_CAUSAL>(s, grid, a); break;
    case MASK_KEYS | MASK_SEGMENT: launch_one<DP, InT, MASK_KEYS | MASK_SEGMENT>(s, grid, a); break;
    default: launch_one<DP, InT, MASK_KEYS | MASK_CAUSAL_SEGMENT>(s, grid, a); break;
  }
}

template <int DP>
void launch_dtype(hipStream_t s, dim3 grid, const AttnArgs &a, int in_dtype, int mask) {
  if (in_dtype == BIQ_DTYPE_BF16) launch_mask<DP, bf16_t>(s, grid, a, mask);
  else if (in_dtype == BIQ_DTYPE_F16) launch_mask<DP, f16_t>(s, grid, a, mask);
  else launch_mask<DP, float>(s, grid, a, mask);
}

}  // namespace

extern "C" int biq_attention(void *stream, const void *q, const void *k, const void *v, void *o,
                             int in_dtype, int out_dtype, int64_t B, int64_t Hq, int64_t Hkv,
                             int64_t Sq, int64_t Skv, int64_t D, const int64_t *q_strides,
                             const int64_t *k_strides, const int64_t *v_strides,
                             const int64_t *o_strides, float scale, int causal,
                             const int32_t *cu_seqlens, int64_t nseg, const uint8_t *key_mask,
                             int64_t key_mask_stride, int key_mask_mode) {
  biq::clear_error();
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides)
    return biq::fail(BIQ_ERR_INVALID_ARG, "null pointer argument");
  if (in_dtype != BIQ_DTYPE_F32 && in_dtype != BIQ_DTYPE_F16 && in_dtype != BIQ_DTYPE_BF16)
    return biq::fail(BIQ_ERR_INVALID_ARG, "attention input dtype must be F32, F16 or BF16");
  if (out_dtype != BIQ_DTYPE_F32 && out_dtype != BIQ_DTYPE_F16 && out_dtype != BIQ_DTYPE_BF16)
    return biq::fail(BIQ_ERR_INVALID_ARG, "attention output dtype must be F32, F16 or BF16");
  if (B <= 0 || Hq <= 0 || Hkv <= 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "attention batch and heads must be non-zero");
  if (Sq <= 0) return biq::fail(BIQ_ERR_INVALID_ARG, "attention query sequence must be non-empty");
  if (Skv <= 0) return biq::fail(BIQ_ERR_INVALID_ARG, "attention key sequence must be non-empty");
  if (Hq % Hkv != 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "GQA query heads must be divisible by key/value heads");
  if (D <= 0 || D > 128 || D % 8 != 0)
    return biq::fail(BIQ_ERR_UNSUPPORTED, "attention head width must be a multiple of 8 up to 128");
  if ((causal || cu_seqlens) && Sq != Skv)
    return biq::fail(BIQ_ERR_INVALID_ARG, "causal and segment masks require Sq == Skv");
  if (cu_seqlens && nseg <= 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "segment mask requires at least one segment");
  if (key_mask && key_mask_mode != BIQ_KEY_MASK_VALID && key_mask_mode != BIQ_KEY_MASK_VALID_FILL_MEAN &&
      key_mask_mode != BIQ_KEY_MASK_MASKED)
    return biq::fail(BIQ_ERR_INVALID_ARG, "unknown key mask mode");
  if (key_mask && key_mask_stride < 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "key mask batch stride must be non-negative");
  const int esz = in_dtype == BIQ_DTYPE_F32 ? 4 : 2;
  const int osz = out_dtype == BIQ_DTYPE_F32 ? 4 : 2;
  const int64_t *st[3] = {q_strides, k_strides, v_strides};
  const void *ptr[3] = {q, k, v};
  for (int t = 0; t < 3; ++t) {
    if (reinterpret_cast<uintptr_t>(ptr[t]) & 15)
      return biq::fail(BIQ_ERR_INVALID_ARG, "attention inputs must be 16-byte aligned");
    for (int j = 0; j < 3; ++j)
      if (((st[t][j] * esz) & 15) != 0)
        return biq::fail(BIQ_ERR_INVALID_ARG, "attention strides must be multiples of 16 bytes");
  }
  if (reinterpret_cast<uintptr_t>(o) & 15)
    return biq::fail(BIQ_ERR_INVALID_ARG, "attention output must be 16-byte aligned");
  for (int j = 0; j < 3; ++j)
    if (((o_strides[j] * osz) & 15) != 0)
      return biq::fail(BIQ_ERR_INVALID_ARG, "attention output strides must be multiples of 16 bytes");
  if (k_strides[2] * esz * BKV >= (1LL << 31) || v_strides[2] * esz * BKV >= (1LL << 31))
    return biq::fail(BIQ_ERR_UNSUPPORTED, "attention key/value row stride too large for 32-bit tile offsets");
  const int mask = (causal ? MASK_CAUSAL : 0) | (cu_seqlens ? MASK_SEGMENT : 0) | (key_mask ? MASK_KEYS : 0);
  const int64_t bq = 32 * wg_waves(mask);
  if ((Sq + bq - 1) / bq * Hq * B > 0x7fffffffLL)
    return biq::fail(BIQ_ERR_UNSUPPORTED, "attention grid too large");

  AttnArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o;
  for (int j = 0; j < 3; ++j) {
    a.qs[j] = q_strides[j]; a.ks[j] = k_strides[j]; a.vs[j] = v_strides[j]; a.os[j] = o_strides[j];
  }
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.Sq = Sq; a.Skv = Skv; a.D = D;
  const double sc = scale > 0.0f ? (double)scale : 1.0 / sqrt((double)D);
  a.scale_log2 = (float)(sc * 1.4426950408889634);
  a.out_dtype = out_dtype;
  a.cu = cu_seqlens;
  a.nseg = nseg;
  a.km = key_mask;
  a.km_stride = key_mask_stride;
  a.km_drop = key_mask_mode == BIQ_KEY_MASK_MASKED ? 1u : 0u;
  a.fill_mean = key_mask_mode == BIQ_KEY_MASK_VALID_FILL_MEAN ? 1 : 0;
  dim3 grid((unsigned)((Sq + bq - 1) / bq * Hq * B));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (D <= 64) launch_dtype<64>(s, grid, a, in_dtype, mask);
  else launch_dtype<128>(s, grid, a, in_dtype, mask);
  return biq::check_launch("attention");
}

// Burn's ModuleOps::attention (patches/burn-cubecl-0.21.0/src/ops/module.rs:342-367).
extern "C" int biq_attention_burn(void *stream, const void *q, const void *k, const void *v, void *o,
                                  int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                  int64_t Skv, int64_t D, const int64_t *q_strides,
                                  const int64_t *k_strides, const int64_t *v_strides,
                                  const int64_t *o_strides, const uint8_t *mask,
                                  const int64_t *mask_strides, const void *attn_bias, int is_causal,
                                  int has_scale, float scale, int has_softcap, float softcap) {
  biq::clear_error();
  (void)softcap;
  if (attn_bias)
    return biq::fail(BIQ_ERR_UNSUPPORTED, "attention: an additive attn_bias is not supported by the flash kernel");
  if (has_softcap)
    return biq::fail(BIQ_ERR_UNSUPPORTED, "attention: softcap is not supported by the flash kernel");
  if (has_scale && !(scale > 0.0f))
    return biq::fail(BIQ_ERR_INVALID_ARG, "attention: an explicit scale must be positive");
  int64_t km_stride = 0;
  if (mask) {
    if (!mask_strides) return biq::fail(BIQ_ERR_INVALID_ARG, "attention: mask strides missing");
    // only a key-padding mask, broadcast over heads and query rows, maps onto the kernel
    if (mask_strides[1] != 0 || mask_strides[2] != 0 || (Skv > 1 && mask_strides[3] != 1))
      return biq::fail(BIQ_ERR_UNSUPPORTED,
                       "attention: only key-padding masks (broadcast over heads and queries, keys contiguous) are supported");
    km_stride = B > 1 ? mask_strides[0] : 0;
  }
  return biq_attention(stream, q, k, v, o, dtype, dtype, B, Hq, Hkv, Sq, Skv, D, q_strides, k_strides,
                       v_strides, o_strides, has_scale ? scale : 0.0f, is_causal, nullptr, 0, mask,
                       km_stride, BIQ_KEY_MASK_MASKED);
}
