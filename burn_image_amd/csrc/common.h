// Shared helpers for the gfx950 kernels of libbiq: vector types, 16-bit conversions, MFMA
// wrappers and the thread-local error state of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/biq.h"

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Raw 16-bit element tags used as kernel template parameters.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

namespace biq {

// ---------------------------------------------------------------------------------------------
// error state (host)
// ---------------------------------------------------------------------------------------------
void set_error(const std::string &msg);
void clear_error();
int fail(int status, const std::string &msg);
// Check the launch status of the last kernel on this thread.
int check_launch(const char *what);
// Device scratch owned by the library for (current device, stream s), at least `bytes` long.
int stream_workspace(hipStream_t s, size_t bytes, void **out);
// A caller-fixed scratch region (device address and size) for launches that must not allocate.
struct Scratch {
  void *ptr;
  size_t bytes;
};
// Scratch of `bytes` for a launch on stream s: the fixed region when `fixed` is given (and large
// enough: BIQ_ERR_UNSUPPORTED otherwise), else the library's grow-only per-stream workspace.
int get_scratch(hipStream_t s, const Scratch *fixed, size_t bytes, void **out);
// Compute units of the current device.
int device_cu_count();

// ---------------------------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------------------------
template <typename T, typename F>
__device__ __forceinline__ T bitcast(const F &f) {
  static_assert(sizeof(T) == sizeof(F), "bitcast size");
  return __builtin_bit_cast(T, f);
}

__device__ __forceinline__ float bf16_lo_to_f32(uint32_t d) { return bitcast<float>(d << 16); }
__device__ __forceinline__ float bf16_hi_to_f32(uint32_t d) { return bitcast<float>(d & 0xffff0000u); }

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)bitcast<_Float16>(h);
}

// Round-to-nearest-even f32 -> bf16 bits (NaN stays NaN): gfx950's v_cvt_pk_bf16_f32, equal to
// the integer rounding (bits + 0x7fff + lsb) >> 16 for every finite input.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return bitcast<uint16_t>((__bf16)f);
}

// Two f32 -> packed bf16 pair (lo in bits 0-15), one conversion instruction.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
  f2_t v = {lo, hi};
  return bitcast<uint32_t>(__builtin_convertvector(v, b2_t));
}

// a / b correctly rounded, given inv = 1 / b correctly rounded: q = a * inv and one residual
// step, q + (a - q b) inv (Markstein's theorem).  Equal to IEEE division bit for bit whenever
// |a|, |b| and |a / b| lie in [2^-100, 2^100], and for a = 0 (checked on gfx950 against every f32
// numerator for six divisors and 2^32 random pairs); outside that range (numerators near the
// bottom of the normal range, subnormal quotients) the residual loses bits and the quotient can
// be one ulp off.  Three VALU operations against the ~10 of IEEE division.
// Pass b from rn_divisor: an infinite b enters as 0 (with inv = 0), which makes the step return
// a / inf exactly (signed zero; NaN for infinite or NaN a).  b = 0 with a nonzero gives NaN where
// division gives an infinity.
__device__ __forceinline__ float div_rn(float a, float b, float inv) {
  const float q = a * inv;
  return __builtin_fmaf(__builtin_fmaf(-q, b, a), inv, q);
}

// (b', 1 / b) for div_rn: b' = b, or 0 when 1 / b is 0.
__device__ __forceinline__ float2 rn_divisor(float b) {
  const float inv = 1.0f / b;
  return make_float2(inv == 0.0f ? 0.0f : b, inv);
}

// f32 -> f16 of the f32 value as it stands.  Without the empty asm, which only pins the value in
// a register, the compiler folds a preceding multiply into the conversion (v_fma_mixlo_f16: the
// exact product rounded once to f16), which differs from converting the f32 product wherever
// that lands on an f16 tie; the reference rounds to f32 first.
__device__ __forceinline__ _Float16 f16_of_f32(float v) {
  asm("" : "+v"(v));
  return (_Float16)v;
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  half2_t h = {(_Float16)lo, (_Float16)hi};
  return bitcast<uint32_t>(h);
}

__device__ __forceinline__ floatx16_t mfma32x32x16_f16(const half8_t &a, const half8_t &b,
                                                       const floatx16_t &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16_t mfma32x32x16_bf16(const bf16x8_t &a, const bf16x8_t &b,
                                                        const floatx16_t &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx16_t zero16() {
  floatx16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

}  // namespace biq
