// float8 streams of the Bayes-layer kernels: the OCP e4m3fn and e5m2
// encodings that torch names float8_e4m3fn and float8_e5m2 (the encodings
// gfx950's conversion instructions read).
//
// Widening (float8 -> float32) is exact and done by the hardware.  Narrowing
// (float32 -> float8, for the gradients of float8 inputs) rounds to nearest
// even exactly as torch's conversion does, including its overflow rules
// (float_to_f8 states them; narrow_f8 uses the hardware conversion, which
// agrees except for NaN):
//   e4m3fn (4 exponent bits, bias 7, 3 mantissa bits, no infinities):
//     magnitudes that round past 448 give the NaN code 0x7f (with the sign);
//   e5m2 (5 exponent bits, bias 15, 2 mantissa bits): they give infinity;
// NaN gives the NaN code 0x7f with the sign.  The same template runs on the
// host (bssm_round_float8) so the rounding can be checked against torch.

#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

#include <hip/hip_runtime.h>

namespace bssm {

// Input formats of keys, queries and values (and of their gradients).
enum InFmt : int { kInF32 = 0, kInBf16 = 1, kInE4M3 = 2, kInE5M2 = 3 };

template <int F>
__host__ __device__ inline uint32_t float_to_f8(float x) {
  static_assert(F == kInE4M3 || F == kInE5M2, "float8 formats only");
  constexpr int MB = F == kInE4M3 ? 3 : 2;            // mantissa bits
  constexpr int BIAS = F == kInE4M3 ? 7 : 15;         // exponent bias
  constexpr uint32_t kTop = F == kInE4M3 ? 0x7fu : 0x7cu;  // NaN (e4m3fn) / infinity (e5m2)
  constexpr float kSub = F == kInE4M3 ? 512.f : 65536.f;   // 1 / smallest subnormal
  uint32_t bits;
#if defined(__HIP_DEVICE_COMPILE__)
  bits = __builtin_bit_cast(uint32_t, x);
#else
  std::memcpy(&bits, &x, 4);
#endif
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t a = bits & 0x7fffffffu;
  uint32_t code;
  if (a > 0x7f800000u) {
    code = 0x7fu;
  } else if (a >= (static_cast<uint32_t>(128 - BIAS) << 23)) {
    // Normal in the target: re-bias the exponent, keep MB mantissa bits and
    // round the dropped ones to nearest even (a carry moves into the exponent).
    constexpr int SH = 23 - MB;
    uint32_t c = (((a >> 23) - (127 - BIAS)) << MB) | ((a >> SH) & ((1u << MB) - 1u));
    const uint32_t rem = a & ((1u << SH) - 1u), half = 1u << (SH - 1);
    c += (rem > half || (rem == half && (c & 1u))) ? 1u : 0u;
    code = c < kTop ? c : kTop;
  } else {
    // Subnormal (or zero) in the target: a multiple of the smallest
    // subnormal, rounded to nearest even; 2^MB is the smallest normal code.
    code = static_cast<uint32_t>(rintf(fabsf(x) * kSub));
  }
  return sign | code;
}

#if defined(__HIPCC__)
typedef float f8v4f __attribute__((ext_vector_type(4)));
typedef float f8v2f __attribute__((ext_vector_type(2)));

// Four float8 values of one 32-bit word (first value in the low byte) to float32.
template <int F>
__device__ __forceinline__ f8v4f widen_f8(uint32_t w) {
  f8v2f lo, hi;
  if constexpr (F == kInE4M3) {
    lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
    hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  } else {
    lo = __builtin_amdgcn_cvt_pk_f32_bf8(static_cast<int>(w), false);
    hi = __builtin_amdgcn_cvt_pk_f32_bf8(static_cast<int>(w), true);
  }
  return f8v4f{lo[0], lo[1], hi[0], hi[1]};
}

// Four float32 values to one word of float8 (first value in the low byte).
// gfx950's conversion (round to nearest even, OCP overflow rules) gives
// torch's codes for every non-NaN input (checked on the whole bfloat16 grid,
// the ties around every float8 value and random values); it writes NaN as a
// negative NaN code whatever the sign, so a word with a NaN input is redone
// by float_to_f8 (a branch no wave takes unless a gradient is NaN).
template <int F>
__device__ __forceinline__ uint32_t narrow_f8(f8v4f x) {
  int w;
  if constexpr (F == kInE4M3) {
    w = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], w, true);
  } else {
    w = __builtin_amdgcn_cvt_pk_bf8_f32(x[0], x[1], 0, false);
    w = __builtin_amdgcn_cvt_pk_bf8_f32(x[2], x[3], w, true);
  }
  uint32_t r = static_cast<uint32_t>(w);
  if (__builtin_isnan(x[0]) | __builtin_isnan(x[1]) | __builtin_isnan(x[2]) | __builtin_isnan(x[3]))
    r = float_to_f8<F>(x[0]) | (float_to_f8<F>(x[1]) << 8) | (float_to_f8<F>(x[2]) << 16) |
        (float_to_f8<F>(x[3]) << 24);
  return r;
}
#endif

}  // namespace bssm
