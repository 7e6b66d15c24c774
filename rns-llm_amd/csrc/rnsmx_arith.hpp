// Device-side modular arithmetic for the rnsmx kernels.
//
// Reduction follows Barrett (1986): for a 32-bit x and magic = floor(2^32/m),
// q = mulhi(x, magic) is floor(x/m) or floor(x/m) - 1, so x - q*m lies in
// [0, 2m) and one conditional subtraction finishes.  Signed 32-bit values are
// biased by 2^31 (an exact XOR of the sign bit) so every int32, including
// INT32_MIN, reduces without a magnitude/negate step; the bias is removed
// with the precomputed 2^31 mod m.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>
#include <utility>

#include "rnsmx.h"

namespace rnsmx {

// Compile-time loop: f(std::integral_constant<int, I>) for I in [0, N).
template <int N, typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F &&f,
                                                std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl<N>(static_cast<F &&>(f), std::make_integer_sequence<int, N>{});
}

// x mod m for any 32-bit x.
__device__ __forceinline__ uint32_t mod_u32(uint32_t x, uint32_t m, uint32_t magic) {
  const uint32_t q = __umulhi(x, magic);
  const uint32_t r = x - q * m;
  return r >= m ? r - m : r;
}

// x mod m for 0 <= x < 2^24 with 24-bit multiplies (full rate on CDNA;
// 32-bit integer multiplies are quarter rate).  m24 = floor(2^24 / m).
// Writing 2^24/m = m24 + f with 0 <= f < 1, x*m24/2^24 = x/m - x*f/2^24 and
// x*f/2^24 < 1, so q = floor(x*m24/2^24) is floor(x/m) or floor(x/m) - 1 and
// x - q*m lies in [0, 2m): one conditional subtraction finishes.  q <= m24
// <= 2^23 - 1 for m >= 2 (x < 2^24), so x - q*m is one signed 24-bit
// multiply-add (the unsigned form is selected as a 32-bit multiply).
// negm = -m, precomputed by the caller.
__device__ __forceinline__ uint32_t mod_small(uint32_t x, uint32_t m, uint32_t m24, int32_t negm) {
  const uint64_t p = static_cast<uint64_t>(x & 0xFFFFFFu) * static_cast<uint64_t>(m24 & 0xFFFFFFu);
  const int32_t q = static_cast<int32_t>(p >> 24);
  const uint32_t r = static_cast<uint32_t>(static_cast<int32_t>(x) + __mul24(q, negm));
  return min(r, r - m);  // r < m: r - m wraps above r
}

// Constants of the 24-bit reduction of one modulus, all derived from
// magic = floor(2^32 / m) (floor(2^k / m) = magic >> (32 - k)).
struct FastMod {
  uint32_t m;     // modulus, 2 <= m <= 255
  uint32_t m24;   // floor(2^24 / m)
  uint32_t c16;   // 2^16 mod m
  uint32_t bias;  // m * floor(2^23 / m), a multiple of m in (2^23 - m, 2^23]
  int32_t negm;   // -m
};

__device__ __forceinline__ FastMod fast_mod_of(uint32_t m, uint32_t magic) {
  return FastMod{m, magic >> 8, 65536u - (magic >> 16) * m, m * (magic >> 9), -static_cast<int32_t>(m)};
}

// Canonical residue in [0, m) of any int32 v.  v = hi * 2^16 + lo with
// hi = v >> 16 in [-2^15, 2^15) and lo in [0, 2^16), so v = hi * c16 + lo
// (mod m).  hi * c16 lies in [-32768 * 254, 32767 * 254]; adding
// bias >= 2^23 - 255 > 32768 * 254 makes t non-negative, and
// t <= 32767 * 254 + 65535 + 2^23 = 16,776,961 < 2^24, the domain of
// mod_small.  Every multiply is 24-bit.
__device__ __forceinline__ uint32_t canon_fast(int32_t v, const FastMod &f) {
  const int32_t hi = v >> 16;
  const uint32_t lo = static_cast<uint32_t>(v) & 0xFFFFu;
  const uint32_t t = static_cast<uint32_t>(__mul24(hi, static_cast<int32_t>(f.c16))) + lo + f.bias;
  return mod_small(t, f.m, f.m24, f.negm);
}

// Canonical residue in [0, m) of a signed 32-bit value.
__device__ __forceinline__ uint32_t canon_i32(int32_t v, uint32_t m, uint32_t magic,
                                              uint32_t c31) {
  const uint32_t r = mod_u32(static_cast<uint32_t>(v) ^ 0x80000000u, m, magic);
  return r >= c31 ? r - c31 : r + m - c31;
}

// Centered residue in [-floor(m/2), floor(m/2)] of a signed 32-bit value.
__device__ __forceinline__ int32_t centered_i32(int32_t v, uint32_t m, uint32_t magic,
                                                uint32_t c31) {
  const uint32_t r = canon_i32(v, m, magic, c31);
  return r > (m >> 1) ? static_cast<int32_t>(r) - static_cast<int32_t>(m)
                      : static_cast<int32_t>(r);
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int t) {
  return (w >> (8 * t)) & 0xFFu;
}

// Round-to-nearest-even float -> bfloat16 bits (finite inputs; NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu))
    return static_cast<uint16_t>((u >> 16) | 0x40u);
  const uint32_t lsb = (u >> 16) & 1u;
  return static_cast<uint16_t>((u + 0x7FFFu + lsb) >> 16);
}

}  // namespace rnsmx
