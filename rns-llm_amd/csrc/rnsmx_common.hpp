// Shared host-side helpers of the rnsmx library: error reporting and small
// integer utilities.  Device arithmetic lives in rnsmx_arith.hpp.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "rnsmx.h"

namespace rnsmx {

// Thread-local last-error text behind rnsmx_last_error().
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

inline int32_t fail(int32_t code, const char *what) {
  set_error("%s", what);
  return code;
}

inline int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// Largest |centered residue| of the set: floor(max(m) / 2).
inline int32_t max_half(const rnsmx_moduli_t &mods) {
  int32_t h = 0;
  for (int i = 0; i < mods.channels; ++i)
    if (mods.moduli[i] / 2 > h) h = mods.moduli[i] / 2;
  return h;
}

// Per-channel int32 accumulators of centered residues cannot overflow when
// K * max_half^2 <= 2^31 - 1 (the bound of cuda_backend.py:210-214, 240).
inline bool accumulator_fits(const rnsmx_moduli_t &mods, int64_t k) {
  const int64_t h = max_half(mods);
  return k * h * h <= 0x7FFFFFFFLL;
}

// The same bound when A enters the MFMA as raw int8 (|a| <= 128) against
// centered weight residues: K * 128 * max_half <= 2^31 - 1.
inline bool raw_accumulator_fits(const rnsmx_moduli_t &mods, int64_t k) {
  return k * 128 * static_cast<int64_t>(max_half(mods)) <= 0x7FFFFFFFLL;
}

// Packed weights: two products of centered residues (|.| <= max_half) by
// weight bytes (|.| <= 128) per K index, plus a per-row term below 256:
// 2 * K * 128 * max_half + 255 <= 2^31 - 1.
inline bool packed_accumulator_fits(const rnsmx_moduli_t &mods, int64_t k) {
  return k * 256 * static_cast<int64_t>(max_half(mods)) + 255 <= 0x7FFFFFFFLL;
}

}  // namespace rnsmx
