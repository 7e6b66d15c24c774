// Host-only part of the rnsmx C ABI: error text, moduli constants, LUT.
#include <cstring>

#include "rnsmx_common.hpp"

namespace rnsmx {

static thread_local char g_error[512] = {0};

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = 0; }

static int64_t gcd64(int64_t a, int64_t b) {
  while (b) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Modular inverse of a modulo m (m <= 255, gcd(a, m) = 1) by search over the
// residues: at most 254 trials, host-side, once per moduli set.
static uint32_t inverse_mod(int64_t a, int64_t m) {
  const int64_t r = ((a % m) + m) % m;
  for (int64_t x = 1; x < m; ++x)
    if ((r * x) % m == 1) return static_cast<uint32_t>(x);
  return m == 1 ? 0u : 0xFFFFFFFFu;
}

}  // namespace rnsmx

extern "C" {

const char *rnsmx_last_error(void) { return rnsmx::g_error; }

int32_t rnsmx_abi_version(void) { return 5; }

int32_t rnsmx_moduli_init(const int32_t *moduli, int32_t channels,
                          rnsmx_moduli_t *out) {
  using namespace rnsmx;
  clear_error();
  if (!moduli || !out) return fail(RNSMX_EINVAL, "null argument");
  if (channels < 1) return fail(RNSMX_EINVAL, "moduli must not be empty");
  if (channels > RNSMX_MAX_CHANNELS) {
    set_error("at most %d channels are supported, got %d", RNSMX_MAX_CHANNELS,
              channels);
    return RNSMX_EINVAL;
  }
  for (int i = 0; i < channels; ++i)
    if (moduli[i] < 2 || moduli[i] > 255)
      return fail(RNSMX_EINVAL, "every modulus must be in [2, 255]");
  for (int i = 0; i < channels; ++i)
    for (int j = i + 1; j < channels; ++j)
      if (gcd64(moduli[i], moduli[j]) != 1) {
        set_error("moduli are not pairwise coprime: %d, %d", moduli[i],
                  moduli[j]);
        return RNSMX_EINVAL;
      }

  rnsmx_moduli_t r;
  std::memset(&r, 0, sizeof(r));
  r.channels = channels;
  // prefix[i] = prod_{j<i} m_j, checked against int64 overflow.
  r.prefix[0] = 1;
  for (int i = 0; i < channels; ++i) {
    const int64_t m = moduli[i];
    if (r.prefix[i] > INT64_MAX / m)
      return fail(RNSMX_ERANGE, "moduli product must fit signed int64");
    r.prefix[i + 1] = r.prefix[i] * m;
  }
  for (int i = 0; i < channels; ++i) {
    const int64_t m = moduli[i];
    r.moduli[i] = moduli[i];
    r.magic[i] = static_cast<uint32_t>((1ULL << 32) / static_cast<uint64_t>(m));
    r.c31[i] = static_cast<uint32_t>((1LL << 31) % m);
    const int64_t p_mod = r.prefix[i] % m;
    r.qinv[i] = inverse_mod(p_mod, m);
    // the Garner digit of channel i straight from its int32 sum v = a2 2^16 +
    // a1 2^8 + a0: v qinv_i = a2 qk16_i + a1 qk8_i + a0 qinv_i (mod m_i)
    const int64_t k16 = (65536 % m) * static_cast<int64_t>(r.qinv[i]) % m;
    r.qk16[i] = static_cast<int32_t>(2 * k16 > m ? k16 - m : k16);
    r.qk8[i] = static_cast<uint32_t>((256 % m) * static_cast<int64_t>(r.qinv[i]) % m);
    for (int j = 0; j < i; ++j) {
      const int64_t pj = r.prefix[j] % m;
      const int64_t t = (pj * static_cast<int64_t>(r.qinv[i])) % m;
      r.ucoef[j][i] = static_cast<uint32_t>((m - t) % m);
    }
  }
  *out = r;
  return RNSMX_OK;
}

int32_t rnsmx_compact_lut(const rnsmx_moduli_t *mods, int16_t *lut) {
  using namespace rnsmx;
  clear_error();
  if (!mods || !lut) return fail(RNSMX_EINVAL, "null argument");
  for (int c = 0; c < mods->channels; ++c) {
    const int64_t m = mods->moduli[c];
    int64_t weight = 1;  // 256^p mod m
    for (int p = 0; p < 4; ++p) {
      for (int b = 0; b < 256; ++b)
        lut[(c * 4 + p) * 256 + b] = static_cast<int16_t>((b * weight) % m);
      weight = (weight * 256) % m;
    }
  }
  return RNSMX_OK;
}

}  // extern "C"
