// rnsmx device code for gfx950 (MI355X): residue encode, per-channel int8
// MFMA GEMM with the fused modular-reduction + Garner (+ dequant) epilogue,
// device-side adaptive channel prefix, Garner decode and operand repacking.
//
// Data layout in HBM
//   residue planes   [R][rows][ld] int8, K contiguous, ld a multiple of 64
//                    and bytes [K, ld) zero, so every MFMA fragment is one
//                    aligned 16-byte load and the K loop needs no tail.
//   prepared weight  [R][N][kp]: B stored K-contiguous (the nn.Linear weight
//                    orientation); the reference keeps [R][K][N]
//                    (cuda_backend.py:68-76, rns_linear.py:185).
//   output           [M][N] int64 (exact) or float32/float16/bfloat16.
//
// MFMA: v_mfma_i32_16x16x64_i8.  Lane l of a wave feeds A row (l & 15) and B
// column (l & 15), both with K bytes [16 * (l >> 4), +16) of a 64-byte step,
// and receives D rows 4 * (l >> 4) + t (t = 0..3) of column (l & 15).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>

#include "rnsmx_arith.hpp"
#include "rnsmx_common.hpp"

namespace rnsmx {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Argument blocks (passed by value; kernarg memory)
// ---------------------------------------------------------------------------
struct GemmArgs {
  const int8_t *a;  // [R][M][a_ld]
  int64_t a_ld, a_cs;
  const int8_t *b;  // [R][N][b_ld]
  int64_t b_ld, b_cs;
  int32_t m, n, kp;  // kp: multiple of 64, <= a_ld, b_ld
  int32_t lut_channels;
  const int16_t *lut;  // [R][4][256]
  // adaptive prefix
  int32_t min_channels;  // 0: all channels
  const int64_t *row_l1;
  const int32_t *w_absmax;
  int64_t *meta;
  // epilogue
  void *out;
  int64_t out_ld;
  int32_t out_dtype;
  const float *a_scale;
  const float *w_scale;
  const float *bias;
  rnsmx_moduli_t mods;
};

struct EncodeArgs {
  const void *values;
  int64_t rows, cols, out_ld, plane;
  int8_t *out;
  int64_t *row_l1;
  int32_t *absmax;
  rnsmx_moduli_t mods;
};

// ---------------------------------------------------------------------------
// Helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t wave_max_i64(int64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int64_t o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Number of moduli channels to use.  Without the adaptive prefix this is the
// full set.  With it, every workgroup derives the same answer from the row
// L1 norms written by the encoder and max|B| written at weight preparation:
// bound = max_i sum_k |a_ik| * max|B| (adaptive.py:44-52); the answer is the
// smallest c >= min_channels with 2 * bound < prod_{i<c} m_i
// (adaptive.py:15-41), i.e. bound <= (P_c - 1) / 2.  When no prefix fits,
// the full set is used and meta[3] flags the overflow (the reference raises
// OverflowError on the host, which a device-side selector cannot).
__device__ int active_channels(const GemmArgs &g, int64_t *red, int *bcast) {
  const int full = g.mods.channels;
  if (g.min_channels <= 0) return full;
  int64_t mx = 0;
  for (int r = threadIdx.x; r < g.m; r += blockDim.x) {
    const int64_t v = g.row_l1[r];
    mx = v > mx ? v : mx;
  }
  mx = wave_max_i64(mx);
  const int nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t best = 0;
    for (int w = 0; w < nw; ++w) best = red[w] > best ? red[w] : best;
    const int64_t wmax = *g.w_absmax;
    const int64_t bound =
        (wmax != 0 && best > LLONG_MAX / wmax) ? LLONG_MAX : best * wmax;
    int c = full, overflow = 1;
    for (int i = g.min_channels; i <= full; ++i) {
      if (bound <= (g.mods.prefix[i] - 1) / 2) {
        c = i;
        overflow = 0;
        break;
      }
    }
    *bcast = c;
    if (g.meta != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
      g.meta[0] = c;
      g.meta[1] = bound;
      g.meta[2] = (g.mods.prefix[c] - 1) / 2;
      g.meta[3] = overflow;
    }
  }
  __syncthreads();
  return *bcast;
}

// Final value of one output element from its mixed-radix digits, centered
// about P_c / 2, written in the requested output type.  The float chain is
// ((float)x * a_scale) * w_scale[col] + bias[col], each step rounded to
// nearest even with no contraction: the op order of rns_linear.py:272-275.
template <int RCAP>
__device__ __forceinline__ void store_element(const GemmArgs &g, int c_act,
                                              const uint32_t (&d)[RCAP], int row,
                                              int col) {
  uint64_t x = 0;
#pragma unroll
  for (int c = 0; c < RCAP; ++c)
    if (c < c_act) x += static_cast<uint64_t>(d[c]) * static_cast<uint64_t>(g.mods.prefix[c]);
  const int64_t p = g.mods.prefix[c_act];
  int64_t y = static_cast<int64_t>(x);
  if (y > (p >> 1)) y -= p;
  const int64_t idx = static_cast<int64_t>(row) * g.out_ld + col;
  if (g.out_dtype == RNSMX_INT64) {
    static_cast<int64_t *>(g.out)[idx] = y;
    return;
  }
  float f = __ll2float_rn(y);
  f = __fmul_rn(f, *g.a_scale);
  f = __fmul_rn(f, g.w_scale[col]);
  if (g.bias != nullptr) f = __fadd_rn(f, g.bias[col]);
  if (g.out_dtype == RNSMX_FLOAT32) {
    static_cast<float *>(g.out)[idx] = f;
  } else if (g.out_dtype == RNSMX_FLOAT16) {
    static_cast<__half *>(g.out)[idx] = __float2half_rn(f);
  } else {
    static_cast<uint16_t *>(g.out)[idx] = f32_to_bf16_rne(f);
  }
}

// Mixed-radix digit of channel C from its canonical residue r and the lower
// digits: d_C = (r * q_C + sum_{j<C} d_j * u_{j,C}) mod m_C, where
// q_C = P_C^-1 mod m_C and u_{j,C} = -P_j q_C mod m_C.  Every term is below
// 2^16 and there are at most 10, so one Barrett reduction suffices.
template <int C, typename DigitAt>
__device__ __forceinline__ uint32_t garner_digit(const rnsmx_moduli_t &mods, uint32_t r,
                                                 DigitAt &&digit_at) {
  uint32_t s = r * mods.qinv[C];
#pragma unroll
  for (int j = 0; j < C; ++j) s += digit_at(j) * mods.ucoef[j][C];
  return mod_u32(s, static_cast<uint32_t>(mods.moduli[C]), mods.magic[C]);
}

// ---------------------------------------------------------------------------
// Tiled GEMM: one workgroup computes a BM x BN output tile for every channel
// in turn (4 waves, 2 x 2, each (BM/2) x (BN/2)).  A and B K-steps of 64
// bytes are staged through double-buffered LDS with 16-byte global loads;
// rows are padded to 80 bytes so the 16-byte fragment reads of 8 lanes hit
// disjoint banks.  The global prefetch runs one step ahead and flows across
// channel boundaries.  After each channel's K loop the int32 accumulators are
// reduced mod m_c and turned into that channel's Garner digit in registers
// (one byte per element); after the last channel the digits are recombined
// and stored.
// ---------------------------------------------------------------------------
constexpr int kLdsRow = 80;

template <int RCAP, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_tile_kernel(const GemmArgs g) {
  constexpr int WM = BM / 32, WN = BN / 32;
  constexpr int AC = BM * 4 / 256, BC = BN * 4 / 256;  // 16-byte chunks per thread
  static_assert(AC >= 1 && BC >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) int8_t As[2][BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * kLdsRow];
  __shared__ int64_t red[4];
  __shared__ int bcast;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int c_act = active_channels(g, red, &bcast);
  const int nk = g.kp >> 6;

  const int8_t *asrc[AC];
  const int8_t *bsrc[BC];
  int alds[AC], blds[BC];
#pragma unroll
  for (int i = 0; i < AC; ++i) {
    const int q = tid + 256 * i, row = q >> 2, part = q & 3;
    const int grow = min(m0 + row, g.m - 1);
    asrc[i] = g.a + grow * g.a_ld + part * 16;
    alds[i] = row * kLdsRow + part * 16;
  }
#pragma unroll
  for (int i = 0; i < BC; ++i) {
    const int q = tid + 256 * i, row = q >> 2, part = q & 3;
    const int gcol = min(n0 + row, g.n - 1);
    bsrc[i] = g.b + gcol * g.b_ld + part * 16;
    blds[i] = row * kLdsRow + part * 16;
  }

  i32x4 ra[AC], rb[BC];
  auto gload = [&](int c, int ks) {
    const int64_t aoff = c * g.a_cs + ks * 64, boff = c * g.b_cs + ks * 64;
#pragma unroll
    for (int i = 0; i < AC; ++i) ra[i] = *reinterpret_cast<const i32x4 *>(asrc[i] + aoff);
#pragma unroll
    for (int i = 0; i < BC; ++i) rb[i] = *reinterpret_cast<const i32x4 *>(bsrc[i] + boff);
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AC; ++i) *reinterpret_cast<i32x4 *>(&As[buf][alds[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < BC; ++i) *reinterpret_cast<i32x4 *>(&Bs[buf][blds[i]]) = rb[i];
  };

  const int a_frag = (wm * (BM / 2) + (lane & 15)) * kLdsRow + (lane >> 4) * 16;
  const int b_frag = (wn * (BN / 2) + (lane & 15)) * kLdsRow + (lane >> 4) * 16;

  uint32_t dig[RCAP][WM * WN];
  i32x4 acc[WM][WN];

  gload(0, 0);
  lstore(0);
  __syncthreads();
  int step = 0;

  static_for<RCAP>([&](auto CC) {
    constexpr int c = decltype(CC)::value;
    if (c >= c_act) return;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

    for (int ks = 0; ks < nk; ++ks, ++step) {
      const int buf = step & 1;
      const bool last_k = (ks + 1 == nk);
      const bool has_next = !last_k || (c + 1 < c_act);
      if (has_next) gload(last_k ? c + 1 : c, last_k ? 0 : ks + 1);
      i32x4 fa[WM], fb[WN];
#pragma unroll
      for (int i = 0; i < WM; ++i)
        fa[i] = *reinterpret_cast<const i32x4 *>(&As[buf][a_frag + i * 16 * kLdsRow]);
#pragma unroll
      for (int j = 0; j < WN; ++j)
        fb[j] = *reinterpret_cast<const i32x4 *>(&Bs[buf][b_frag + j * 16 * kLdsRow]);
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
      if (has_next) lstore(buf ^ 1);
      __syncthreads();
    }

    // channel epilogue: canonical residue -> Garner digit (bytes in dig[c])
    const uint32_t m = static_cast<uint32_t>(g.mods.moduli[c]);
    const uint32_t magic = g.mods.magic[c], c31 = g.mods.c31[c];
    const bool use_lut = c < g.lut_channels;
    const int16_t *lut = g.lut + c * 1024;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        uint32_t packed = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int32_t v = acc[i][j][t];
          const uint32_t r = use_lut ? canon_i32_lut(v, lut, m, c31) : canon_i32(v, m, magic, c31);
          const uint32_t d = garner_digit<c>(g.mods, r, [&](int jj) {
            return byte_of(dig[jj][i * WN + j], t);
          });
          packed |= d << (8 * t);
        }
        dig[c][i * WN + j] = packed;
      }
  });

  // recombine and store
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int col = n0 + wn * (BN / 2) + j * 16 + (lane & 15);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + t;
        if (row < g.m && col < g.n) {
          uint32_t d[RCAP];
#pragma unroll
          for (int c = 0; c < RCAP; ++c) d[c] = byte_of(dig[c][i * WN + j], t);
          store_element<RCAP>(g, c_act, d, row, col);
        }
      }
    }
}

// ---------------------------------------------------------------------------
// Skinny GEMM (M <= 16 * MB rows per workgroup; decode and small batches).
// Waves are split over (channel, K slice): wave w owns channel w % R and K
// slice w / R, loads its MFMA fragments straight from global memory (the
// 16-byte K-contiguous layout makes each fragment one load) and keeps several
// K steps of loads in flight.  Each wave reduces its partial sums mod m_c to
// canonical bytes in LDS; (sum_s p_s) mod m = (sum_s (p_s mod m)) mod m, so
// the slices combine with one more reduction.  All threads then run Garner
// per output element and write coalesced rows.
// ---------------------------------------------------------------------------
template <int RCAP, int MB, int WN>
__global__ __launch_bounds__(1024) void gemm_skinny_kernel(const GemmArgs g) {
  constexpr int BMS = 16 * MB, BNS = 16 * WN;
  constexpr int U = (MB + WN <= 3) ? 4 : 2;  // K steps in flight per wave
  __shared__ uint8_t res[16][BMS * BNS];
  __shared__ int64_t red[16];
  __shared__ int bcast;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = blockDim.x >> 6;
  const int R = g.mods.channels;
  const int ks_n = nw / R;
  const int c = wave % R, s = wave / R;
  const int c_act = active_channels(g, red, &bcast);
  const int m0 = blockIdx.y * BMS, n0 = blockIdx.x * BNS;
  const int nk = g.kp >> 6;

  if (c < c_act && s < ks_n) {
    const int k_begin = s * nk / ks_n, k_end = (s + 1) * nk / ks_n;
    const int8_t *ap[MB];
    const int8_t *bp[WN];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int row = min(m0 + i * 16 + (lane & 15), g.m - 1);
      ap[i] = g.a + c * g.a_cs + row * g.a_ld + (lane >> 4) * 16;
    }
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int col = min(n0 + j * 16 + (lane & 15), g.n - 1);
      bp[j] = g.b + c * g.b_cs + col * g.b_ld + (lane >> 4) * 16;
    }
    i32x4 acc[MB][WN];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

    int ks = k_begin;
    for (; ks + U <= k_end; ks += U) {
      i32x4 fa[U][MB], fb[U][WN];
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int j = 0; j < WN; ++j)
          fb[u][j] = *reinterpret_cast<const i32x4 *>(bp[j] + (ks + u) * 64);
#pragma unroll
        for (int i = 0; i < MB; ++i)
          fa[u][i] = *reinterpret_cast<const i32x4 *>(ap[i] + (ks + u) * 64);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u][i], fb[u][j], acc[i][j], 0, 0, 0);
    }
    for (; ks < k_end; ++ks) {
      i32x4 fa[MB], fb[WN];
#pragma unroll
      for (int j = 0; j < WN; ++j) fb[j] = *reinterpret_cast<const i32x4 *>(bp[j] + ks * 64);
#pragma unroll
      for (int i = 0; i < MB; ++i) fa[i] = *reinterpret_cast<const i32x4 *>(ap[i] + ks * 64);
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }

    const uint32_t m = static_cast<uint32_t>(g.mods.moduli[c]);
    const uint32_t magic = g.mods.magic[c], c31 = g.mods.c31[c];
    const bool use_lut = c < g.lut_channels;
    const int16_t *lut = g.lut + c * 1024;
    uint8_t *rw = res[wave];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int32_t v = acc[i][j][t];
          const uint32_t r = use_lut ? canon_i32_lut(v, lut, m, c31) : canon_i32(v, m, magic, c31);
          rw[(i * 16 + 4 * (lane >> 4) + t) * BNS + j * 16 + (lane & 15)] = static_cast<uint8_t>(r);
        }
  }
  __syncthreads();

  const int rows_here = min(BMS, g.m - m0);
  for (int e = tid; e < rows_here * BNS; e += blockDim.x) {
    const int row = e / BNS, col = e % BNS;
    const int gcol = n0 + col;
    if (gcol >= g.n) continue;
    uint32_t d[RCAP];
    static_for<RCAP>([&](auto CC) {
      constexpr int cc = decltype(CC)::value;
      if (cc >= c_act) {
        d[cc] = 0;
        return;
      }
      uint32_t sum = 0;
      for (int s2 = 0; s2 < ks_n; ++s2) sum += res[s2 * R + cc][e];
      const uint32_t m = static_cast<uint32_t>(g.mods.moduli[cc]);
      const uint32_t r = mod_u32(sum, m, g.mods.magic[cc]);
      d[cc] = garner_digit<cc>(g.mods, r, [&](int jj) { return d[jj]; });
    });
    store_element<RCAP>(g, c_act, d, m0 + row, gcol);
  }
}

// ---------------------------------------------------------------------------
// Encoders
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void load16(const T *p, int32_t (&v)[16]) {
  if constexpr (sizeof(T) == 1) {
    const i32x4 w = *reinterpret_cast<const i32x4 *>(p);
#pragma unroll
    for (int q = 0; q < 16; ++q)
      v[q] = static_cast<int8_t>((static_cast<uint32_t>(w[q >> 2]) >> (8 * (q & 3))) & 0xFF);
  } else if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const i32x4 w = *reinterpret_cast<const i32x4 *>(p + 8 * h);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        v[8 * h + q] = static_cast<int16_t>((static_cast<uint32_t>(w[q >> 1]) >> (16 * (q & 1))) & 0xFFFF);
    }
  } else {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const i32x4 w = *reinterpret_cast<const i32x4 *>(p + 4 * h);
#pragma unroll
      for (int q = 0; q < 4; ++q) v[4 * h + q] = w[q];
    }
  }
}

// One wave per row: 16 values per lane per step, R residue planes written as
// 16-byte stores, zero padding to out_ld, row L1 and max |v| reduced in-wave.
template <typename T>
__global__ __launch_bounds__(256) void encode_rows_kernel(const EncodeArgs e) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= e.rows) return;
  const T *src = static_cast<const T *>(e.values) + row * e.cols;
  const bool vec = (e.cols % 16) == 0;
  int64_t l1 = 0;
  int32_t amax = 0;
  const int R = e.mods.channels;
  for (int64_t k0 = static_cast<int64_t>(lane) * 16; k0 < e.out_ld; k0 += 64 * 16) {
    int32_t v[16];
    if (vec && k0 + 16 <= e.cols) {
      load16<T>(src + k0, v);
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = (k0 + q < e.cols) ? static_cast<int32_t>(src[k0 + q]) : 0;
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int32_t a = v[q] < 0 ? -v[q] : v[q];  // |INT32_MIN| wraps; widened below
      const int64_t a64 = v[q] < 0 ? -static_cast<int64_t>(v[q]) : v[q];
      l1 += a64;
      amax = static_cast<uint32_t>(a) > static_cast<uint32_t>(amax) ? a : amax;
    }
    for (int c = 0; c < R; ++c) {
      const uint32_t m = static_cast<uint32_t>(e.mods.moduli[c]);
      const uint32_t magic = e.mods.magic[c], c31 = e.mods.c31[c];
      i32x4 w;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        uint32_t packed = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          packed |= (static_cast<uint32_t>(centered_i32(v[4 * d + q], m, magic, c31)) & 0xFFu) << (8 * q);
        w[d] = static_cast<int32_t>(packed);
      }
      *reinterpret_cast<i32x4 *>(e.out + c * e.plane + row * e.out_ld + k0) = w;
    }
  }
  if (e.row_l1 != nullptr) {
    l1 = wave_sum_i64(l1);
    if (lane == 0) e.row_l1[row] = l1;
  }
  if (e.absmax != nullptr) {
    int64_t am = wave_max_i64(static_cast<int64_t>(static_cast<uint32_t>(amax)));
    if (lane == 0) atomicMax(e.absmax, static_cast<int32_t>(am > INT_MAX ? INT_MAX : am));
  }
}

// Flat form of the reference encoder: values [numel] -> [R][numel].
template <typename T>
__global__ __launch_bounds__(256) void encode_flat_kernel(const EncodeArgs e) {
  const int64_t numel = e.cols;
  const int64_t chunks = (numel + 15) / 16;
  const T *src = static_cast<const T *>(e.values);
  const bool vec = (numel % 16) == 0;
  const int R = e.mods.channels;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < chunks;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t k0 = q * 16;
    int32_t v[16];
    if (vec) {
      load16<T>(src + k0, v);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = (k0 + i < numel) ? static_cast<int32_t>(src[k0 + i]) : 0;
    }
    int32_t amax = 0;
    for (int c = 0; c < R; ++c) {
      const uint32_t m = static_cast<uint32_t>(e.mods.moduli[c]);
      const uint32_t magic = e.mods.magic[c], c31 = e.mods.c31[c];
      int8_t *dst = e.out + c * numel + k0;
      if (vec) {
        i32x4 w;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          uint32_t packed = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            packed |= (static_cast<uint32_t>(centered_i32(v[4 * d + i], m, magic, c31)) & 0xFFu) << (8 * i);
          w[d] = static_cast<int32_t>(packed);
        }
        *reinterpret_cast<i32x4 *>(dst) = w;
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (k0 + i < numel) dst[i] = static_cast<int8_t>(centered_i32(v[i], m, magic, c31));
      }
    }
    if (e.absmax != nullptr) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int32_t a = v[i] < 0 ? -v[i] : v[i];
        amax = static_cast<uint32_t>(a) > static_cast<uint32_t>(amax) ? a : amax;
      }
      if (amax < 0) amax = INT_MAX;
      atomicMax(e.absmax, amax);
    }
  }
}

// ---------------------------------------------------------------------------
// Garner decode of centered residue planes (drop-in decode_garner)
// ---------------------------------------------------------------------------
struct DecodeArgs {
  const int8_t *res;
  int64_t count;
  int64_t *out;
  rnsmx_moduli_t mods;
};

template <int RCAP>
__global__ __launch_bounds__(256) void decode_garner_kernel(const DecodeArgs a) {
  const int R = a.mods.channels;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < a.count;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    uint32_t d[RCAP];
    static_for<RCAP>([&](auto CC) {
      constexpr int c = decltype(CC)::value;
      if (c >= R) {
        d[c] = 0;
        return;
      }
      const int32_t m = a.mods.moduli[c];
      const int32_t v = a.res[c * a.count + e];
      const uint32_t r = static_cast<uint32_t>(v < 0 ? v + m : v) % static_cast<uint32_t>(m);
      d[c] = garner_digit<c>(a.mods, r, [&](int jj) { return d[jj]; });
    });
    uint64_t x = 0;
#pragma unroll
    for (int c = 0; c < RCAP; ++c)
      if (c < R) x += static_cast<uint64_t>(d[c]) * static_cast<uint64_t>(a.mods.prefix[c]);
    const int64_t p = a.mods.prefix[R];
    int64_t y = static_cast<int64_t>(x);
    if (y > (p >> 1)) y -= p;
    a.out[e] = y;
  }
}

// ---------------------------------------------------------------------------
// Repacking for the drop-in op (reference layouts -> K-contiguous, padded)
// ---------------------------------------------------------------------------
// src [R][K][N] -> dst [R][N][ld], zero in [K, ld); 64 x 64 byte tiles via LDS.
__global__ __launch_bounds__(256) void transpose_kn_kernel(const int8_t *__restrict__ src,
                                                           int64_t k, int64_t n, int64_t ld,
                                                           int8_t *__restrict__ dst) {
  __shared__ int8_t tile[64][65];
  const int64_t c = blockIdx.z;
  const int64_t k0 = static_cast<int64_t>(blockIdx.y) * 64, n0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int8_t *s = src + c * k * n;
  int8_t *d = dst + c * n * ld;
  for (int q = threadIdx.x; q < 64 * 64; q += 256) {
    const int r = q >> 6, col = q & 63;
    const int64_t kk = k0 + r, nn = n0 + col;
    tile[r][col] = (kk < k && nn < n) ? s[kk * n + nn] : static_cast<int8_t>(0);
  }
  __syncthreads();
  for (int q = threadIdx.x; q < 64 * 64; q += 256) {
    const int r = q >> 6, col = q & 63;  // r indexes n, col indexes k
    const int64_t nn = n0 + r, kk = k0 + col;
    if (nn < n && kk < ld) d[nn * ld + kk] = tile[col][r];
  }
}

// src [R][rows][K] -> dst [R][rows][ld], zero in [K, ld).
__global__ __launch_bounds__(256) void pad_rows_kernel(const int8_t *__restrict__ src, int64_t rows,
                                                       int64_t k, int64_t ld, int64_t total,
                                                       int8_t *__restrict__ dst) {
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < total;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t col = q % ld, rr = q / ld;  // rr = c * rows + row
    dst[q] = col < k ? src[rr * k + col] : static_cast<int8_t>(0);
  }
}

// ---------------------------------------------------------------------------
// Host side: dispatch
// ---------------------------------------------------------------------------
static int rcap_for(int channels) {
  if (channels <= 3) return 3;
  if (channels <= 4) return 4;
  if (channels <= 6) return 6;
  return 10;
}

static int32_t check_launch(const char *what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(err));
    return RNSMX_ELAUNCH;
  }
  return RNSMX_OK;
}

template <int RCAP>
static void launch_skinny(const GemmArgs &g, int mb, int wn, int waves, hipStream_t st) {
  const dim3 block(64 * waves);
#define RNSMX_SKINNY(MB_, WN_)                                                           \
  if (mb == MB_ && wn == WN_) {                                                          \
    const dim3 grid((g.n + 16 * WN_ - 1) / (16 * WN_), (g.m + 16 * MB_ - 1) / (16 * MB_)); \
    hipLaunchKernelGGL((gemm_skinny_kernel<RCAP, MB_, WN_>), grid, block, 0, st, g);      \
    return;                                                                              \
  }
  RNSMX_SKINNY(1, 1)
  RNSMX_SKINNY(1, 2)
  RNSMX_SKINNY(2, 1)
  RNSMX_SKINNY(2, 2)
  RNSMX_SKINNY(4, 1)
  RNSMX_SKINNY(4, 2)
#undef RNSMX_SKINNY
}

template <int RCAP>
static void launch_tile(const GemmArgs &g, int bm, int bn, hipStream_t st) {
  const dim3 block(256);
#define RNSMX_TILE(BM_, BN_)                                                  \
  if (bm == BM_ && bn == BN_) {                                               \
    const dim3 grid((g.n + BN_ - 1) / BN_, (g.m + BM_ - 1) / BM_);            \
    hipLaunchKernelGGL((gemm_tile_kernel<RCAP, BM_, BN_>), grid, block, 0, st, g); \
    return;                                                                   \
  }
  RNSMX_TILE(64, 64)
  if constexpr (RCAP <= 4) {
    RNSMX_TILE(128, 128)
  }
#undef RNSMX_TILE
}

// Chooses the kernel family and tile for an M x N x kp problem.
static int32_t launch_gemm(const GemmArgs &g, hipStream_t st) {
  const int R = g.mods.channels;
  const int rc = rcap_for(R);
  if (g.m <= 64) {
    const int mb = g.m <= 16 ? 1 : (g.m <= 32 ? 2 : 4);
    const int wn = 1;
    const int nk = g.kp / 64;
    int ks = std::max(1, 16 / R);
    ks = std::min(ks, std::max(1, nk));
    const int waves = R * ks;
    switch (rc) {
      case 3: launch_skinny<3>(g, mb, wn, waves, st); break;
      case 4: launch_skinny<4>(g, mb, wn, waves, st); break;
      case 6: launch_skinny<6>(g, mb, wn, waves, st); break;
      default: launch_skinny<10>(g, mb, wn, waves, st); break;
    }
    return check_launch("gemm_skinny");
  }
  const int64_t tiles128 = static_cast<int64_t>((g.m + 127) / 128) * ((g.n + 127) / 128);
  const int t = (tiles128 >= 256 && rc <= 4) ? 128 : 64;
  switch (rc) {
    case 3: launch_tile<3>(g, t, t, st); break;
    case 4: launch_tile<4>(g, t, t, st); break;
    case 6: launch_tile<6>(g, t, t, st); break;
    default: launch_tile<10>(g, t, t, st); break;
  }
  return check_launch("gemm_tile");
}

static int32_t launch_encode_rows(int32_t dtype, const EncodeArgs &e, hipStream_t st) {
  if (e.rows == 0) return RNSMX_OK;
  const dim3 grid(static_cast<unsigned>((e.rows + 3) / 4)), block(256);
  switch (dtype) {
    case RNSMX_INT8: hipLaunchKernelGGL(encode_rows_kernel<int8_t>, grid, block, 0, st, e); break;
    case RNSMX_INT16: hipLaunchKernelGGL(encode_rows_kernel<int16_t>, grid, block, 0, st, e); break;
    case RNSMX_INT32: hipLaunchKernelGGL(encode_rows_kernel<int32_t>, grid, block, 0, st, e); break;
    default: return fail(RNSMX_EINVAL, "encoder supports int8, int16 and int32");
  }
  return check_launch("encode_rows");
}

static size_t dtype_size(int32_t dtype) {
  switch (dtype) {
    case RNSMX_INT8: return 1;
    case RNSMX_INT16: return 2;
    case RNSMX_INT32: return 4;
    default: return 0;
  }
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace rnsmx

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using namespace rnsmx;

extern "C" {

int32_t rnsmx_encode_centered(const void *values_dev, int32_t dtype, int64_t rows, int64_t cols,
                              int64_t out_ld, const rnsmx_moduli_t *mods, int8_t *out_dev,
                              int64_t *row_l1_dev, int32_t *absmax_dev, void *stream) {
  clear_error();
  if (!mods || mods->channels < 1) return fail(RNSMX_EINVAL, "moduli are not initialised");
  if (dtype_size(dtype) == 0) return fail(RNSMX_EINVAL, "centered encoder supports int8, int16 and int32");
  if (rows < 0 || cols < 0 || out_ld < cols) return fail(RNSMX_EINVAL, "bad encode shape");
  if (rows == 0 || out_ld == 0) return RNSMX_OK;
  if (!values_dev || !out_dev) return fail(RNSMX_EINVAL, "null tensor pointer");
  if (!aligned16(values_dev) || !aligned16(out_dev))
    return fail(RNSMX_EINVAL, "encode buffers must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  EncodeArgs e{};
  e.values = values_dev;
  e.out = out_dev;
  e.row_l1 = row_l1_dev;
  e.absmax = absmax_dev;
  e.mods = *mods;
  if (out_ld == cols && row_l1_dev == nullptr) {
    // flat reference form [R][numel]
    e.rows = 1;
    e.cols = rows * cols;
    e.out_ld = rows * cols;
    e.plane = rows * cols;
    const int64_t chunks = (e.cols + 15) / 16;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((chunks + 255) / 256, 8192));
    switch (dtype) {
      case RNSMX_INT8: hipLaunchKernelGGL(encode_flat_kernel<int8_t>, dim3(blocks), dim3(256), 0, st, e); break;
      case RNSMX_INT16: hipLaunchKernelGGL(encode_flat_kernel<int16_t>, dim3(blocks), dim3(256), 0, st, e); break;
      default: hipLaunchKernelGGL(encode_flat_kernel<int32_t>, dim3(blocks), dim3(256), 0, st, e); break;
    }
    return check_launch("encode_flat");
  }
  if (out_ld % 16 != 0) return fail(RNSMX_EINVAL, "padded encode needs out_ld % 16 == 0");
  e.rows = rows;
  e.cols = cols;
  e.out_ld = out_ld;
  e.plane = rows * out_ld;
  return launch_encode_rows(dtype, e, st);
}

int64_t rnsmx_fused_workspace_bytes(int64_t m, int64_t k, int64_t n, int32_t channels) {
  if (m < 0 || k < 0 || n < 0 || channels < 1) return -1;
  const int64_t kp = round_up(std::max<int64_t>(k, 1), RNSMX_K_ALIGN);
  const int64_t a = (k % RNSMX_K_ALIGN == 0) ? 0 : round_up(channels * m * kp, 256);
  const int64_t b = round_up(channels * n * kp, 256);
  return a + b;
}

int32_t rnsmx_matmul_centered_fused_out(const int8_t *a_dev, const int8_t *b_dev, int32_t m, int32_t k,
                                        int32_t n, const rnsmx_moduli_t *mods, const int16_t *lut_dev,
                                        int32_t lut_channels, void *workspace_dev, int64_t workspace_bytes,
                                        int64_t *out_dev, void *stream) {
  clear_error();
  if (!mods || mods->channels < 1) return fail(RNSMX_EINVAL, "moduli are not initialised");
  if (m < 0 || k < 1 || n < 0) return fail(RNSMX_EINVAL, "bad GEMM shape");
  if (lut_channels < 0 || lut_channels > 2 || lut_channels > mods->channels)
    return fail(RNSMX_EINVAL, "lut_channels must be 0, 1 or 2 and <= channel count");
  if (lut_channels > 0 && !lut_dev) return fail(RNSMX_EINVAL, "lut_channels > 0 needs the LUT");
  if (!accumulator_fits(*mods, k))
    return fail(RNSMX_ERANGE, "K * max(floor(m/2))^2 exceeds the int32 accumulator");
  if (m == 0 || n == 0) return RNSMX_OK;
  if (!a_dev || !b_dev || !out_dev || !workspace_dev) return fail(RNSMX_EINVAL, "null tensor pointer");
  const int64_t need = rnsmx_fused_workspace_bytes(m, k, n, mods->channels);
  if (workspace_bytes < need) {
    set_error("workspace too small: %lld < %lld bytes", static_cast<long long>(workspace_bytes),
              static_cast<long long>(need));
    return RNSMX_ESPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int R = mods->channels;
  const int64_t kp = round_up(k, RNSMX_K_ALIGN);
  int8_t *ws = static_cast<int8_t *>(workspace_dev);
  const int8_t *a_use = a_dev;
  int64_t a_ld = k;
  if (k % RNSMX_K_ALIGN != 0 || !aligned16(a_dev)) {
    int8_t *a_pad = ws;
    ws += round_up(R * static_cast<int64_t>(m) * kp, 256);
    const int64_t total = R * static_cast<int64_t>(m) * kp;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 16384));
    hipLaunchKernelGGL(pad_rows_kernel, dim3(blocks), dim3(256), 0, st, a_dev, static_cast<int64_t>(m),
                       static_cast<int64_t>(k), kp, total, a_pad);
    if (int32_t rc = check_launch("pad_rows")) return rc;
    a_use = a_pad;
    a_ld = kp;
  }
  int8_t *b_nk = ws;
  {
    const dim3 grid((n + 63) / 64, static_cast<unsigned>((kp + 63) / 64), R);
    hipLaunchKernelGGL(transpose_kn_kernel, grid, dim3(256), 0, st, b_dev, static_cast<int64_t>(k),
                       static_cast<int64_t>(n), kp, b_nk);
    if (int32_t rc = check_launch("transpose_kn")) return rc;
  }
  GemmArgs g{};
  g.a = a_use;
  g.a_ld = a_ld;
  g.a_cs = a_ld * m;
  g.b = b_nk;
  g.b_ld = kp;
  g.b_cs = kp * n;
  g.m = m;
  g.n = n;
  g.kp = static_cast<int32_t>(kp);
  g.lut_channels = lut_channels;
  g.lut = lut_dev;
  g.min_channels = 0;
  g.out = out_dev;
  g.out_ld = n;
  g.out_dtype = RNSMX_INT64;
  g.mods = *mods;
  return launch_gemm(g, st);
}

int32_t rnsmx_prepare_weight(const void *b_nk_dev, int32_t dtype, int32_t n, int32_t k,
                             const rnsmx_moduli_t *mods, int8_t *packed_dev, int32_t *absmax_dev,
                             void *stream) {
  clear_error();
  if (!mods || mods->channels < 1) return fail(RNSMX_EINVAL, "moduli are not initialised");
  if (n < 0 || k < 1) return fail(RNSMX_EINVAL, "bad weight shape");
  if (dtype_size(dtype) == 0) return fail(RNSMX_EINVAL, "prepared weights support int8/int16/int32");
  if (n == 0) return RNSMX_OK;
  if (!b_nk_dev || !packed_dev) return fail(RNSMX_EINVAL, "null tensor pointer");
  if (!aligned16(b_nk_dev) || !aligned16(packed_dev))
    return fail(RNSMX_EINVAL, "weight buffers must be 16-byte aligned");
  const int64_t kp = round_up(k, RNSMX_K_ALIGN);
  EncodeArgs e{};
  e.values = b_nk_dev;
  e.rows = n;
  e.cols = k;
  e.out_ld = kp;
  e.plane = static_cast<int64_t>(n) * kp;
  e.out = packed_dev;
  e.row_l1 = nullptr;
  e.absmax = absmax_dev;
  e.mods = *mods;
  return launch_encode_rows(dtype, e, static_cast<hipStream_t>(stream));
}

int64_t rnsmx_prepared_workspace_bytes(int64_t m, int64_t k, int32_t channels) {
  if (m < 0 || k < 0 || channels < 1) return -1;
  const int64_t kp = round_up(std::max<int64_t>(k, 1), RNSMX_K_ALIGN);
  return round_up(channels * m * kp, 256) + round_up(8 * m, 256);
}

int32_t rnsmx_matmul_prepared_fused(const void *a_dev, int32_t a_dtype, int32_t m, int32_t k, int32_t n,
                                    const int8_t *packed_dev, const rnsmx_moduli_t *mods,
                                    const int16_t *lut_dev, int32_t lut_channels,
                                    const rnsmx_adaptive_t *adaptive, const rnsmx_epilogue_t *epilogue,
                                    void *workspace_dev, int64_t workspace_bytes, void *out_dev,
                                    void *stream) {
  clear_error();
  if (!mods || mods->channels < 1) return fail(RNSMX_EINVAL, "moduli are not initialised");
  if (m < 0 || k < 1 || n < 0) return fail(RNSMX_EINVAL, "bad GEMM shape");
  if (dtype_size(a_dtype) == 0) return fail(RNSMX_EINVAL, "a must be int8/int16/int32");
  if (lut_channels < 0 || lut_channels > 2 || lut_channels > mods->channels)
    return fail(RNSMX_EINVAL, "lut_channels must be 0, 1 or 2 and <= channel count");
  if (lut_channels > 0 && !lut_dev) return fail(RNSMX_EINVAL, "lut_channels > 0 needs the LUT");
  if (!accumulator_fits(*mods, k))
    return fail(RNSMX_ERANGE, "K * max(floor(m/2))^2 exceeds the int32 accumulator");
  const int32_t out_dtype = epilogue ? epilogue->out_dtype : RNSMX_INT64;
  if (out_dtype != RNSMX_INT64 && out_dtype != RNSMX_FLOAT32 && out_dtype != RNSMX_FLOAT16 &&
      out_dtype != RNSMX_BFLOAT16)
    return fail(RNSMX_EINVAL, "unsupported output dtype");
  if (out_dtype != RNSMX_INT64 && (!epilogue->a_scale_dev || !epilogue->w_scale_dev))
    return fail(RNSMX_EINVAL, "float output needs a_scale and w_scale");
  const int32_t min_ch = adaptive ? adaptive->min_channels : 0;
  if (min_ch != 0 && (min_ch < 2 || min_ch > mods->channels))
    return fail(RNSMX_EINVAL, "min_channels must be between 2 and full channel count");
  if (min_ch != 0 && !adaptive->w_absmax_dev) return fail(RNSMX_EINVAL, "adaptive needs max|B|");
  if (m == 0 || n == 0) return RNSMX_OK;
  if (!a_dev || !packed_dev || !out_dev || !workspace_dev) return fail(RNSMX_EINVAL, "null tensor pointer");
  const int64_t need = rnsmx_prepared_workspace_bytes(m, k, mods->channels);
  if (workspace_bytes < need) {
    set_error("workspace too small: %lld < %lld bytes", static_cast<long long>(workspace_bytes),
              static_cast<long long>(need));
    return RNSMX_ESPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int R = mods->channels;
  const int64_t kp = round_up(k, RNSMX_K_ALIGN);
  int8_t *a_res = static_cast<int8_t *>(workspace_dev);
  int64_t *row_l1 = reinterpret_cast<int64_t *>(a_res + round_up(R * static_cast<int64_t>(m) * kp, 256));

  EncodeArgs e{};
  e.values = a_dev;
  e.rows = m;
  e.cols = k;
  e.out_ld = kp;
  e.plane = static_cast<int64_t>(m) * kp;
  e.out = a_res;
  e.row_l1 = min_ch != 0 ? row_l1 : nullptr;
  e.absmax = nullptr;
  e.mods = *mods;
  if (!aligned16(a_dev)) return fail(RNSMX_EINVAL, "activations must be 16-byte aligned");
  if (int32_t rc = launch_encode_rows(a_dtype, e, st)) return rc;

  GemmArgs g{};
  g.a = a_res;
  g.a_ld = kp;
  g.a_cs = kp * m;
  g.b = packed_dev;
  g.b_ld = kp;
  g.b_cs = kp * n;
  g.m = m;
  g.n = n;
  g.kp = static_cast<int32_t>(kp);
  g.lut_channels = lut_channels;
  g.lut = lut_dev;
  g.min_channels = min_ch;
  g.row_l1 = row_l1;
  g.w_absmax = min_ch != 0 ? adaptive->w_absmax_dev : nullptr;
  g.meta = min_ch != 0 ? adaptive->meta_dev : nullptr;
  g.out = out_dev;
  g.out_ld = n;
  g.out_dtype = out_dtype;
  g.a_scale = epilogue ? epilogue->a_scale_dev : nullptr;
  g.w_scale = epilogue ? epilogue->w_scale_dev : nullptr;
  g.bias = epilogue ? epilogue->bias_dev : nullptr;
  g.mods = *mods;
  return launch_gemm(g, st);
}

int32_t rnsmx_matmul_residues_prepared(const int8_t *a_res_dev, int64_t a_ld, int32_t m, int32_t k,
                                       int32_t n, const int8_t *packed_dev,
                                       const rnsmx_moduli_t *mods, const int16_t *lut_dev,
                                       int32_t lut_channels, const rnsmx_epilogue_t *epilogue,
                                       void *out_dev, void *stream) {
  clear_error();
  if (!mods || mods->channels < 1) return fail(RNSMX_EINVAL, "moduli are not initialised");
  if (m < 0 || k < 1 || n < 0) return fail(RNSMX_EINVAL, "bad GEMM shape");
  const int64_t kp = round_up(k, RNSMX_K_ALIGN);
  if (a_ld < kp || a_ld % RNSMX_K_ALIGN != 0)
    return fail(RNSMX_EINVAL, "a_ld must be a multiple of 64 and >= round_up(K, 64)");
  if (lut_channels < 0 || lut_channels > 2 || lut_channels > mods->channels)
    return fail(RNSMX_EINVAL, "lut_channels must be 0, 1 or 2 and <= channel count");
  if (lut_channels > 0 && !lut_dev) return fail(RNSMX_EINVAL, "lut_channels > 0 needs the LUT");
  if (!accumulator_fits(*mods, k))
    return fail(RNSMX_ERANGE, "K * max(floor(m/2))^2 exceeds the int32 accumulator");
  const int32_t out_dtype = epilogue ? epilogue->out_dtype : RNSMX_INT64;
  if (out_dtype != RNSMX_INT64 && out_dtype != RNSMX_FLOAT32 && out_dtype != RNSMX_FLOAT16 &&
      out_dtype != RNSMX_BFLOAT16)
    return fail(RNSMX_EINVAL, "unsupported output dtype");
  if (out_dtype != RNSMX_INT64 && (!epilogue->a_scale_dev || !epilogue->w_scale_dev))
    return fail(RNSMX_EINVAL, "float output needs a_scale and w_scale");
  if (m == 0 || n == 0) return RNSMX_OK;
  if (!a_res_dev || !packed_dev || !out_dev) return fail(RNSMX_EINVAL, "null tensor pointer");
  if (!aligned16(a_res_dev) || !aligned16(packed_dev))
    return fail(RNSMX_EINVAL, "residue buffers must be 16-byte aligned");
  GemmArgs g{};
  g.a = a_res_dev;
  g.a_ld = a_ld;
  g.a_cs = a_ld * m;
  g.b = packed_dev;
  g.b_ld = kp;
  g.b_cs = kp * n;
  g.m = m;
  g.n = n;
  g.kp = static_cast<int32_t>(kp);
  g.lut_channels = lut_channels;
  g.lut = lut_dev;
  g.min_channels = 0;
  g.out = out_dev;
  g.out_ld = n;
  g.out_dtype = out_dtype;
  g.a_scale = epilogue ? epilogue->a_scale_dev : nullptr;
  g.w_scale = epilogue ? epilogue->w_scale_dev : nullptr;
  g.bias = epilogue ? epilogue->bias_dev : nullptr;
  g.mods = *mods;
  return launch_gemm(g, static_cast<hipStream_t>(stream));
}

int32_t rnsmx_decode_garner(const int8_t *residues_dev, int64_t count, const rnsmx_moduli_t *mods,
                            int64_t *out_dev, void *stream) {
  clear_error();
  if (!mods || mods->channels < 1) return fail(RNSMX_EINVAL, "moduli are not initialised");
  if (count < 0) return fail(RNSMX_EINVAL, "bad element count");
  if (count == 0) return RNSMX_OK;
  if (!residues_dev || !out_dev) return fail(RNSMX_EINVAL, "null tensor pointer");
  DecodeArgs a{};
  a.res = residues_dev;
  a.count = count;
  a.out = out_dev;
  a.mods = *mods;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((count + 255) / 256, 16384));
  switch (rcap_for(mods->channels)) {
    case 3: hipLaunchKernelGGL(decode_garner_kernel<3>, dim3(blocks), dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL(decode_garner_kernel<4>, dim3(blocks), dim3(256), 0, st, a); break;
    case 6: hipLaunchKernelGGL(decode_garner_kernel<6>, dim3(blocks), dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(decode_garner_kernel<10>, dim3(blocks), dim3(256), 0, st, a); break;
  }
  return check_launch("decode_garner");
}

}  // extern "C"
