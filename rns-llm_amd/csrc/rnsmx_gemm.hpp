// RNS GEMM kernels for gfx950 (MI355X): per-channel int8 products with the
// modular reduction, Garner mixed-radix reconstruction, signed correction
// and optional dequantization fused into the epilogue.
//
// Three families, chosen by the number of output rows M, K and the tile
// count (choose_gemm):
//   stream_kernel  decode and small batches: MFMA tiles of (16*MB) x (16*NB),
//                  K split over the waves of a workgroup, every wave issuing
//                  all loads of its K slice before its first MFMA
//   mfma_kernel    larger M: tiles of (16*MB) x (64*NB), A staged through
//                  LDS with quad-contiguous loads, B streamed into a register
//                  ring, P K steps of loads in flight
//   lds_kernel     large M and K (raw int8 A, up to 4 channels): 256 x 64
//                  tiles, A and B staged by direct-to-LDS loads, 8 waves
//
// Layouts: A is [M][a_ld] int8 activations shared by every channel (a_cs = 0;
// an int8 value is its own representative mod every m_c, so the channel-c
// product of raw activations has the residue of the product of centered
// residues) or [R][M][a_ld] centered residue planes.  B is the prepared
// weight in fragment-major order [R][N16][kp/64][64 lanes x 16 bytes]: the
// 1 KB fragment of column block jb and K step ks holds, at byte 16*l, column
// 16*jb + (l & 15) and K bytes 64*ks + 16*(l >> 4) .. +16, the MFMA B-operand
// layout, so every B load is one contiguous 1 KB (b_ld = bytes per column
// block, b_cs = bytes per channel; columns past N and K past K are zero).
//
// Packed weights (the *_packed_kernel instances): B is two byte planes in
// the same fragment order whatever the channel count, hi = v >> 8 and
// lo = (v & 255) - 128 of each int16 weight v, so v = 256 hi + lo + 128 and,
// with d_c = 256 mod m_c, v = d_c hi + lo + 128 (mod m_c).  Channel c's sum
// is then sum_k a'_k hi_k + sum_k a_k lo_k + 128 sum_k a_k (mod m_c), where
// a_k is the centered residue of the activation and a'_k that of d_c a_k:
// two MFMAs per channel and K step, and a per-row term.  A holds 2R planes
// [a (R planes) | a' (R planes)] followed by int32 [R][packed_corr_ld(M)]
// with (128 sum_k a_k) mod m_c per row (rnsmx_kernels.hip encodes them).
//
// MFMA v_mfma_i32_16x16x64_i8: lane l feeds A row (l & 15) and B column
// (l & 15), both with K bytes [16 * (l >> 4), +16) of a 64-byte step, and
// receives D rows 4 * (l >> 4) + t (t = 0..3) of column (l & 15).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <climits>
#include <cstring>

#include "rnsmx_arith.hpp"
#include "rnsmx_common.hpp"

namespace rnsmx {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// The GEMM's moduli constants for up to RCAP channels: the fields of
// rnsmx_moduli_t the kernels read, sized for their channel capacity, so a
// launch passes a few hundred bytes of arguments instead of the 10-channel
// block (the runtime writes the argument block for every launch, and its
// host cost grows with the size: 0.9 KB measured 1 us more per launch than
// 16 bytes).
template <int RCAP>
struct GemmMods {
  int32_t channels;
  uint32_t moduli[RCAP];
  uint32_t magic[RCAP];
  uint32_t qinv[RCAP];
  int32_t qk16[RCAP];
  uint32_t qk8[RCAP];
  uint32_t ucoef[RCAP][RCAP];
  int64_t prefix[RCAP + 1];
};

// Arguments of one GEMM launch.  The host fills GemmArgs (with the full
// moduli block); each kernel instantiation receives GemmArgsK<RCAP>, the
// same fields with its compact constants (compact_args).
template <typename Mods>
struct GemmArgsOf {
  const int8_t *a;  // [R][M][a_ld] residue planes, or [M][a_ld] int8 (a_cs = 0)
  int64_t a_ld, a_cs;
  const int8_t *b;  // [R][N16][kp/64][1024] fragment-major
  int64_t b_ld, b_cs;  // bytes per column block, per channel
  int32_t m, n, kp;  // kp: multiple of 64, <= b_ld
  int32_t a_k;       // A bytes per row that are read; 16-byte chunks at or past it load as 0
  int32_t tiles_m, tiles_n;  // output tile grid (set at launch)
  int32_t threads;           // workgroup size (set at launch; read here rather than
                             // from the hidden arguments, a cache line of its own)
  // K split over workgroups (split_exchange): tiles [0, split_from) run
  // whole; every later tile is computed by `splits` workgroups, split s
  // taking K steps [s * kchunk, (s + 1) * kchunk) (the last one the rest).
  // splits = 1, split_from = tiles, kchunk = kp / 64 without a split.
  int32_t splits, kchunk, split_from;
  uint32_t *tickets;  // one arrival counter per (tile, wave), zero between calls
  int8_t *xchg;       // partial residues, [tile * waves + wave][split][MI * NJ][4 words][64 lanes] x 4 bytes
  // adaptive prefix
  int32_t min_channels;  // 0: all channels
  int32_t l1_rows;       // words at row_l1 to fold: row norms, or row_l1_max_kernel's maxima of them
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
  Mods mods;  // last: every other field has the same offset in every instantiation
};
using GemmArgs = GemmArgsOf<rnsmx_moduli_t>;
template <int RCAP>
using GemmArgsK = GemmArgsOf<GemmMods<RCAP>>;

// The kernel-side arguments of `g` for channel capacity RCAP (g.mods.channels
// <= RCAP; unused channels are zero).
template <int RCAP>
inline GemmArgsK<RCAP> compact_args(const GemmArgs &g) {
  static_assert(offsetof(GemmArgs, mods) == offsetof(GemmArgsK<RCAP>, mods), "shared leading fields");
  GemmArgsK<RCAP> k{};
  std::memcpy(static_cast<void *>(&k), static_cast<const void *>(&g), offsetof(GemmArgs, mods));
  const rnsmx_moduli_t &f = g.mods;
  k.mods.channels = f.channels;
  for (int c = 0; c < RCAP && c < RNSMX_MAX_CHANNELS; ++c) {
    k.mods.moduli[c] = static_cast<uint32_t>(f.moduli[c]);
    k.mods.magic[c] = f.magic[c];
    k.mods.qinv[c] = f.qinv[c];
    k.mods.qk16[c] = f.qk16[c];
    k.mods.qk8[c] = f.qk8[c];
    for (int j = 0; j < RCAP && j < RNSMX_MAX_CHANNELS; ++j) k.mods.ucoef[j][c] = f.ucoef[j][c];
  }
  for (int c = 0; c <= RCAP && c <= RNSMX_MAX_CHANNELS; ++c) k.mods.prefix[c] = f.prefix[c];
  return k;
}

// kStreamWide: the stream kernel with chunks of up to 8 K steps (long K).
// kMfma3: the MFMA kernel with three column waves (48*nb-column tiles).
// kRows: packed weights at decode (rows_packed_kernel: MFMA rows are channels).
// kLdsWide: the LDS-staged kernel with 256 x 96 tiles (lds_wide_kernel).
enum GemmKind {
  kAuto = 0,
  kStream = 1,
  kMfma = 2,
  kLds = 3,
  kStreamWide = 4,
  kMfma3 = 5,
  kRows = 6,
  kLdsWide = 7,
  kLdsPlanes = 8
};

// ks: waves splitting K (stream kernel) or ring depth, 0 = automatic (MFMA
// kernel); splits: workgroups splitting K (1 = none); tail: only the tiles
// of the last, partial round of 256 are split (the others run whole).
struct GemmChoice {
  int kind, mb, nb, ks, splits, tail;
};

// Geometry of one launch: output tiles, waves per workgroup, and the 16-byte
// accumulator chunks per lane of one wave's block (the exchange unit of a
// K split).
struct GemmGrid {
  int64_t tiles;
  int waves, chunks;
};

// The kernels are instantiated in parts, one translation unit each
// (rnsmx_gemm_part.hip built once per channel capacity R and part P) so the
// library compiles in parallel:
//   P0 stream kernels, P1 MFMA kernels with raw int8 A and 64-column tiles,
//   P2 MFMA kernels with raw int8 A and 128-column tiles, P3 MFMA kernels
//   with residue-plane A, P4 the LDS-staged kernel, P5 the stream and MFMA
//   kernels for packed weights (channel capacities 4 and 6).
// launch_gemm_rR_pP returns false when the part has no kernel for the choice.
constexpr int kGemmParts = 6;
inline int gemm_part_of(const GemmChoice &c, bool araw, bool packed = false) {
  if (packed) return 5;
  if (c.kind == kStream || c.kind == kStreamWide) return 0;
  if (c.kind == kLds || c.kind == kLdsWide || c.kind == kLdsPlanes) return 4;
  if (!araw) return 3;
  return c.nb == 1 ? 1 : 2;
}
#define RNSMX_GEMM_PART_NAME(R, P) launch_gemm_r##R##_p##P
#define RNSMX_GEMM_PART_DECL(R, P) \
  bool RNSMX_GEMM_PART_NAME(R, P)(const GemmArgs &g, bool araw, const GemmChoice &c, hipStream_t st);
#define RNSMX_GEMM_PARTS_DECL(R)                                                             \
  RNSMX_GEMM_PART_DECL(R, 0) RNSMX_GEMM_PART_DECL(R, 1) RNSMX_GEMM_PART_DECL(R, 2) \
  RNSMX_GEMM_PART_DECL(R, 3) RNSMX_GEMM_PART_DECL(R, 4) RNSMX_GEMM_PART_DECL(R, 5)
RNSMX_GEMM_PARTS_DECL(3)
RNSMX_GEMM_PARTS_DECL(4)
RNSMX_GEMM_PARTS_DECL(6)
RNSMX_GEMM_PARTS_DECL(10)

// Kernel arguments read in place from the kernarg segment (constant address
// space, scalar loads).  A by-value struct parameter used as an ordinary
// object can be copied whole into per-lane scratch memory by the compiler
// (it does so for the larger GEMM instances); a reference to the segment
// never is.  Valid for kernels whose only parameter is the struct, which
// then sits at offset 0 of the segment.
#define RNSMX_KARG(T) const __attribute__((address_space(4))) T
template <typename T>
__device__ __forceinline__ RNSMX_KARG(T) & kernel_args() {
  return *(RNSMX_KARG(T) *)(__builtin_amdgcn_kernarg_segment_ptr());
}
template <int RCAP>
using KArgs = RNSMX_KARG(GemmArgsK<RCAP>);

// Touches the first BYTES of the argument block, one read per 64-byte line,
// in one round at kernel entry.  The block is written for each launch, so
// its first reads miss the caches; the kernels read the fields that the
// first operand loads depend on in dependent rounds (the adaptive check,
// then the tile counts, then the operand pointers), and each of those would
// otherwise wait a full memory round trip.  With the lines in the scalar
// cache the later reads hit.  The stream kernels read only the fields their
// first operand loads need (load_hot_args, or this touch of the first
// kGemmHotArgBytes) and leave the epilogue's constants (the moduli block)
// to a round of their own that overlaps those loads: a longer first round
// measured 1-2 % slower at decode shapes.  The kernels that stage through
// LDS take the whole block: scalar loads and LDS
// reads share one completion counter, so epilogue constants still in flight
// would hold up every LDS wait of the first K steps (C2 M=256: 13.1 -> 12.4 us).
template <int BYTES>
__device__ __forceinline__ void prefetch_kernel_args() {
  const __attribute__((address_space(4))) uint32_t *p =
      (const __attribute__((address_space(4))) uint32_t *)(__builtin_amdgcn_kernarg_segment_ptr());
  uint32_t x = 0;
  static_for<(BYTES + 63) / 64>([&](auto L) { x ^= p[decltype(L)::value * 16]; });
  asm volatile("" : : "s"(x));
}
// Reads every field that the first operand loads depend on in one round of
// scalar loads, with one wait.  Left to itself the compiler issues each read
// next to its first use and waits after each one (five dependent waits on
// the stream kernel's way to its first loads); later uses of the same
// fields reuse these values, the argument block being read-only.  Measured
// 0.06-0.08 us per launch on the C2 and C3 shapes.
template <typename G>
__device__ __forceinline__ void load_hot_args(G &g) {
  const int8_t *a = g.a, *b = g.b;
  const int64_t a_ld = g.a_ld, a_cs = g.a_cs, b_ld = g.b_ld, b_cs = g.b_cs;
  const int m = g.m, n = g.n, kp = g.kp, a_k = g.a_k, tiles_m = g.tiles_m, tiles_n = g.tiles_n;
  const int threads = g.threads, splits = g.splits, kchunk = g.kchunk, split_from = g.split_from;
  const int min_channels = g.min_channels, channels = g.mods.channels;
  asm volatile("" : : "s"(a), "s"(b), "s"(a_ld), "s"(a_cs), "s"(b_ld), "s"(b_cs), "s"(m), "s"(n), "s"(kp),
               "s"(a_k), "s"(tiles_m), "s"(tiles_n), "s"(threads), "s"(splits), "s"(kchunk), "s"(split_from),
               "s"(min_channels), "s"(channels));
}
// GemmArgs through mods.channels: every field read before the first
// operand loads of the GEMM kernels
constexpr int kGemmHotArgBytes = static_cast<int>(offsetof(GemmArgs, mods) + sizeof(int32_t));
template <int RCAP>
constexpr int kGemmArgBytes = static_cast<int>(sizeof(GemmArgsK<RCAP>));

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

__device__ __forceinline__ i32x4 load16(const int8_t *p) { return *reinterpret_cast<const i32x4 *>(p); }

// acc + sum of |b| over the 16 signed bytes of w: each byte biased by 128
// (sign bit flipped) and v_sad_u8 against 128 in every byte, 2 instructions
// per 4 bytes.
__device__ __forceinline__ uint32_t abs_sum_i8x16(i32x4 w, uint32_t acc) {
  static_for<4>([&](auto Q) {
    constexpr int q = decltype(Q)::value;
    acc = __builtin_amdgcn_sad_u8(static_cast<uint32_t>(w[q]) ^ 0x80808080u, 0x80808080u, acc);
  });
  return acc;
}
// Streaming load (non-temporal hint) for weight bytes that one launch reads
// once.  Measured on the decode kernels that stream their weights from HBM
// (a single row tile): 7-13 % faster than plain loads; where several row
// tiles share each weight byte through L2 (C2 M=256) the hint cost 2-3 %.
__device__ __forceinline__ i32x4 load16_nt(const int8_t *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(p));
}

// Initial value of one MFMA accumulator: zero, hidden from the compiler.
// With a plain constant every accumulator of a K loop starts from the same
// folded zero, and the register allocator then keeps rotating accumulators
// between registers inside the loop (accvgpr moves and copies around every
// MFMA); a distinct opaque zero per accumulator avoids that.
__device__ __forceinline__ i32x4 acc_zero() {
  i32x4 z = {0, 0, 0, 0};
  asm volatile("" : "+v"(z));
  return z;
}

// prefix[idx] for a runtime idx <= RCAP, as a select chain over constant
// indices: a runtime index into the kernel-argument block would make the
// compiler copy the whole block to scratch memory.
template <int RCAP, typename Mods>
__device__ __forceinline__ int64_t prefix_at(const Mods &mods, int idx) {
  int64_t p = mods.prefix[0];
  static_for<RCAP + 1>([&](auto I) {
    if (idx == decltype(I)::value) p = mods.prefix[decltype(I)::value];
  });
  return p;
}

// Number of moduli channels to use.  Without the adaptive prefix this is the
// full set.  With it, every workgroup derives the same answer from the row
// L1 norms (l1_rows words to fold: the norms, or at most 256 maxima of
// them written by row_l1_max_kernel; or, when row_l1 is null, summed here
// from the raw int8 activations: the launcher does so for a few rows only,
// since every workgroup reads them) and max|B| written at weight preparation:
// bound = max_i sum_k |a_ik| * max|B| (adaptive.py:44-52); the answer is the
// smallest c >= min_channels with 2 * bound < prod_{i<c} m_i
// (adaptive.py:15-41), i.e. bound <= (P_c - 1) / 2.  When no prefix fits,
// the full set is used and meta[3] flags the overflow (the reference raises
// OverflowError on the host, which a device-side selector cannot).
template <int RCAP>
__device__ __forceinline__ int active_channels(KArgs<RCAP> &g, int64_t *red, int *bcast, int nthreads) {
  const int full = g.mods.channels;
  if (g.min_channels <= 0) return full;
  if (g.row_l1 != nullptr && g.l1_rows <= 256) {
    // at most 256 words (row norms, or row_l1_max_kernel's maxima of them):
    // every wave folds them itself, reads max|B| with a scalar load and
    // decides alone, with no barrier
    const int lane = threadIdx.x & 63;
    int64_t mx = 0;
    static_for<4>([&](auto J) {
      const int r = lane + 64 * decltype(J)::value;
      if (r < g.l1_rows) {
        const int64_t v = g.row_l1[r];
        mx = v > mx ? v : mx;
      }
    });
    mx = wave_max_i64(mx);  // every lane holds the maximum
    const int64_t best = static_cast<int64_t>(
        (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(mx) >> 32))) << 32) |
        __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(mx)));
    const int64_t wmax = *g.w_absmax;
    int64_t bound;
    if (__builtin_mul_overflow(best, wmax, &bound)) bound = LLONG_MAX;
    int c = full, overflow = 1;
    static_for<RCAP + 1>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if (overflow && i >= g.min_channels && i <= full && bound <= (g.mods.prefix[i] - 1) / 2) {
        c = i;
        overflow = 0;
      }
    });
    if (g.meta != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
      g.meta[0] = c;
      g.meta[1] = bound;
      g.meta[2] = (prefix_at<RCAP>(g.mods, c) - 1) / 2;
      g.meta[3] = overflow;
    }
    return __builtin_amdgcn_readfirstlane(c);
  }
  const int nw = nthreads >> 6;
  int64_t best = 0;  // max_i sum_k |a_ik|, in thread 0
  // max|B| in flight with the row norms, not after them
  const int64_t wmax = threadIdx.x == 0 ? *g.w_absmax : 0;
  if (g.row_l1 != nullptr) {
    int64_t mx = 0;
    for (int r = threadIdx.x; r < g.l1_rows; r += nthreads) {
      const int64_t v = g.row_l1[r];
      mx = v > mx ? v : mx;
    }
    mx = wave_max_i64(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0)
      for (int w = 0; w < nw; ++w) best = red[w] > best ? red[w] : best;
  } else {
    // raw int8 rows of a_ld bytes, a_k of them read (a multiple of 16); the
    // launcher does this for a few rows only
    for (int r = 0; r < g.m; ++r) {
      uint32_t part = 0;  // 128 * K < 2^31
      for (int k0 = threadIdx.x * 16; k0 < g.a_k; k0 += nthreads * 16)
        part = abs_sum_i8x16(*reinterpret_cast<const i32x4 *>(g.a + static_cast<int64_t>(r) * g.a_ld + k0), part);
      const int64_t sum = wave_sum_i64(static_cast<int64_t>(part));
      if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
      __syncthreads();
      if (threadIdx.x == 0) {
        int64_t row = 0;
        for (int w = 0; w < nw; ++w) row += red[w];
        best = row > best ? row : best;
      }
      __syncthreads();
    }
  }
  if (threadIdx.x == 0) {
    int64_t bound;
    if (__builtin_mul_overflow(best, wmax, &bound)) bound = LLONG_MAX;
    int c = full, overflow = 1;
    static_for<RCAP + 1>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if (overflow && i >= g.min_channels && i <= full && bound <= (g.mods.prefix[i] - 1) / 2) {
        c = i;
        overflow = 0;
      }
    });
    *bcast = c;
    if (g.meta != nullptr && blockIdx.x == 0) {
      g.meta[0] = c;
      g.meta[1] = bound;
      g.meta[2] = (prefix_at<RCAP>(g.mods, c) - 1) / 2;
      g.meta[3] = overflow;
    }
  }
  __syncthreads();
  return *bcast;
}

// Everything the epilogue needs, read from the kernel arguments once per
// kernel and pinned in scalar registers (pin_epi) right after the first
// global loads are issued: left to itself the compiler re-issues these
// scalar loads at their first use in the epilogue, where each dependent
// round of scalar-cache misses is exposed.
template <int RCAP>
struct Epi {
  uint32_t m[RCAP], m24[RCAP], c16[RCAP], bias[RCAP], qinv[RCAP], qk8[RCAP];
  int32_t negm[RCAP], qk16[RCAP];
  uint32_t u[RCAP][RCAP];  // u[j][c], j < c
  int64_t prefix[RCAP + 1];
  int64_t p_act;  // prefix[c_act], the modulus of the signed correction
  int32_t out_dtype;
  int64_t out_ld;
  void *out;
  const float *w_scale;
  const float *bias_ptr;
  float a_scale;
};

// Moduli constants of Epi from a moduli block (kernel arguments or a
// by-value copy).
template <int RCAP, typename Mods>
__device__ __forceinline__ void fill_moduli(Epi<RCAP> &e, const Mods &mods, int c_act) {
  static_for<RCAP>([&](auto C) {
    constexpr int c = decltype(C)::value;
    const uint32_t m = static_cast<uint32_t>(mods.moduli[c]), magic = mods.magic[c];
    e.m[c] = m;
    e.qinv[c] = mods.qinv[c];
    e.qk16[c] = mods.qk16[c];
    e.qk8[c] = mods.qk8[c];
    static_for<c>([&](auto J) { e.u[decltype(J)::value][c] = mods.ucoef[decltype(J)::value][c]; });
    // the 24-bit reduction constants (see canon_fast); channels past the
    // set's size have m = 0 and are never used
    e.m24[c] = magic >> 8;
    e.c16[c] = 65536u - (magic >> 16) * m;
    e.bias[c] = m * (magic >> 9);
    e.negm[c] = -static_cast<int32_t>(m);
  });
  static_for<RCAP + 1>([&](auto C) { e.prefix[decltype(C)::value] = mods.prefix[decltype(C)::value]; });
  e.p_act = prefix_at<RCAP>(mods, c_act);
}

template <int RCAP>
__device__ __forceinline__ void load_epi(KArgs<RCAP> &g, Epi<RCAP> &e, int c_act) {
  fill_moduli<RCAP>(e, g.mods, c_act);
  e.out_dtype = g.out_dtype;
  e.out_ld = g.out_ld;
  e.out = g.out;
  e.w_scale = g.w_scale;
  e.bias_ptr = g.bias;
  e.a_scale = g.out_dtype != RNSMX_INT64 ? *g.a_scale : 0.0f;
}

template <typename T>
__device__ __forceinline__ void pin_sgpr(T &v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values only");
  if constexpr (sizeof(T) == 4) {
    uint32_t w = __builtin_bit_cast(uint32_t, v);
    w = __builtin_amdgcn_readfirstlane(w);
    asm volatile("" : "+s"(w));
    v = __builtin_bit_cast(T, w);
  } else {
    uint64_t w = __builtin_bit_cast(uint64_t, v);
    uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(w));
    uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(w >> 32));
    asm volatile("" : "+s"(lo), "+s"(hi));
    v = __builtin_bit_cast(T, (static_cast<uint64_t>(hi) << 32) | lo);
  }
}

template <int RCAP>
__device__ __forceinline__ void pin_epi(Epi<RCAP> &e) {
  static_for<RCAP>([&](auto C) {
    constexpr int c = decltype(C)::value;
    pin_sgpr(e.m[c]);
    pin_sgpr(e.m24[c]);
    pin_sgpr(e.c16[c]);
    pin_sgpr(e.bias[c]);
    pin_sgpr(e.negm[c]);
    pin_sgpr(e.qinv[c]);
    if constexpr (c > 0) {
      pin_sgpr(e.qk16[c]);
      pin_sgpr(e.qk8[c]);
    }
    static_for<c>([&](auto J) { pin_sgpr(e.u[decltype(J)::value][c]); });
  });
  static_for<RCAP + 1>([&](auto C) { pin_sgpr(e.prefix[decltype(C)::value]); });
  pin_sgpr(e.p_act);
  pin_sgpr(e.out_ld);
  pin_sgpr(e.out);
  pin_sgpr(e.out_dtype);
  pin_sgpr(e.a_scale);
  pin_sgpr(e.w_scale);
  pin_sgpr(e.bias_ptr);
}

// Canonical residue of one int32 accumulator of channel c.  The reference
// reduces its first lut_channels channels through a byte table
// (csrc/rns_cuda.cu:69-96) and the rest with Barrett; the residue is unique,
// so every channel here takes the 24-bit arithmetic reduction, which needs
// no table loads (those would queue behind the output stores).
template <int RCAP>
__device__ __forceinline__ uint32_t reduce_acc(const Epi<RCAP> &e, int c, int32_t v) {
  return canon_fast(v, FastMod{e.m[c], e.m24[c], e.c16[c], e.bias[c], e.negm[c]});
}

// Signed integer from the canonical residues r[0..c_act) of the first c_act
// channels.  Mixed-radix digits d_c = (r_c * q_c + sum_{j<c} d_j * u_{j,c})
// mod m_c with q_c = P_c^-1 mod m_c and u_{j,c} = -P_j q_c mod m_c
// (P_c = prod_{j<c} m_j): the same unique digits as the reference's
// pairwise-inverse recurrence (csrc/rns_cuda.cu:389-400) with one reduction
// per digit.  Every term is below 2^16 and there are at most 10, so each sum
// is below 2^24 (24-bit multiplies, mod_small).  x = sum d_c P_c: for c < 4,
// P_c <= 255^3 < 2^24 and the partial sums stay below P_4 <= 255^4 < 2^32,
// so they accumulate in 32 bits; later digits in 64 bits.  x > P/2 maps to
// x - P (P = P_{c_act}), the reference's signed correction.
template <int RCAP>
__device__ __forceinline__ int64_t garner_value(const Epi<RCAP> &e, const uint32_t (&r)[RCAP], int c_act) {
  uint32_t d[RCAP];
  uint32_t x32 = 0;
  uint64_t x64 = 0;
  static_for<RCAP>([&](auto C) {
    constexpr int c = decltype(C)::value;
    if (c >= c_act) {
      d[c] = 0;
      return;
    }
    if constexpr (c == 0) {
      d[0] = r[0];  // q_0 = 1 and r_0 < m_0
    } else {
      uint32_t s = __umul24(r[c], e.qinv[c]);
      static_for<c>([&](auto J) { s += __umul24(d[decltype(J)::value], e.u[decltype(J)::value][c]); });
      d[c] = mod_small(s, e.m[c], e.m24[c], e.negm[c]);
    }
    if constexpr (c < 4) {
      x32 += __umul24(d[c], static_cast<uint32_t>(e.prefix[c]));
    } else {
      x64 += static_cast<uint64_t>(d[c]) * static_cast<uint64_t>(e.prefix[c]);
    }
  });
  if constexpr (RCAP <= 4) {
    // x = x32 < P <= 255^4 < 2^32: the correction x - P lies in [-P/2, 0),
    // so its high word is -1 and its low word is x - P mod 2^32.
    const uint32_t p32 = static_cast<uint32_t>(e.p_act);
    const bool neg = x32 > (p32 >> 1);
    const uint32_t lo = neg ? x32 - p32 : x32;
    const uint32_t hi = neg ? 0xFFFFFFFFu : 0u;
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
  } else {
    const int64_t p = e.p_act;
    int64_t y = static_cast<int64_t>(static_cast<uint64_t>(x32) + x64);
    if (y > (p >> 1)) y -= p;
    return y;
  }
}

// The same signed integer straight from the int32 channel sums v[0..c_act).
// Channel 0's digit is its canonical residue; every later digit takes one
// reduction instead of two (residue, then digit): with v = a2 2^16 + a1 2^8
// + a0 (a2 = v >> 16 signed, a1 and a0 bytes),
//   v q_c = a2 qk16_c + a1 qk8_c + a0 q_c (mod m_c),
// qk16_c = 2^16 q_c mod m_c centered (|qk16_c| <= 127) and qk8_c = 2^8 q_c
// mod m_c.  |a2 qk16_c| <= 2^15 * 127 = 4,161,536 < bias_c (a multiple of
// m_c above 2^23 - 256), so s = a2 qk16_c + a1 qk8_c + a0 q_c + bias_c +
// sum_{j<c} d_j u_{j,c} is positive and at most 4,161,536 + 2 * 255 * 254 +
// 2^23 + 9 * 254^2 = 13,260,328 < 2^24: one mod_small gives d_c.  Every
// multiply is 24-bit.
template <int RCAP>
__device__ __forceinline__ int64_t garner_from_sums(const Epi<RCAP> &e, const int32_t (&v)[RCAP], int c_act) {
  uint32_t d[RCAP];
  uint32_t x32 = 0;
  uint64_t x64 = 0;
  static_for<RCAP>([&](auto C) {
    constexpr int c = decltype(C)::value;
    if (c >= c_act) {
      d[c] = 0;
      return;
    }
    if constexpr (c == 0) {
      d[0] = reduce_acc<RCAP>(e, 0, v[0]);  // q_0 = 1
    } else {
      const int32_t a2 = v[c] >> 16;
      const uint32_t a1 = (static_cast<uint32_t>(v[c]) >> 8) & 0xFFu, a0 = static_cast<uint32_t>(v[c]) & 0xFFu;
      uint32_t s = static_cast<uint32_t>(__mul24(a2, e.qk16[c])) + __umul24(a1, e.qk8[c]) +
                   __umul24(a0, e.qinv[c]) + e.bias[c];
      static_for<c>([&](auto J) { s += __umul24(d[decltype(J)::value], e.u[decltype(J)::value][c]); });
      d[c] = mod_small(s, e.m[c], e.m24[c], e.negm[c]);
    }
    if constexpr (c == 0) {
      x32 = d[0];  // P_0 = 1
    } else if constexpr (c < 4) {
      x32 += __umul24(d[c], static_cast<uint32_t>(e.prefix[c]));
    } else {
      x64 += static_cast<uint64_t>(d[c]) * static_cast<uint64_t>(e.prefix[c]);
    }
  });
  if constexpr (RCAP <= 4) {
    const uint32_t p32 = static_cast<uint32_t>(e.p_act);
    const bool neg = x32 > (p32 >> 1);
    const uint32_t lo = neg ? x32 - p32 : x32;
    const uint32_t hi = neg ? 0xFFFFFFFFu : 0u;
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
  } else {
    const int64_t p = e.p_act;
    int64_t y = static_cast<int64_t>(static_cast<uint64_t>(x32) + x64);
    if (y > (p >> 1)) y -= p;
    return y;
  }
}

// The output pointers arrive as generic pointers inside the argument block;
// naming their address space lets the compiler emit global (not flat)
// memory instructions.
template <typename T>
using gptr = __attribute__((address_space(1))) T *;
template <typename T, typename U>
__device__ __forceinline__ gptr<T> as_global(U *p) {
  return (gptr<T>)(p);
}

// Output element kinds of the epilogue variants: int64, the float chain
// (float32/float16/bfloat16 chosen per element), or any (generic path).
enum EpiOut { kOutInt64 = 0, kOutFloat = 1, kOutAny = 2 };

// Per-column factors of the float epilogue (w_scale[col], bias[col]), read
// once per column before any output store: on this hardware loads and
// stores share one completion counter, so a load issued after stores would
// also wait for those stores.
struct ColScale {
  float w, b;
};

// Int64 outputs load nothing here (a uniform branch, not taken): loading
// unconditionally from a dummy address measured 2-3 % slower on the
// headline and C3 shapes.
template <int RCAP>
__device__ __forceinline__ ColScale col_scale(const Epi<RCAP> &e, int col, int n_lim) {
  ColScale cs{0.0f, 0.0f};
  if (e.out_dtype != RNSMX_INT64) {
    const int c = min(col, n_lim - 1);
    cs.w = as_global<const float>(e.w_scale)[c];
    if (e.bias_ptr != nullptr) cs.b = as_global<const float>(e.bias_ptr)[c];
  }
  return cs;
}

// Writes one output element.  The float chain is
// ((float)y * a_scale) * w_scale[col] + bias[col], each step rounded to
// nearest even with no contraction: the op order of rns_linear.py:272-275.
// The operators are written here, under the pragma, on purpose: HIP's
// __fmul_rn / __fadd_rn are plain operators compiled with contraction on
// in their own header, and after inlining the multiply and the add would
// fuse into an FMA (one rounding instead of two).
// Int64 outputs are written with non-temporal stores: the kernel never
// reads them back, and streaming them past the L2 keeps the A and weight
// lines the other tiles still read (C2 M=256 8.98 -> 8.72 us, C5 M=2048
// about 1 % faster, measured A/B on one box).
template <int RCAP, int OUT>
__device__ __forceinline__ void store_value(const Epi<RCAP> &e, int64_t y, int64_t idx, ColScale cs) {
#pragma clang fp contract(off)
  if (OUT == kOutInt64 || (OUT == kOutAny && e.out_dtype == RNSMX_INT64)) {
    __builtin_nontemporal_store(y, &as_global<int64_t>(e.out)[idx]);
    return;
  }
  // with up to 4 channels |y| <= P/2 < 2^31: the 32-bit conversion rounds
  // the same integer the same way, in one instruction
  float f = RCAP <= 4 ? static_cast<float>(static_cast<int32_t>(y)) : __ll2float_rn(y);
  f = f * e.a_scale;
  f = f * cs.w;
  if (e.bias_ptr != nullptr) f = f + cs.b;
  if (e.out_dtype == RNSMX_FLOAT32) {
    as_global<float>(e.out)[idx] = f;
  } else if (e.out_dtype == RNSMX_FLOAT16) {
    as_global<uint16_t>(e.out)[idx] = __half_as_ushort(__float2half_rn(f));
  } else {
    as_global<uint16_t>(e.out)[idx] = f32_to_bf16_rne(f);
  }
}

// Reduction + reconstruction + store of one element from its channel sums.
// FAST: every channel active (the common case), so the channel loop and
// Garner run with no per-element branch.
// idx = row * out_ld + col, the element's offset in the output; cs the
// column's float-epilogue factors (col_scale).
template <int RCAP, bool FAST, int OUT>
__device__ __forceinline__ void finish_element(KArgs<RCAP> &g, const Epi<RCAP> &e, int c_act,
                                               const int32_t (&v)[RCAP], int64_t idx, ColScale cs) {
  const int64_t y = garner_from_sums<RCAP>(e, v, FAST ? RCAP : c_act);
  store_value<RCAP, OUT>(e, y, idx, cs);
}

// Calls f(FAST, OUT) with the epilogue variant for this call: a uniform
// branch taken once per workgroup instead of once per element.
template <int RCAP, typename F>
__device__ __forceinline__ void with_epilogue(const Epi<RCAP> &e, int c_act, F &&f) {
  if (c_act == RCAP) {
    if (e.out_dtype == RNSMX_INT64)
      f(std::true_type{}, std::integral_constant<int, kOutInt64>{});
    else
      f(std::true_type{}, std::integral_constant<int, kOutFloat>{});
  } else {
    f(std::false_type{}, std::integral_constant<int, kOutAny>{});
  }
}

// Reduction + reconstruction + stores of a wave's (16 MI) x (16 NJ) tile
// straight from its MFMA accumulators: the lane holds rows 4 (lane >> 4) + t
// of column lane & 15 of each 16 x 16 block, whose top-left output element
// is (r0, c0) (wave-uniform).  The row offsets are uniform and kept in
// scalar registers (left to itself the compiler forms each element's 64-bit
// offset with a quarter-rate vector multiply-add), and a tile that lies
// wholly inside the output (nearly every tile) runs a copy of the loop with
// no per-element bounds test.
// The lane's value exchanged with its neighbour (lane ^ 1), by DPP.
__device__ __forceinline__ int64_t swap_adjacent(int64_t v) {
  constexpr int kQuadSwap = 0xB1;  // quad_perm [1, 0, 3, 2]
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), kQuadSwap, 0xF, 0xF, false));
  const uint32_t hi =
      static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v >> 32), kQuadSwap, 0xF, 0xF, false));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Int64 outputs of one 16 x 16 block whose four rows per lane are y[0..3]
// (rows 4 (lane >> 4) + t of column lane & 15), written two columns per
// lane: neighbouring lanes swap half their values, so the even lane holds
// rows t = 0 and 2 and the odd lane rows 1 and 3, each at the two columns
// (lane & 14), (lane & 14) + 1 — one 16-byte store per row.  Half the store
// instructions of one store per element: the output writes are bound by the
// store instructions a CU has in flight, not by their bytes.  `at` points to
// the element (4 (lane >> 4), lane & 14) of the block; ld is even and `at`
// 16-byte aligned.
__device__ __forceinline__ void store_int64_pairs(const int64_t (&y)[4], gptr<int64_t> at, int64_t ld) {
  typedef int64_t i64x2 __attribute__((ext_vector_type(2)));
  const bool odd = (threadIdx.x & 1) != 0;
  const int64_t ra = swap_adjacent(odd ? y[0] : y[1]);
  const int64_t rb = swap_adjacent(odd ? y[2] : y[3]);
  i64x2 v0, v1;
  v0.x = odd ? ra : y[0];
  v0.y = odd ? y[1] : ra;
  v1.x = odd ? rb : y[2];
  v1.y = odd ? y[3] : rb;
  gptr<int64_t> p = at + (odd ? ld : 0);
  __builtin_nontemporal_store(v0, reinterpret_cast<__attribute__((address_space(1))) i64x2 *>(p));
  __builtin_nontemporal_store(v1, reinterpret_cast<__attribute__((address_space(1))) i64x2 *>(p + 2 * ld));
}

template <int RCAP, int MI, int NJ>
__device__ __forceinline__ void register_epilogue(KArgs<RCAP> &g, const Epi<RCAP> &e, int c_act,
                                                  const i32x4 (&acc)[RCAP][MI][NJ], int r0, int c0,
                                                  int m_lim, int n_lim, const ColScale (&cs)[NJ]) {
  const int lane = threadIdx.x & 63;
  const int64_t idx0 = static_cast<int64_t>(r0 + 4 * (lane >> 4)) * e.out_ld + c0 + (lane & 15);
  const bool interior = r0 + 16 * MI <= m_lim && c0 + 16 * NJ <= n_lim;
  // int64 interior tiles with 16-byte aligned rows: two columns per store
  const bool pairs = interior && e.out_dtype == RNSMX_INT64 && c_act == RCAP && (e.out_ld & 1) == 0 &&
                     (reinterpret_cast<uintptr_t>(e.out) & 15) == 0 && (c0 & 1) == 0;
  if (pairs) {
    const int64_t pidx0 = static_cast<int64_t>(r0 + 4 * (lane >> 4)) * e.out_ld + c0 + (lane & 14);
    static_for<MI>([&](auto I) {
      constexpr int i = decltype(I)::value;
      int64_t roff = i * 16 * e.out_ld;
      pin_sgpr(roff);
      static_for<NJ>([&](auto J) {
        constexpr int j = decltype(J)::value;
        int64_t y[4];
        static_for<4>([&](auto T) {
          constexpr int t = decltype(T)::value;
          int32_t v[RCAP];
          static_for<RCAP>([&](auto C) { v[decltype(C)::value] = acc[decltype(C)::value][i][j][t]; });
          y[t] = garner_from_sums<RCAP>(e, v, RCAP);
        });
        store_int64_pairs(y, as_global<int64_t>(e.out) + pidx0 + roff + j * 16, e.out_ld);
      });
    });
    return;
  }
  // always inlined: a call would pass the accumulators by reference, i.e.
  // through memory for the whole kernel (the inliner gives up on the
  // generic variant's size once a wave holds 64 x 64 x 6 channels)
  auto run = [&](auto FAST, auto OUT, auto INTERIOR) __attribute__((always_inline)) {
    static_for<MI>([&](auto I) {
      constexpr int i = decltype(I)::value;
      static_for<4>([&](auto T) {
        constexpr int t = decltype(T)::value;
        int64_t roff = (i * 16 + t) * e.out_ld;
        pin_sgpr(roff);
        const int row = r0 + i * 16 + 4 * (lane >> 4) + t;
        static_for<NJ>([&](auto J) {
          constexpr int j = decltype(J)::value;
          const int col = c0 + j * 16 + (lane & 15);
          if (decltype(INTERIOR)::value || (row < m_lim && col < n_lim)) {
            int32_t v[RCAP];
            static_for<RCAP>([&](auto C) { v[decltype(C)::value] = acc[decltype(C)::value][i][j][t]; });
            finish_element<RCAP, decltype(FAST)::value, decltype(OUT)::value>(g, e, c_act, v,
                                                                              idx0 + roff + j * 16, cs[j]);
          }
        });
      });
    });
  };
  with_epilogue<RCAP>(e, c_act, [&](auto FAST, auto OUT) __attribute__((always_inline)) {
    if (interior)
      run(FAST, OUT, std::true_type{});
    else
      run(FAST, OUT, std::false_type{});
  });
}

// Byte offset of channel c's plane with the channel clamped to a valid one:
// loads of channels at or past the active count read channel 0 again (their
// products are never used), so every load in the main loops is
// unconditional.  Loads under a branch or an execution mask make the
// compiler wait for every outstanding load at the join, which empties the
// prefetch pipeline.
__device__ __forceinline__ int64_t plane_off(int c, int c_act, int64_t stride) {
  return (c < c_act ? c : 0) * stride;
}

__device__ __forceinline__ i32x4 select16(bool keep, i32x4 v) {
  const i32x4 zero = {0, 0, 0, 0};
  return keep ? v : zero;
}

// Packed weights: the row stride of the per-row terms after the 2R
// activation planes, past every row a tile of up to 64 rows can address.
__host__ __device__ constexpr int64_t packed_corr_ld(int64_t m) { return (m + 63) / 64 * 64 + 64; }

// Byte offset of activation plane p of a packed-weight product: planes
// [0, RCAP) are the residues a of channel p, [RCAP, 2 RCAP) the residues a'
// of channel p - RCAP, which start after all `channels` a planes.  Channels
// at or past the active count read channel 0 (as plane_off).
template <int RCAP>
__device__ __forceinline__ int64_t packed_plane_off(int p, int c_act, int channels, int64_t stride) {
  const int c = p < RCAP ? p : p - RCAP;
  return (p < RCAP ? 0 : channels * stride) + plane_off(c, c_act, stride);
}

// Adds each row's term (128 sum_k a_k) mod m_c to the channel sums of a
// (16 MI) x (16 NJ) block whose top row is r0 (packed weights; added once
// per tile, before any exchange).  The lane's rows 4 (lane >> 4) .. +3 of
// each 16-row block are one aligned 16-byte load.
template <int RCAP, int MI, int NJ>
__device__ __forceinline__ void add_packed_rows(KArgs<RCAP> &g, i32x4 (&acc)[RCAP][MI][NJ], int r0, int c_act) {
  const int lane = threadIdx.x & 63;
  const int64_t ld = packed_corr_ld(g.m);
  const int32_t *terms = reinterpret_cast<const int32_t *>(g.a + 2 * g.mods.channels * g.a_cs);
  static_for<RCAP>([&](auto C) {
    constexpr int c = decltype(C)::value;
    if (c >= c_act) return;
    static_for<MI>([&](auto I) {
      constexpr int i = decltype(I)::value;
      const i32x4 t = *reinterpret_cast<const i32x4 *>(terms + c * ld + r0 + 16 * i + 4 * (lane >> 4));
      static_for<NJ>([&](auto J) { acc[c][i][decltype(J)::value] += t; });
    });
  });
}

// Bijection of [0, total) that gives each XCD one contiguous run of unit
// numbers.  Workgroups are handed to the 8 XCDs round-robin (workgroup b
// runs on XCD b % 8), and each XCD has its own L2; units are numbered
// M-block fastest, so contiguous runs keep the workgroups that read the
// same weight columns (and K range) on the same L2.
__device__ __forceinline__ int xcd_order(int b, int total) {
  const int xcd = b & 7, local = b >> 3;
  const int base = total >> 3, rem = total & 7;
  return xcd * base + min(xcd, rem) + local;
}

// What one workgroup computes: output tile (mt, nt) and its K split
// (split < 0: the whole K range), and for a split tile its index among the
// split tiles (the exchange slot).  Workgroups [0, split_from) take the
// whole tiles [0, split_from): they are dispatched first and spread over
// every XCD.  The rest take (tile, split) units of the tiles from
// split_from on, split-minor: with each XCD's contiguous run of units, the
// splits of one tile run on one XCD and exchange their residues through
// its L2 (split-major put the halves of a tile on different XCDs, so the
// exchange went through the MALL).
struct WorkUnit {
  int mt, nt, split, split_tile;
};

template <typename G>
__device__ __forceinline__ WorkUnit work_of(G &g) {
  const int tiles = g.tiles_m * g.tiles_n;
  const int whole = g.split_from;
  const int b = blockIdx.x;
  WorkUnit w;
  int t;
  if (b < whole) {
    t = xcd_order(b, whole);
    w.split = -1;
  } else {
    const int parted = tiles - whole;
    const int u = xcd_order(b - whole, parted * g.splits);
    w.split = u % g.splits;
    t = whole + u / g.splits;
  }
  w.mt = t % g.tiles_m;
  w.nt = t / g.tiles_m;
  w.split_tile = t - whole;
  return w;
}

// The K range of one split, in 64-byte steps from ks0: nk steps (at least
// one: the launcher sizes kchunk so every split has work), and the A bytes
// per row that lie inside the true K from ks0 on (a_k in GemmArgs, less the
// bytes before the split).
struct KRange {
  int ks0, nk, a_k;
};

template <typename G>
__device__ __forceinline__ KRange k_range(G &g, int split) {
  KRange r;
  if (split < 0) {
    r.ks0 = 0;
    r.nk = g.kp >> 6;
    r.a_k = g.a_k;
  } else {
    r.ks0 = split * g.kchunk;
    r.nk = min(g.kchunk, (g.kp >> 6) - r.ks0);
    r.a_k = g.a_k - r.ks0 * 64;
  }
  return r;
}

// ---------------------------------------------------------------------------
// Residue exchange of a K split.  The S workgroups of one output tile hold
// int32 partial sums over disjoint K ranges; the channel-c accumulator of
// the whole K is their sum, so its residue mod m_c is the sum of the
// partials' residues mod m_c (the K split is exact in RNS, whatever the
// split).  Each wave reduces its partial sums to canonical residues (one
// byte per channel, so up to four channels pack into one 32-bit word per
// element), writes them to its slot of the exchange area, and takes a
// ticket on its (tile, wave) counter.  The wave that draws the last ticket
// adds the other splits' residues to its own partial sums (each an int32
// congruent to the whole accumulator afterwards, which is all the Garner
// epilogue needs), returns the counter to zero for the next call, and
// finishes the tile; the others are done.  No wave waits for another, so
// the protocol needs neither co-residency nor a spin loop.
//
// Visibility across XCDs (each has its own L2): the residues are written
// and read with agent-scope atomic accesses (writes through to, and reads
// from, the device-coherent level, not a possibly stale L2 copy), and the
// writer's stores complete (vmcnt 0) before its ticket increment issues;
// the reader's loads issue only after its ticket returned.  This gives the
// release/acquire order of the handoff without an L2 writeback or
// invalidate, which would also flush or drop the weight columns other
// workgroups on the same XCD are still reading.
// ---------------------------------------------------------------------------
// One 16-byte exchange word group of a lane, stored word-major: word q of
// lane l sits at byte 256 q + 4 l of its 1 KB chunk, so each of the four
// 32-bit agent-scope stores (or loads) of a wave covers 256 contiguous
// bytes (whole cache lines: written through, a partly covered line would
// be merged at the memory side).
__device__ __forceinline__ void store_coherent(int8_t *p, i32x4 v) {
  static_for<4>([&](auto Q) {
    constexpr int q = decltype(Q)::value;
    __hip_atomic_store(reinterpret_cast<uint32_t *>(p + 256 * q), static_cast<uint32_t>(v[q]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  });
}

__device__ __forceinline__ i32x4 load_coherent(const int8_t *p) {
  i32x4 v;
  static_for<4>([&](auto Q) {
    constexpr int q = decltype(Q)::value;
    v[q] = static_cast<int32_t>(__hip_atomic_load(reinterpret_cast<uint32_t *>(const_cast<int8_t *>(p + 256 * q)),
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  });
  return v;
}

// s_waitcnt vmcnt(0) alone (expcnt and lgkmcnt left at their maxima), with
// compiler barriers so no memory access moves across it.
__device__ __forceinline__ void wait_vm_all() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));
  asm volatile("" ::: "memory");
}

// The tiles built with the exchange (the host splits K only for these):
// up to 4 channels, and few enough accumulators that the exchange code does
// not raise the kernel's register count (and so lower its occupancy, split
// or not): stream tiles of one or two 16 x 16 blocks down a column, MFMA
// tiles of one column block per wave; the LDS kernel always.
constexpr bool stream_splits(int rcap, int mb, int nb) { return rcap <= 4 && nb == 1 && mb <= 2; }
constexpr bool mfma_splits(int rcap, int mb, int nb) { return rcap <= 4 && nb == 1; }

// One wave's part of the exchange, for a (16 MI) x (16 NJ) block of
// accumulators per channel: one residue byte per channel, four channels per
// 32-bit word, XW = ceil(R / 4) words per element (chunk (i, j) of split s
// is XW consecutive 1 KB blocks, word-major).  slot = tile * waves + wave.
// Returns true in the wave that finishes the tile, whose acc then holds
// sums congruent to the whole-K accumulators.
template <int RCAP>
constexpr int xchg_words() {
  return (RCAP + 3) / 4;
}

template <int RCAP, int MI, int NJ>
__device__ __forceinline__ bool split_exchange(KArgs<RCAP> &g, const Epi<RCAP> &e, i32x4 (&acc)[RCAP][MI][NJ],
                                               int64_t slot, int split) {
  static_assert(RCAP <= 8, "at most two words of residue bytes per element");
  constexpr int XW = xchg_words<RCAP>();
  constexpr int CH = MI * NJ * XW;  // 1 KB blocks per wave and split
  const int lane = threadIdx.x & 63;
  const int S = g.splits;
  int8_t *base = g.xchg + slot * S * CH * 1024 + lane * 4;
  auto block = [&](int s, int i, int j, int wd) {
    return base + (static_cast<int64_t>(s) * CH + (i * NJ + j) * XW + wd) * 1024;
  };
  // canonical residues of this split's partial sums
  static_for<MI>([&](auto I) {
    constexpr int i = decltype(I)::value;
    static_for<NJ>([&](auto J) {
      constexpr int j = decltype(J)::value;
      static_for<XW>([&](auto WD) {
        constexpr int wd = decltype(WD)::value;
        i32x4 w;
        static_for<4>([&](auto T) {
          constexpr int t = decltype(T)::value;
          uint32_t packed = 0;
          static_for<4>([&](auto B) {
            constexpr int c = 4 * wd + decltype(B)::value;
            if constexpr (c < RCAP) packed |= (reduce_acc<RCAP>(e, c, acc[c][i][j][t]) & 0xFFu) << (8 * (c % 4));
          });
          w[t] = static_cast<int32_t>(packed);
        });
        store_coherent(block(split, i, j, wd), w);
      });
    });
  });
  wait_vm_all();
  uint32_t old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(g.tickets + slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old != static_cast<uint32_t>(S - 1)) return false;
  // the last ticket: every other split's residues are in place.  They are
  // read G splits at a time, every load of a group issued before the first
  // is used (own split and splits past S read a valid slot and are masked).
  asm volatile("" ::: "memory");
  auto add_word = [&](auto I, auto J, auto WD, auto T, uint32_t word) {
    constexpr int i = decltype(I)::value, j = decltype(J)::value, wd = decltype(WD)::value, t = decltype(T)::value;
    static_for<4>([&](auto B) {
      constexpr int c = 4 * wd + decltype(B)::value;
      if constexpr (c < RCAP) acc[c][i][j][t] += static_cast<int32_t>(byte_of(word, c % 4));
    });
  };
  if constexpr (CH > 8) {
    // large wave tiles (192 accumulators): one row of NJ blocks in flight,
    // so the loads need few registers next to the accumulators
    for (int s = 0; s < S; ++s) {
      if (s == split) continue;
      static_for<MI>([&](auto I) {
        constexpr int i = decltype(I)::value;
        static_for<XW>([&](auto WD) {
          i32x4 w[NJ];
          static_for<NJ>([&](auto J) { w[J] = load_coherent(block(s, i, decltype(J)::value, decltype(WD)::value)); });
          static_for<NJ>([&](auto J) {
            static_for<4>([&](auto T) { add_word(I, J, WD, T, static_cast<uint32_t>(w[J][decltype(T)::value])); });
          });
        });
      });
    }
    if (lane == 0) __hip_atomic_store(g.tickets + slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  constexpr int G = CH >= 4 ? 1 : 4 / CH;  // at most 4 blocks (16 registers) in flight, or one split
  for (int s0 = 0; s0 < S; s0 += G) {
    i32x4 w[G][MI][NJ][XW];
    static_for<G>([&](auto U) {
      constexpr int u = decltype(U)::value;
      const int s = min(s0 + u, S - 1);
      static_for<MI>([&](auto I) {
        static_for<NJ>([&](auto J) {
          static_for<XW>([&](auto WD) {
            constexpr int i = decltype(I)::value, j = decltype(J)::value, wd = decltype(WD)::value;
            w[u][i][j][wd] = load_coherent(block(s, i, j, wd));
          });
        });
      });
    });
    static_for<G>([&](auto U) {
      constexpr int u = decltype(U)::value;
      const bool use = s0 + u < S && s0 + u != split;
      static_for<MI>([&](auto I) {
        static_for<NJ>([&](auto J) {
          static_for<XW>([&](auto WD) {
            static_for<4>([&](auto T) {
              const i32x4 &x = w[u][decltype(I)::value][decltype(J)::value][decltype(WD)::value];
              add_word(I, J, WD, T, use ? static_cast<uint32_t>(x[decltype(T)::value]) : 0u);
            });
          });
        });
      });
    });
  }
  if (lane == 0) __hip_atomic_store(g.tickets + slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// ---------------------------------------------------------------------------
// Stream GEMM (M <= 128: decode, continuous batches, small C2 shapes).  The weight
// residues are read once and the problem is a few MB, so latency rules:
// every wave issues all the loads of a chunk of U K steps before its first
// MFMA.  A workgroup owns a (16*MB) x (16*NB) output tile; its KS waves
// split K (wave w takes chunks w, w + KS, ... of U steps) and each wave
// accumulates every channel.  With KS > 1 the int32 partial sums meet in LDS
// (atomic adds: a sum of partial sums over disjoint K ranges is the full
// accumulator, which fits int32); each element is then reduced once.  With
// KS = 1 the epilogue runs straight from the MFMA registers.
// ---------------------------------------------------------------------------
// K steps per chunk: as many as fit next to the accumulators in 240
// registers (two waves per SIMD), at most ucap (4; 8 for the wide form,
// which long-K decode takes: C5 M=1 39.5 us against 42.5 with 4, while at
// K = 768 the larger chunks cost 7-15 %).
constexpr int stream_u_of(int rcap, bool araw, int mb, int nb, int ucap = 4, bool pk = false) {
  // 16-byte loads per K step (packed weights: 2R activation planes, 2 weight planes)
  const int frags = (pk ? 2 * rcap : araw ? 1 : rcap) * mb + (pk ? 2 : rcap) * nb;
  const int u = (240 - 4 * rcap * mb * nb) / (4 * frags);
  return u < 1 ? 1 : (u > ucap ? ucap : u);
}

// PK: packed weights (two byte planes; activations as 2R residue planes).
// CA: channels computed (the adaptive prefix when it is shorter than the
// capacity: loads and MFMAs of the channels past it are not issued; the
// packed form computes every channel).
template <int RCAP, int MB, int NB, bool ARAW, int UCAP, bool PK, int CA>
__device__ __forceinline__ void stream_main(KArgs<RCAP> &g, const int c_act) {
  static_assert(!(PK && ARAW), "packed weights take residue-plane activations");
  static_assert(CA >= 1 && CA <= RCAP && (!PK || CA == RCAP), "channels computed");
  constexpr int BM = 16 * MB, BN = 16 * NB, TILE = BM * BN;
  constexpr int AP = PK ? 2 * RCAP : ARAW ? 1 : RCAP;  // activation planes per K step
  constexpr int BP = PK ? 2 : RCAP;                    // weight planes per K step
  constexpr int APE = PK ? 2 * RCAP : ARAW ? 1 : CA;   // ... of them loaded
  constexpr int BPE = PK ? 2 : CA;
  constexpr int U = stream_u_of(RCAP, ARAW, MB, NB, UCAP, PK);
  extern __shared__ __attribute__((aligned(16))) int32_t sacc[];  // [RCAP][TILE] when KS > 1

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nthreads = g.threads, ks_n = nthreads >> 6;
  const WorkUnit wu = work_of(g);
  const int mt = wu.mt, nt = wu.nt, split = wu.split;
  const int m0 = mt * BM, n0 = nt * BN;
  const KRange kr = k_range(g, split);
  const int nk = kr.nk, a_k = kr.a_k;
  const int kofs = (lane >> 4) * 16;

  const int8_t *ap[MB];
  const int8_t *bp[NB];
  static_for<MB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    const int row = min(m0 + i * 16 + (lane & 15), g.m - 1);
    ap[i] = g.a + static_cast<int64_t>(row) * g.a_ld + kr.ks0 * 64;
  });
  const int nblk = (g.n + 15) >> 4;
  static_for<NB>([&](auto J) {
    constexpr int j = decltype(J)::value;
    const int jb = min(nt * NB + j, nblk - 1);
    bp[j] = g.b + static_cast<int64_t>(jb) * g.b_ld + kr.ks0 * 1024 + lane * 16;
  });
  int64_t boff[BP], aoff[AP];
  static_for<BP>([&](auto C) {
    constexpr int c = decltype(C)::value;
    boff[c] = PK ? c * g.b_cs : plane_off(c, c_act, g.b_cs);
  });
  static_for<AP>([&](auto PP) {
    constexpr int p = decltype(PP)::value;
    aoff[p] = PK ? packed_plane_off<RCAP>(p, c_act, g.mods.channels, g.a_cs) : plane_off(p, c_act, g.a_cs);
  });

  const i32x4 zero = {0, 0, 0, 0};
  i32x4 acc[RCAP][MB][NB];
  static_for<RCAP>([&](auto C) {
    static_for<MB>([&](auto I) {
      static_for<NB>([&](auto J) { acc[C][I][J] = decltype(C)::value < CA ? acc_zero() : zero; });
    });
  });

  i32x4 fa[U][AP][MB], fb[U][BP][NB];
  // loads and MFMAs of the chunk's steps [P0, P1)
  auto load_part = [&](int q, auto P0, auto P1) {
    static_for<U>([&](auto UU) {
      constexpr int u = decltype(UU)::value;
      if constexpr (u >= decltype(P0)::value && u < decltype(P1)::value) {
        const int ks = min(q + u, nk - 1);
        const int ka = ks * 64 + kofs;
        const bool av = (q + u < nk) && (ka < a_k);
        const int kac = min(ka, a_k - 16);
        static_for<APE>([&](auto PP) {
          constexpr int p = decltype(PP)::value;
          static_for<MB>([&](auto I) {
            constexpr int i = decltype(I)::value;
            fa[u][p][i] = select16(av, load16(ap[i] + aoff[p] + kac));
          });
        });
        static_for<BPE>([&](auto C) {
          constexpr int c = decltype(C)::value;
          static_for<NB>([&](auto J) {
            constexpr int j = decltype(J)::value;
            // the 8-step chunks serve decode over a long K (a few 16-row
            // tiles): weights loaded with the streaming hint (C5 M=1: 34.3
            // against 38.1 us; neutral at 2-4 row tiles)
            fb[u][c][j] = UCAP == 8 ? load16_nt(bp[j] + boff[c] + ks * 1024) : load16(bp[j] + boff[c] + ks * 1024);
          });
        });
      }
    });
  };
  auto load_chunk = [&](int q) { load_part(q, std::integral_constant<int, 0>{}, std::integral_constant<int, U>{}); };
  auto mfma_part = [&](auto P0, auto P1) {
    static_for<U>([&](auto UU) {
      constexpr int u = decltype(UU)::value;
      if constexpr (u >= decltype(P0)::value && u < decltype(P1)::value) {
        // every computed channel, with no branch (with CA = RCAP, channels
        // past the prefix read channel 0's plane; their sums are dropped by
        // the epilogue)
        static_for<CA>([&](auto C) {
          constexpr int c = decltype(C)::value;
          static_for<MB>([&](auto I) {
            constexpr int i = decltype(I)::value;
            static_for<NB>([&](auto J) {
              constexpr int j = decltype(J)::value;
              if constexpr (PK) {
                // a' x hi + a x lo: the channel's residue of the weight, formed by the MFMAs
                acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u][RCAP + c][i], fb[u][0][j],
                                                                     acc[c][i][j], 0, 0, 0);
                acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u][c][i], fb[u][1][j],
                                                                     acc[c][i][j], 0, 0, 0);
              } else {
                acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u][ARAW ? 0 : c][i], fb[u][c][j],
                                                                     acc[c][i][j], 0, 0, 0);
              }
            });
          });
        });
      }
    });
  };
  auto mfma_chunk = [&]() { mfma_part(std::integral_constant<int, 0>{}, std::integral_constant<int, U>{}); };

  // first chunk in flight before the epilogue constants are waited for
  load_chunk(wave * U);
  Epi<RCAP> e;
  load_epi<RCAP>(g, e, c_act);
  pin_epi<RCAP>(e);
  int m_lim = g.m, n_lim = g.n;
  pin_sgpr(m_lim);
  pin_sgpr(n_lim);
  // float-epilogue column factors, read now so their latency hides behind
  // the K loop: columns n0 + 16 j + (lane & 15) for the register epilogue
  // (ks_n == 1, j < NB <= 4), n0 + (4 tid) % BN + v for the LDS one (the
  // stride 4 * blockDim.x is a multiple of BN, so each thread keeps its
  // columns every trip)
  ColScale cs4[4];
  static_for<4>([&](auto V) {
    constexpr int v = decltype(V)::value;
    const int col = ks_n == 1 ? n0 + (v < NB ? v : 0) * 16 + (lane & 15) : n0 + (threadIdx.x * 4) % BN + v;
    cs4[v] = col_scale<RCAP>(e, col, n_lim);
  });
  // the column of a thread that finishes one element (few rows, below)
  const ColScale cs1 = col_scale<RCAP>(e, n0 + threadIdx.x % BN, n_lim);
  if constexpr (U == 8) {
    // long K: the two halves of the chunk in turn, the next chunk's first
    // half loaded while the second half's MFMAs wait for their loads
    constexpr std::integral_constant<int, 0> h0{};
    constexpr std::integral_constant<int, U / 2> h1{};
    constexpr std::integral_constant<int, U> h2{};
    int q = wave * U;
    if (q < nk) {
      for (;;) {
        const int qn = q + ks_n * U;
        mfma_part(h0, h1);
        if (qn < nk) load_part(qn, h0, h1);
        mfma_part(h1, h2);
        if (qn >= nk) break;
        load_part(qn, h1, h2);
        q = qn;
      }
    }
  } else {
    if (wave * U < nk) mfma_chunk();
    for (int q = wave * U + ks_n * U; q < nk; q += ks_n * U) {
      load_chunk(q);
      mfma_chunk();
    }
  }
  // packed weights: the per-row term, once per tile (wave 0 of the whole K
  // or of its first split)
  if constexpr (PK) {
    if (wave == 0 && split <= 0) add_packed_rows<RCAP, MB, NB>(g, acc, m0, c_act);
  }

  if (ks_n == 1) {
    // a K split over workgroups (one wave each): only the last to finish
    // this tile goes on
    if constexpr (stream_splits(RCAP, MB, NB)) {
      if (split >= 0 && !split_exchange<RCAP, MB, NB>(g, e, acc, wu.split_tile, split))
        return;
    }
    const int64_t idx0 = static_cast<int64_t>(m0 + 4 * (lane >> 4)) * e.out_ld + n0 + (lane & 15);
    ColScale cs[NB];
    static_for<NB>([&](auto J) { cs[J] = cs4[decltype(J)::value]; });
    with_epilogue<RCAP>(e, c_act, [&](auto FAST, auto OUT) {
      static_for<MB>([&](auto I) {
        constexpr int i = decltype(I)::value;
        static_for<NB>([&](auto J) {
          constexpr int j = decltype(J)::value;
          const int col = n0 + j * 16 + (lane & 15);
          static_for<4>([&](auto T) {
            constexpr int t = decltype(T)::value;
            const int row = m0 + i * 16 + 4 * (lane >> 4) + t;
            if (row < m_lim && col < n_lim) {
              int32_t v[RCAP];
              static_for<RCAP>([&](auto C) { v[decltype(C)::value] = acc[decltype(C)::value][i][j][t]; });
              // the row step is uniform: only idx0 is per lane
              const int64_t idx = idx0 + (i * 16 + t) * e.out_ld + j * 16;
              finish_element<RCAP, decltype(FAST)::value, decltype(OUT)::value>(g, e, c_act, v, idx, cs[j]);
            }
          });
        });
      });
    });
    return;
  }

  for (int i = threadIdx.x; i < RCAP * TILE; i += nthreads) sacc[i] = 0;
  __syncthreads();
  static_for<RCAP>([&](auto C) {
    constexpr int c = decltype(C)::value;
    if (c >= c_act) return;
    static_for<MB>([&](auto I) {
      constexpr int i = decltype(I)::value;
      static_for<NB>([&](auto J) {
        constexpr int j = decltype(J)::value;
        static_for<4>([&](auto T) {
          constexpr int t = decltype(T)::value;
          atomicAdd(&sacc[c * TILE + (i * 16 + 4 * (lane >> 4) + t) * BN + j * 16 + (lane & 15)],
                    acc[c][i][j][t]);
        });
      });
    });
  });
  __syncthreads();

  const int rows_here = min(BM, m_lim - m0);
  if (rows_here * BN <= nthreads) {
    // few rows (decode): one element per thread, so the Garner chains of
    // the tile run side by side (C3: 16 elements on 16 threads instead of 4)
    const int x = threadIdx.x;
    with_epilogue<RCAP>(e, c_act, [&](auto FAST, auto OUT) {
      if (x < rows_here * BN && n0 + x % BN < n_lim) {
        int32_t v[RCAP];
        static_for<RCAP>([&](auto C) { v[decltype(C)::value] = sacc[decltype(C)::value * TILE + x]; });
        finish_element<RCAP, decltype(FAST)::value, decltype(OUT)::value>(
            g, e, c_act, v, static_cast<int64_t>(m0 + x / BN) * e.out_ld + n0 + x % BN, cs1);
      }
    });
    return;
  }
  // each thread finishes 4 adjacent columns of one row; the stride
  // 4 * blockDim.x is a multiple of BN, so the columns are the same every trip
  const ColScale(&cs)[4] = cs4;
  with_epilogue<RCAP>(e, c_act, [&](auto FAST, auto OUT) {
    for (int x = threadIdx.x * 4; x < rows_here * BN; x += nthreads * 4) {
      const int row = x / BN, col = x % BN;
      i32x4 sv[RCAP];
      static_for<RCAP>([&](auto C) {
        constexpr int c = decltype(C)::value;
        sv[c] = *reinterpret_cast<const i32x4 *>(&sacc[c * TILE + x]);
      });
      static_for<4>([&](auto V) {
        constexpr int v4 = decltype(V)::value;
        if (n0 + col + v4 < n_lim) {
          int32_t v[RCAP];
          static_for<RCAP>([&](auto C) { v[decltype(C)::value] = sv[decltype(C)::value][v4]; });
          finish_element<RCAP, decltype(FAST)::value, decltype(OUT)::value>(
              g, e, c_act, v, static_cast<int64_t>(m0 + row) * e.out_ld + n0 + col + v4, cs[v4]);
        }
      });
    }
  });
}

template <int RCAP, int MB, int NB, bool ARAW, int UCAP, bool PK>
__device__ __forceinline__ void stream_body() {
  KArgs<RCAP> &g = kernel_args<GemmArgsK<RCAP>>();
  load_hot_args(g);
  __shared__ int64_t red[4];
  __shared__ int bcast;
  const int c_act = active_channels<RCAP>(g, red, &bcast, g.threads);
  // a prefix one channel short of the capacity runs a body without that
  // channel's loads and MFMAs (C5-shaped decode: 3 of 4 weight planes)
  if constexpr (!PK && (RCAP == 4 || RCAP == 6)) {
    if (c_act == RCAP - 1) {
      stream_main<RCAP, MB, NB, ARAW, UCAP, PK, RCAP - 1>(g, c_act);
      return;
    }
  }
  stream_main<RCAP, MB, NB, ARAW, UCAP, PK, RCAP>(g, c_act);
}

template <int RCAP, int MB, int NB, bool ARAW, int UCAP>
__global__ __launch_bounds__(256) void stream_kernel(const GemmArgsK<RCAP> args) {
  stream_body<RCAP, MB, NB, ARAW, UCAP, false>();
}

template <int RCAP, int MB, int NB, int UCAP>
__global__ __launch_bounds__(256) void stream_packed_kernel(const GemmArgsK<RCAP> args) {
  stream_body<RCAP, MB, NB, false, UCAP, true>();
}

// ---------------------------------------------------------------------------
// Packed weights at decode (a few tokens): the MFMA rows carry channels.
// The packed weight bytes hi and lo are the same for every channel, so one
// 16-row A fragment can hold RCAP channels of TPB = 16 / RCAP tokens (row
// t * RCAP + c: token t, channel c) and a single MFMA against hi (or lo)
// makes every channel's product at once: per K step two B loads, two A
// loads per block of TPB tokens and three MFMAs (a' x hi + a x lo into the
// sums, a x ones into the row sums that carry the 128 sum_k a_k term),
// where the per-channel form issues 2R A loads and 2R MFMAs per 16 rows.
// A is encoded for this kernel as [block][a' | a][kp/64][1 KB] fragments
// (a_cs = bytes per block); rows past the tokens or channels are zero.
// A workgroup owns 16 columns and every token (NBLK = 1, 2, 4 or 8 blocks;
// the B fragments of a step serve them all); its KS waves split K as in
// stream_kernel, chunks of U steps in flight per wave (fewer with more
// blocks: their A fragments share the registers).  The
// sums meet in LDS, where each thread gathers the RCAP channel sums of one
// output element (a column of the fragment) for the Garner epilogue.  The
// row-sum term keeps |sum| <= 2 K 128 max_half + 128 K max_half (host
// bound: K <= 44,035 for max_half = 127).
// ---------------------------------------------------------------------------
template <int RCAP, int NBLK>
__global__ __launch_bounds__(256) void rows_packed_kernel(const GemmArgsK<RCAP> args) {
  KArgs<RCAP> &g = kernel_args<GemmArgsK<RCAP>>();
  prefetch_kernel_args<kGemmHotArgBytes>();
  static_assert(RCAP == 4 || RCAP == 6, "4 or 6 channel rows per token");
  constexpr int TPB = 16 / RCAP;                                   // tokens per 16-row block
  // K steps per chunk: the most that keep 3 waves per SIMD (all 768
  // workgroups of N=12288 in one round) up to 4 blocks (2 blocks with 6
  // steps: 204 VGPRs, M=4 37.1 against 35.4 us; 4 blocks with 4: 272, M=8
  // 46.1 against 42.8); 8 blocks keep 2 steps at one wave per SIMD (one step
  // at two waves measured slower, M=16 74.4 against 69.3 us)
  constexpr int U = NBLK == 1 ? 8 : NBLK == 2 ? 4 : 2;
  __shared__ __attribute__((aligned(16))) int32_t sums[NBLK][16][16];
  __shared__ int64_t red[4];
  __shared__ int bcast;

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nthreads = g.threads, ks_n = nthreads >> 6;
  const int c_act = active_channels<RCAP>(g, red, &bcast, nthreads);
  const int n0 = blockIdx.x * 16;
  const int nk = g.kp >> 6;
  const int64_t mstride = static_cast<int64_t>(nk) * 1024;  // a' fragments, then a fragments
  const int8_t *ap = g.a + lane * 16;
  const int8_t *bp = g.b + static_cast<int64_t>(blockIdx.x) * g.b_ld + lane * 16;
  const i32x4 ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};

  i32x4 acc[NBLK], rsum[NBLK];
  static_for<NBLK>([&](auto B) {
    acc[decltype(B)::value] = acc_zero();
    rsum[decltype(B)::value] = acc_zero();
  });
  // rows past the block's tokens hold zeros: their lanes skip the A loads
  // (M=1/8/16 at K=4096: 26.8/47.3/69.3 against 29.2/51.2/73.5 us with
  // every lane loading).  With two blocks the unmasked loads measured
  // faster (M=4: 38.3 against 40.3 us), as did a buffer resource whose
  // out-of-range offsets read zeros (M=16: 80.1 us).
  bool rowv[NBLK];
  static_for<NBLK>([&](auto B) {
    constexpr int b = decltype(B)::value;
    rowv[b] = (lane & 15) < min(TPB, max(0, g.m - b * TPB)) * RCAP;
  });
  i32x4 fh[U], fl[U], fa2[U][NBLK], fa[U][NBLK];
  // loads and MFMAs of the chunk's steps [P0, P1)
  auto load_part = [&](int q, auto P0, auto P1) {
    static_for<U>([&](auto UU) {
      constexpr int u = decltype(UU)::value;
      if constexpr (u >= decltype(P0)::value && u < decltype(P1)::value) {
        const int ks = min(q + u, nk - 1);
        const bool live = q + u < nk;  // steps past K: zero activations
        fh[u] = load16_nt(bp + ks * 1024);
        fl[u] = load16_nt(bp + g.b_cs + ks * 1024);
        static_for<NBLK>([&](auto B) {
          constexpr int b = decltype(B)::value;
          if constexpr (NBLK == 2) {
            fa2[u][b] = select16(live, load16(ap + b * g.a_cs + ks * 1024));
            fa[u][b] = select16(live, load16(ap + b * g.a_cs + mstride + ks * 1024));
          } else {
            i32x4 x2 = {0, 0, 0, 0}, x = {0, 0, 0, 0};
            if (live && rowv[b]) {
              x2 = load16(ap + b * g.a_cs + ks * 1024);
              x = load16(ap + b * g.a_cs + mstride + ks * 1024);
            }
            fa2[u][b] = x2;
            fa[u][b] = x;
          }
        });
      }
    });
  };
  auto mfma_part = [&](auto P0, auto P1) {
    static_for<U>([&](auto UU) {
      constexpr int u = decltype(UU)::value;
      if constexpr (u >= decltype(P0)::value && u < decltype(P1)::value) {
        static_for<NBLK>([&](auto B) {
          constexpr int b = decltype(B)::value;
          acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa2[u][b], fh[u], acc[b], 0, 0, 0);
          acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u][b], fl[u], acc[b], 0, 0, 0);
          rsum[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u][b], ones, rsum[b], 0, 0, 0);
        });
      }
    });
  };
  // Two halves of the register chunk in turn: the next chunk's first half
  // is loaded while the second half's MFMAs wait, so each wave keeps loads
  // in flight across its chunks (loads complete in order: the MFMAs of a
  // half wait only for that half).
  constexpr std::integral_constant<int, 0> h0{};
  constexpr std::integral_constant<int, U / 2> h1{};
  constexpr std::integral_constant<int, U> h2{};
  int q = wave * U;
  load_part(q, h0, h1);
  load_part(q, h1, h2);
  Epi<RCAP> e;
  load_epi<RCAP>(g, e, c_act);
  pin_epi<RCAP>(e);
  for (int i = threadIdx.x; i < NBLK * 256; i += nthreads) (&sums[0][0][0])[i] = 0;
  if (q < nk) {
    for (;;) {
      const int qn = q + ks_n * U;
      mfma_part(h0, h1);
      if (qn < nk) load_part(qn, h0, h1);
      mfma_part(h1, h2);
      if (qn >= nk) break;
      load_part(qn, h1, h2);
      q = qn;
    }
  }
  __syncthreads();
  // channel sums of every element: a' hi + a lo + 128 sum_k a
  static_for<NBLK>([&](auto B) {
    constexpr int b = decltype(B)::value;
    static_for<4>([&](auto T) {
      constexpr int t = decltype(T)::value;
      atomicAdd(&sums[b][4 * (lane >> 4) + t][lane & 15], acc[b][t] + 128 * rsum[b][t]);
    });
  });
  __syncthreads();

  const int m_lim = g.m, n_lim = g.n;
  with_epilogue<RCAP>(e, c_act, [&](auto FAST, auto OUT) {
    for (int x = threadIdx.x; x < m_lim * 16; x += nthreads) {
      const int token = x >> 4, j = x & 15, col = n0 + j;
      if (col >= n_lim) continue;
      const int b = token / TPB, row0 = (token % TPB) * RCAP;
      int32_t v[RCAP];
      static_for<RCAP>([&](auto C) { v[decltype(C)::value] = sums[b][row0 + decltype(C)::value][j]; });
      finish_element<RCAP, decltype(FAST)::value, decltype(OUT)::value>(
          g, e, c_act, v, static_cast<int64_t>(token) * e.out_ld + col, col_scale<RCAP>(e, col, n_lim));
    }
  });
}

// ---------------------------------------------------------------------------
// MFMA GEMM (M > 128 where the LDS kernel does not apply: C2 M=256, C4;
// also smaller batches of wide or long-K shapes, e.g. C5 M=32-128).  A
// workgroup of 4 waves owns a (16*MB) x (4*16*NB) tile: the A rows (shared by
// all waves, and in raw mode by all channels) pass through a P-deep register
// ring into double-buffered LDS, 64-byte rows whose four 16-byte chunks are
// XOR-swizzled by row bits 1-2 (a_chunk_off), so both the row-wise writes
// (4 lanes per row) and the fragment reads (16 lanes down a column of
// chunks) hit disjoint banks in every group of 8 lanes; each wave owns 16*NB
// columns and streams their weight residues straight from global memory into
// a P-deep register ring.  Loads of K step ks + P are issued while step ks
// computes; the loop runs a multiple of P steps with the steps past K fed
// zero A rows, so it has no branch around a load.  Every K step feeds all
// channels, so all channel accumulators finish together and the reduction +
// Garner + store run from registers.
// ---------------------------------------------------------------------------
constexpr int kLdsRow = 64;

// LDS offset of 16-byte chunk `part` (0..3) of A row `row` in one plane.
__device__ __forceinline__ int a_chunk_off(int row, int part) {
  return row * kLdsRow + ((part ^ ((row >> 1) & 3)) << 4);
}

// NWV: waves (column groups of 16*NB) per workgroup, 4 or 3.  PK: packed
// weights (two byte planes; activations as 2R residue planes).  NTB: weight
// loads with the streaming hint (one row tile: each weight byte is read
// once per launch).
template <int RCAP, int MB, int NB, int P, bool ARAW, int NWV, bool PK, bool NTB = false>
__device__ __forceinline__ void mfma_body() {
  KArgs<RCAP> &g = kernel_args<GemmArgsK<RCAP>>();
  prefetch_kernel_args<kGemmArgBytes<RCAP>>();
  load_hot_args(g);
  static_assert(!(PK && ARAW), "packed weights take residue-plane activations");
  constexpr int BM = 16 * MB, BNW = 16 * NB;
  constexpr int AP = PK ? 2 * RCAP : ARAW ? 1 : RCAP;  // activation planes staged per K step
  constexpr int BP = PK ? 2 : RCAP;                    // weight planes per K step
  constexpr int PLANE = BM * kLdsRow;
  constexpr int ACH = AP * BM * 4;  // 16-byte A chunks per K step
  constexpr int NT = 64 * NWV;
  static_assert(NWV == 3 || NWV == 4, "3 or 4 column waves");
  constexpr int AC = (ACH + NT - 1) / NT;
  // one spare 16-byte slot takes the stores of threads without an A chunk
  __shared__ __attribute__((aligned(16))) int8_t As[2][AP * PLANE + 16];
  __shared__ int64_t red[4];
  __shared__ int bcast;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c_act = active_channels<RCAP>(g, red, &bcast, NT);
  const WorkUnit wu = work_of(g);
  const int mt = wu.mt, nt = wu.nt, split = wu.split;
  const int m0 = mt * BM, n0 = nt * (NWV * BNW) + wave * BNW;
  const KRange kr = k_range(g, split);
  const int nk = kr.nk, a_k = kr.a_k;

  // A staging: chunk q -> plane p, row, 16-byte part
  const int8_t *asrc[AC];
  int alds[AC], apart[AC];
  bool aon[AC];
  static_for<AC>([&](auto II) {
    constexpr int i = decltype(II)::value;
    const int q = tid + NT * i;
    const bool inside = q < ACH;
    const int qq = inside ? q : 0;
    const int p = qq / (BM * 4), w = qq % (BM * 4), row = w >> 2, part = w & 3;
    const int grow = min(m0 + row, g.m - 1);
    const int64_t poff = PK ? packed_plane_off<RCAP>(p, c_act, g.mods.channels, g.a_cs) : plane_off(p, c_act, g.a_cs);
    asrc[i] = g.a + poff + static_cast<int64_t>(grow) * g.a_ld + kr.ks0 * 64;
    alds[i] = inside ? p * PLANE + a_chunk_off(row, part) : AP * PLANE;
    apart[i] = part * 16;
    aon[i] = inside && (ARAW || (PK ? p % RCAP : p) < c_act);
  });
  const int8_t *bp[NB];
  const int nblk = (g.n + 15) >> 4;
  static_for<NB>([&](auto J) {
    constexpr int j = decltype(J)::value;
    const int jb = min((n0 >> 4) + j, nblk - 1);
    bp[j] = g.b + static_cast<int64_t>(jb) * g.b_ld + kr.ks0 * 1024 + lane * 16;
  });
  int64_t boff[BP];
  static_for<BP>([&](auto C) {
    constexpr int c = decltype(C)::value;
    boff[c] = PK ? c * g.b_cs : plane_off(c, c_act, g.b_cs);
  });

  const i32x4 zero = {0, 0, 0, 0};
  i32x4 ra[P][AC];
  bool akeep[P][AC];
  i32x4 fb[P][BP][NB];
  // loads of K step ks (clamped to the last one; A of steps past K is
  // zero).  The zeroing is applied when the A chunk is stored to LDS, P - 1
  // steps later: a select right after the load would make the wave wait for
  // that load (and, loads completing in order, for every load before it),
  // emptying the ring once per trip.
  auto gload = [&](auto SLOT, int ks) {
    constexpr int s = decltype(SLOT)::value;
    const int kc = min(ks, nk - 1);
    static_for<AC>([&](auto II) {
      constexpr int i = decltype(II)::value;
      const int ka = kc * 64 + apart[i];
      akeep[s][i] = aon[i] && ks < nk && ka < a_k;
      ra[s][i] = load16(asrc[i] + min(ka, a_k - 16));
    });
    static_for<BP>([&](auto C) {
      constexpr int c = decltype(C)::value;
      static_for<NB>([&](auto J) {
        constexpr int j = decltype(J)::value;
        fb[s][c][j] = NTB ? load16_nt(bp[j] + boff[c] + kc * 1024) : load16(bp[j] + boff[c] + kc * 1024);
      });
    });
  };
  auto lstore = [&](auto SLOT, int buf) {
    constexpr int s = decltype(SLOT)::value;
    static_for<AC>([&](auto II) {
      constexpr int i = decltype(II)::value;
      *reinterpret_cast<i32x4 *>(&As[buf][alds[i]]) = select16(akeep[s][i], ra[s][i]);
    });
  };

  i32x4 acc[RCAP][MB][NB];
  static_for<RCAP>([&](auto C) {
    static_for<MB>([&](auto I) { static_for<NB>([&](auto J) { acc[C][I][J] = acc_zero(); }); });
  });

  Epi<RCAP> e;
  load_epi<RCAP>(g, e, c_act);
  static_for<P>([&](auto SS) { gload(SS, decltype(SS)::value); });
  pin_epi<RCAP>(e);
  int m_lim = g.m, n_lim = g.n;
  pin_sgpr(m_lim);
  pin_sgpr(n_lim);
  // float-epilogue column factors, read now so their latency hides behind the K loop
  ColScale cs[NB];
  static_for<NB>([&](auto J) { cs[J] = col_scale<RCAP>(e, n0 + decltype(J)::value * 16 + (lane & 15), n_lim); });
  lstore(std::integral_constant<int, 0>{}, 0);
  __syncthreads();

  const int steps = (nk + P - 1) / P * P;
  // rows 16 i + (lane & 15) share (row >> 1) & 3 for every i: one per-lane offset
  const int a_frag = a_chunk_off(lane & 15, lane >> 4);
  // One trip round the ring.  MORE: later trips follow, so each step issues
  // the loads of step ks + P; the last trip issues none (every step it
  // could load lies past K), and its last step stages nothing.
  auto trip = [&](int ks0, auto MORE) {
    constexpr bool more = decltype(MORE)::value;
    static_for<P>([&](auto SS) {
      constexpr int s = decltype(SS)::value;
      const int ks = ks0 + s;
      const int buf = ks & 1;
      i32x4 fa[MB], fa2[MB];
      // skip inactive channels and the steps past K (a straight-line form
      // measured 13 % slower here: C2 M=256 12.2 -> 13.8 us)
      static_for<RCAP>([&](auto C) {
        constexpr int c = decltype(C)::value;
        if (c >= c_act || ks >= nk) return;
        if (!ARAW || c == 0) {
          static_for<MB>([&](auto I) {
            constexpr int i = decltype(I)::value;
            fa[i] = *reinterpret_cast<const i32x4 *>(&As[buf][(ARAW ? 0 : c) * PLANE + a_frag + i * 16 * kLdsRow]);
            if constexpr (PK)
              fa2[i] = *reinterpret_cast<const i32x4 *>(&As[buf][(RCAP + c) * PLANE + a_frag + i * 16 * kLdsRow]);
          });
        }
        static_for<MB>([&](auto I) {
          constexpr int i = decltype(I)::value;
          static_for<NB>([&](auto J) {
            constexpr int j = decltype(J)::value;
            if constexpr (PK) {
              // a' x hi + a x lo: the channel's residue of the weight, formed by the MFMAs
              acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa2[i], fb[s][0][j], acc[c][i][j], 0, 0, 0);
              acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[s][1][j], acc[c][i][j], 0, 0, 0);
            } else {
              acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[s][c][j], acc[c][i][j], 0, 0, 0);
            }
          });
        });
      });
      if constexpr (more) gload(SS, ks + P);
      if constexpr (more || s + 1 < P) {
        lstore(std::integral_constant<int, (s + 1) % P>{}, buf ^ 1);
        __syncthreads();
      }
    });
  };
  for (int ks0 = 0; ks0 < steps - P; ks0 += P) trip(ks0, std::true_type{});
  trip(steps - P, std::false_type{});

  // packed weights: the per-row term, once per tile (the whole K or its first split)
  if constexpr (PK) {
    if (split <= 0) add_packed_rows<RCAP, MB, NB>(g, acc, m0, c_act);
  }
  if constexpr (mfma_splits(RCAP, MB, NB)) {
    if (split >= 0 &&
        !split_exchange<RCAP, MB, NB>(g, e, acc, static_cast<int64_t>(wu.split_tile) * NWV + wave, split))
      return;
  }
  register_epilogue<RCAP, MB, NB>(g, e, c_act, acc, m0, n0, m_lim, n_lim, cs);
}

template <int RCAP, int MB, int NB, int P, bool ARAW, int NWV = 4, bool NTB = false>
__global__ __launch_bounds__(64 * NWV) void mfma_kernel(const GemmArgsK<RCAP> args) {
  mfma_body<RCAP, MB, NB, P, ARAW, NWV, false, NTB>();
}

template <int RCAP, int MB, int NB, int P>
__global__ __launch_bounds__(256) void mfma_packed_kernel(const GemmArgsK<RCAP> args) {
  mfma_body<RCAP, MB, NB, P, false, 4, true>();
}

// ---------------------------------------------------------------------------
// Large-M GEMM with LDS staging (raw int8 A, up to 4 channels).  A workgroup
// of NW waves owns a 256 x 64 output tile for every channel; per K step of
// 64 bytes it stages 256 rows of A and 4*R B fragments (64 columns x R
// channels, 1 KB each in MFMA fragment order) with direct-to-LDS loads
// (global_load_lds_dwordx4: no register staging, so S - 1 steps of loads
// are in flight).  A is loaded two K steps at a time as whole 128-byte row
// segments, so every load instruction touches 8 cache lines rather than 16
// half-used ones: the vector-memory address unit, not the MFMAs, bounds
// this loop, and A's share of its work halves.  The waves split the tile
// (NW / 2) x 2; while a wave runs the MFMAs of step k it reads the
// fragments of step k + 1 from LDS into the registers the MFMAs have just
// released.  One barrier per K step.  Rows past M and columns past N are
// clamped to the last valid ones (their products are dropped).  With
// NW = 8 the accumulators (128 registers for R = 4) fit two waves per SIMD
// with VGPR-form MFMAs, which hide each other's LDS latency.
// ---------------------------------------------------------------------------
constexpr int kLdsBM = 256, kLdsBN = 64, kLdsStages = 4;

// One direct-to-LDS load: lane l's 16 bytes at gbase + voff land at LDS
// address sbase + OFF + 16 * l (gbase and sbase wave-uniform).  Written as
// inline assembly so that the compiler does not track the LDS write: it
// would otherwise wait for every such load in flight before each LDS read
// it cannot prove disjoint, draining the pipeline.  The callers order these
// loads and the reads of the same stage with explicit vmcnt waits and
// barriers.  M0 holds the LDS address (the compiler keeps no value in M0
// across this point on gfx9); one wait state separates its write from the
// load.
template <int OFF>
__device__ __forceinline__ void lds_dma16(const int8_t *gbase, uint32_t voff, uint32_t sbase) {
  asm volatile("s_add_u32 m0, %0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3"
               :
               : "s"(sbase), "i"(OFF), "v"(voff), "s"(gbase)
               : "memory", "scc");
}

// s_waitcnt with only the vector-memory counter limited (to n <= 63).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// CA: channels computed (as lds_wide_body).
template <int RCAP, int NW, int CA>
__device__ __forceinline__ void lds_body(KArgs<RCAP> &g, int8_t *smem, const int c_act, const WorkUnit wu) {
  static_assert(RCAP <= 4, "the 256 x 64 x R tile holds R <= 4 channels");
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  static_assert(CA >= 1 && CA <= RCAP, "channels computed");
  constexpr int S = kLdsStages;               // even: each step's stage is a constant in a trip
  constexpr int AF = kLdsBM / 16;             // A fragments per stage
  constexpr int BF = RCAP * (kLdsBN / 16);    // B fragments per stage
  constexpr int STAGE = (AF + BF) * 1024;
  constexpr int WM = NW / 2, WN = 2;          // wave grid
  constexpr int MI = AF / WM, NJ = kLdsBN / 16 / WN;  // fragments of a wave's tile
  constexpr int BU = BF / NW;                 // B loads per wave per step
  static_assert(BF % NW == 0, "B fragments split evenly over the waves");

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int mt = wu.mt, nt = wu.nt, split = wu.split;
  const int m0 = mt * kLdsBM, n0 = nt * kLdsBN;
  const KRange kr = k_range(g, split);
  const int nk = kr.nk;  // a multiple of the stage count (the launcher sizes kchunk so)

  // Direct-to-LDS sources.  A is loaded two K steps at a time, as whole
  // 128-byte row segments: block b (8 rows, 1 KB) of the pair of steps
  // (e, e + 1), e even, lands in the A region of stage (e % S) + b / 16 at
  // slot (b % 16); its LDS 16-byte chunk s holds row 8 b + (s >> 3) and
  // bytes 16 ((s & 7) ^ (s >> 3)) of the 128-byte segment (the XOR spreads
  // the 8 rows that one fragment read serves over distinct banks).  Block
  // b = wave + NW u is loaded by this wave: a per-lane offset from A's base.
  // B fragment q = wave + NW u: channel q / 4, column block q % 4 (clamped
  // to the last), one contiguous 1 KB block per K step: a per-wave base and
  // offset 16 * lane.  Channels past c_act read channel 0 (their sums are
  // not used).
  constexpr int ABLK = kLdsBM / 8;            // A blocks per pair of steps
  constexpr int AU2 = ABLK / NW;              // A loads per wave per pair
  static_assert(ABLK % NW == 0 && 16 % NW == 0 && ABLK == 2 * AF, "A blocks split evenly, 16 per stage");
  static_assert(S % 2 == 0, "pairs of steps share a stage pair");
  uint32_t aoff[AU2];
  static_for<AU2>([&](auto U) {
    constexpr int u = decltype(U)::value;
    const int row = min(m0 + (wave + NW * u) * 8 + (lane >> 3), g.m - 1);
    aoff[u] = static_cast<uint32_t>(row * g.a_ld + ((lane & 7) ^ (lane >> 3)) * 16);
  });
  const int8_t *bbase[BU];
  const int nblk = (g.n + 15) >> 4;
  static_for<BU>([&](auto U) {
    constexpr int u = decltype(U)::value;
    const int q = wave + NW * u, c = q / (kLdsBN / 16);
    const int jb = min((n0 >> 4) + q % (kLdsBN / 16), nblk - 1);
    bbase[u] = g.b + plane_off(c, c_act, g.b_cs) + static_cast<int64_t>(jb) * g.b_ld + kr.ks0 * 1024;
  });
  const uint32_t boff = static_cast<uint32_t>(lane * 16);
  const int8_t *abase = g.a + kr.ks0 * 64;
  const uint32_t sbase = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int8_t *)(smem))) +
      wave * 1024);
  // B load L of K step ks into stage ST; A load U of the pair of steps
  // starting at ks (even) into the stage pair starting at ST.  Loads past
  // K, issued near the end, load the last step (pair) again into stages
  // that are never read.
  auto dma_b = [&](auto ST, auto L, int ks) {
    constexpr int st = decltype(ST)::value, l = decltype(L)::value;
    const int kc = min(ks, nk - 1);
    lds_dma16<st * STAGE + (AF + NW * l) * 1024>(bbase[l] + static_cast<int64_t>(kc) * 1024, boff, sbase);
  };
  auto dma_a = [&](auto ST, auto U, int ks) {
    constexpr int st = decltype(ST)::value, u = decltype(U)::value;
    const int kc = min(ks, nk - 2);
    // block wave + NW u: stage st + (NW u) / 16, slot (NW u) % 16 + wave
    lds_dma16<(st + (NW * u) / 16) * STAGE + ((NW * u) % 16) * 1024>(abase + kc * 64, aoff[u], sbase);
  };
  // the loads of step k (stage st = k % S): B of step k + S - 1 and, when
  // k is odd, the A pair (k + S - 1, k + S); spread over the (c, j) groups
  constexpr int NLE = BU, NLO = BU + AU2;     // loads issued at even / odd steps
  auto dma_part = [&](auto H, auto L, int k) {
    constexpr int h = decltype(H)::value, l = decltype(L)::value;
    if constexpr (l < BU)
      dma_b(std::integral_constant<int, (h + S - 1) % S>{}, L, k + S - 1);
    else
      dma_a(std::integral_constant<int, (h + S - 1) % S>{}, std::integral_constant<int, l - BU>{}, k + S - 1);
  };

  // Fragment registers: B fragment (c, j) of the next step is read as soon
  // as the last MFMA of this step that uses it has issued; A fragments are
  // double-buffered by step parity and the next step's are read during the
  // first MI (c, j) groups, so every read has most of a step to land before
  // its first use and no read waits at the step boundary.
  i32x4 fa[2][MI], fb[RCAP][NJ];
  const int8_t *rbase = smem + lane * 16;
  // A fragment i of this wave, parity p of a pair: rows 16 f + (lane & 15)
  // with f = wm MI + i, i.e. block 2 f + ((lane >> 3) & 1), chunk
  // 4 p + (lane >> 4) of row (lane & 7)
  static_assert(16 % (2 * MI) == 0, "a wave's A fragments share one stage of the pair");
  const int8_t *rabase[2];
  static_for<2>([&](auto P) {
    constexpr int p = decltype(P)::value;
    const int f0 = wm * MI;
    rabase[p] = smem + ((2 * f0) / 16) * STAGE + ((2 * f0) % 16) * 1024 + ((lane >> 3) & 1) * 1024 +
                ((lane & 7) * 8 + ((4 * p + (lane >> 4)) ^ (lane & 7))) * 16;
  });
  auto read_a = [&](auto H, auto BUF, auto I) {
    constexpr int h = decltype(H)::value, buf = decltype(BUF)::value, i = decltype(I)::value;
    fa[buf][i] = *reinterpret_cast<const i32x4 *>(rabase[h & 1] + (h & ~1) * STAGE + 2 * i * 1024);
  };
  auto read_b = [&](auto ST, auto C, auto J) {
    constexpr int st = decltype(ST)::value, c = decltype(C)::value, j = decltype(J)::value;
    fb[c][j] = *reinterpret_cast<const i32x4 *>(rbase + st * STAGE + (AF + c * 4 + wn * NJ + j) * 1024);
  };
  i32x4 acc[RCAP][MI][NJ];
  static_for<RCAP>([&](auto C) {
    static_for<MI>([&](auto I) {
      static_for<NJ>([&](auto J) {
        if constexpr (decltype(C)::value < CA)
          acc[C][I][J] = acc_zero();
        else
          acc[C][I][J] = i32x4{0, 0, 0, 0};
      });
    });
  });
  // one K step k at stage h: wait until step k + 1 landed (own loads, then
  // everyone's, which also frees the stage of k - 1 and, at odd k with the
  // LDS reads of this step drained first, the A region of stage k), refill
  // them, then the MFMAs of step k (every channel: no branch in the loop,
  // inactive channels' sums are dropped by the epilogue) with the reads of
  // step k + 1's fragments between them.  The loads of step k - 1 may still
  // be in flight: NLO of them after an odd step, NLE after an even one.
  static_assert(CA * NJ >= MI, "the A reads ride on the first MI (c, j) groups");
  static_assert(CA * NJ >= NLO, "a step's loads fit one per (c, j) group");
  auto step = [&](auto H, int k) {
    constexpr int h = decltype(H)::value;
    constexpr int nxt = (h + 1) % S, buf = h & 1, nl = (h & 1) ? NLO : NLE;
    // odd steps overwrite this step's A region: this wave's reads of it (the
    // A fragments read during the previous step, each followed by at least
    // LAFTER B reads in issue order) must have completed before the barrier.
    // LDS reads complete in order, so lgkmcnt(LAFTER) suffices and the
    // trailing B reads stay in flight.  Other LGKM-counted operations (scalar
    // loads, which may complete out of order) can only make this wait
    // stricter: while any is outstanding it counts toward LAFTER, so fewer
    // LDS reads are left in flight, never more (and the compiled loop issues
    // none).
    constexpr int LAFTER = CA * NJ - MI;
    static_assert(LAFTER >= 0 && LAFTER < 16, "lgkmcnt is 4 bits");
    if constexpr (h & 1) __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (LAFTER << 8) | (0x3 << 14));
    wait_vmcnt<(h & 1) ? NLE : NLO>();
    __builtin_amdgcn_s_barrier();
    static_for<CA>([&](auto C) {
      constexpr int c = decltype(C)::value;
      static_for<NJ>([&](auto J) {
        constexpr int j = decltype(J)::value, q = c * NJ + j;
        // load L at group (L * groups) / nl
        static_for<nl>([&](auto L) {
          constexpr int l = decltype(L)::value;
          if constexpr ((l * CA * NJ) / nl == q) dma_part(H, L, k);
        });
        static_for<MI>([&](auto I) {
          constexpr int i = decltype(I)::value;
          acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[buf][i], fb[c][j], acc[c][i][j], 0, 0, 0);
        });
        read_b(std::integral_constant<int, nxt>{}, C, J);
        if constexpr (q < MI)
          read_a(std::integral_constant<int, nxt>{}, std::integral_constant<int, buf ^ 1>{},
                 std::integral_constant<int, q>{});
        // keep the reads where they are: the scheduler otherwise sinks each
        // one to just before its first use, which exposes its latency
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  };

  // prologue: steps 0 .. S-2 in flight (A pairs (0, 1) and (2, 3), B of
  // steps 0 .. 2), in the order the loop's waits count them
  static_assert(S == 4, "the prologue covers one trip's first three steps");
  static_for<AU2>([&](auto U) { dma_a(std::integral_constant<int, 0>{}, U, 0); });
  static_for<BU>([&](auto L) { dma_b(std::integral_constant<int, 0>{}, L, 0); });
  static_for<BU>([&](auto L) { dma_b(std::integral_constant<int, 1>{}, L, 1); });
  static_for<AU2>([&](auto U) { dma_a(std::integral_constant<int, 2>{}, U, 2); });
  static_for<BU>([&](auto L) { dma_b(std::integral_constant<int, 2>{}, L, 2); });
  Epi<RCAP> e;
  load_epi<RCAP>(g, e, c_act);
  pin_epi<RCAP>(e);
  int m_lim = g.m, n_lim = g.n;
  pin_sgpr(m_lim);
  pin_sgpr(n_lim);
  // float-epilogue column factors (loads complete in order, so the waits
  // below cover them too)
  const int rw0 = m0 + wm * (MI * 16), cw0 = n0 + wn * (NJ * 16);
  ColScale cs[NJ];
  static_for<NJ>([&](auto J) { cs[J] = col_scale<RCAP>(e, cw0 + decltype(J)::value * 16 + (lane & 15), n_lim); });
  // step 0 landed: at most the B loads of steps 1, 2 and the second A pair
  // (or fewer, when column factors were loaded after them) in flight
  wait_vmcnt<2 * BU + AU2>();
  __builtin_amdgcn_s_barrier();
  // the loop's read order, so the wait counts at the loop head are the
  // same whether it is entered from here or from the last step of a trip
  static_for<CA>([&](auto C) {
    static_for<NJ>([&](auto J) {
      constexpr int q = decltype(C)::value * NJ + decltype(J)::value;
      read_b(std::integral_constant<int, 0>{}, C, J);
      if constexpr (q < MI)
        read_a(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, q>{});
      __builtin_amdgcn_sched_barrier(0);
    });
  });

  // S steps per trip (the stage of each step is a constant); the launcher
  // guarantees nk % S == 0 and K % 64 == 0
  for (int ks0 = 0; ks0 < nk; ks0 += S) {
    static_for<S>([&](auto H) { step(H, ks0 + decltype(H)::value); });
  }
  // the loads issued for steps past K land before the workgroup ends
  wait_vmcnt<0>();

  if (split >= 0 &&
      !split_exchange<RCAP, MI, NJ>(g, e, acc, static_cast<int64_t>(wu.split_tile) * NW + wave, split))
    return;
  register_epilogue<RCAP, MI, NJ>(g, e, c_act, acc, rw0, cw0, m_lim, n_lim, cs);
}

template <int RCAP, int NW>
__global__ __launch_bounds__(64 * NW) void lds_kernel(const GemmArgsK<RCAP> args) {
  constexpr int STAGE = (kLdsBM / 16 + RCAP * (kLdsBN / 16)) * 1024;
  KArgs<RCAP> &g = kernel_args<GemmArgsK<RCAP>>();
  prefetch_kernel_args<kGemmArgBytes<RCAP>>();
  __shared__ __attribute__((aligned(1024))) int8_t smem[kLdsStages * STAGE];
  __shared__ int64_t red[NW];
  __shared__ int bcast;
  const int c_act = active_channels<RCAP>(g, red, &bcast, 64 * NW);
  const WorkUnit wu = work_of(g);
  if constexpr (RCAP == 4) {
    if (c_act == RCAP - 1) {
      lds_body<RCAP, NW, RCAP - 1>(g, smem, RCAP - 1, wu);
      return;
    }
  }
  lds_body<RCAP, NW, RCAP>(g, smem, c_act, wu);  // every channel computed, the prefix's used
}

// ---------------------------------------------------------------------------
// Wide LDS-staged GEMM: 256 x 96 tiles, 4 channels, 8 waves (4 x 2, each
// 64 x 48 x 4 channels: 192 accumulator registers), four 40 KB stages (all
// of the CU's 160 KB of LDS).  Against the 256 x 64 tile it stages 25 %
// fewer bytes per MFMA, and its tile count fits the chip better on the
// OPT-6.7B projection: N = 12288 is 128 tiles wide, so M = 512 is exactly
// one round of 256 workgroups (the 64-column tile needs 1.5 rounds) and
// M = 2048 four rounds (against six).
//
// The register file holds the accumulators only with single-buffered
// fragments, so the schedule differs from lds_kernel's:
//  * the B fragments of one channel are read while the MFMAs of the
//    channel before run (two buffers of NJ fragments, alternating), and
//    those of the next step's first channel during the last channel;
//  * the A fragments of the next step are read one by one during the last
//    channel's MFMAs, each right after the last MFMA that uses it (that
//    channel runs row by row);
//  * A pairs of K steps are loaded at even steps, two steps ahead, into the
//    stage pair of the previous two steps: every wave has finished those
//    steps' MFMAs (and so their fragment reads) at the barrier that starts
//    the step, so no wave waits for its LDS reads before a barrier.  B is
//    loaded three steps ahead as before.  Per step a wave waits only for
//    the loads that the next step needs (vmcnt BU: the last step's B loads
//    may stay in flight).
// CA: channels computed (the adaptive prefix, fixed per launch: the MFMAs
// and fragment reads of channels past it are not issued at all; their B
// loads re-read channel 0's plane so every wave issues the same loads).
// ---------------------------------------------------------------------------
constexpr int kLdsWBN = 96;

template <int RCAP, int CA>
__device__ __forceinline__ void lds_wide_body(KArgs<RCAP> &g, int8_t *smem, const int c_act, const WorkUnit wu) {
  static_assert(RCAP == 4 && CA >= 1 && CA <= RCAP, "4-channel capacity");
  constexpr int NW = 8, S = kLdsStages, BN = kLdsWBN;
  constexpr int AF = kLdsBM / 16;             // A fragments per stage
  constexpr int NB = BN / 16;                 // column blocks of the tile
  constexpr int BF = RCAP * NB;               // B fragments per stage
  constexpr int ASTAGE = AF * 1024, BSTAGE = BF * 1024;
  constexpr int BAREA = S * ASTAGE;           // the B stages follow the four A stages
  constexpr int WN = 2, WM = NW / WN;         // wave grid
  constexpr int MI = AF / WM, NJ = NB / WN;   // a wave's fragments: 4 x 3
  constexpr int BU = BF / NW;                 // B loads per wave per step
  constexpr int ABLK = kLdsBM / 8;            // A blocks (8 rows x 128 bytes) per pair of steps
  constexpr int AU2 = ABLK / NW;              // A loads per wave per pair
  static_assert(BF % NW == 0 && ABLK % NW == 0 && 16 % NW == 0 && ABLK == 2 * AF, "loads split evenly");
  static_assert(S == 4, "A pairs alternate between the two stage pairs");
  // LDS read offsets are 16-bit immediates: the A area (64 KB) is addressed
  // from one base per step parity, the B area from one base per stage pair
  static_assert(S * ASTAGE <= 65536 && 2 * BSTAGE <= 65536, "immediate read offsets");

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int mt = wu.mt, nt = wu.nt, split = wu.split;
  const int m0 = mt * kLdsBM, n0 = nt * BN;
  const KRange kr = k_range(g, split);
  const int nk = kr.nk;  // a multiple of S (the launcher sizes kchunk so)

  // A: block b = wave + NW u of a pair of steps (e, e + 1) lands in A stage
  // e % S + b / 16, slot b % 16; its 16-byte chunk s holds row 8 b + (s >> 3),
  // bytes 16 ((s & 7) ^ (s >> 3)) of the row's 128-byte segment (as lds_kernel).
  uint32_t aoff[AU2];
  static_for<AU2>([&](auto U) {
    constexpr int u = decltype(U)::value;
    const int row = min(m0 + (wave + NW * u) * 8 + (lane >> 3), g.m - 1);
    aoff[u] = static_cast<uint32_t>(row * g.a_ld + ((lane & 7) ^ (lane >> 3)) * 16);
  });
  // B: fragment q = wave + NW u is channel q / NB, column block q % NB
  // (clamped to the last), one contiguous 1 KB per K step
  const int8_t *bbase[BU];
  const int nblk = (g.n + 15) >> 4;
  static_for<BU>([&](auto U) {
    constexpr int u = decltype(U)::value;
    const int q = wave + NW * u, c = q / NB;
    const int jb = min((n0 >> 4) + q % NB, nblk - 1);
    bbase[u] = g.b + plane_off(c, c_act, g.b_cs) + static_cast<int64_t>(jb) * g.b_ld + kr.ks0 * 1024;
  });
  const uint32_t boff = static_cast<uint32_t>(lane * 16);
  const int8_t *abase = g.a + kr.ks0 * 64;
  const uint32_t sbase = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int8_t *)(smem))) +
      wave * 1024);
  auto dma_b = [&](auto ST, auto L, int ks) {
    constexpr int st = decltype(ST)::value, l = decltype(L)::value;
    const int kc = min(ks, nk - 1);
    lds_dma16<BAREA + st * BSTAGE + NW * l * 1024>(bbase[l] + static_cast<int64_t>(kc) * 1024, boff, sbase);
  };
  auto dma_a = [&](auto ST, auto U, int ks) {  // ks: the pair's first step (even)
    constexpr int st = decltype(ST)::value, u = decltype(U)::value;
    const int kc = min(ks, nk - 2);
    lds_dma16<(st + (NW * u) / 16) * ASTAGE + ((NW * u) % 16) * 1024>(abase + kc * 64, aoff[u], sbase);
  };

  // fragment reads
  i32x4 fa[MI], fb[2][NJ];
  const int f0 = wm * MI;
  const int8_t *rabase[2];
  static_for<2>([&](auto P) {
    constexpr int p = decltype(P)::value;
    rabase[p] = smem + ((2 * f0) / 16) * ASTAGE + ((2 * f0) % 16) * 1024 + ((lane >> 3) & 1) * 1024 +
                ((lane & 7) * 8 + ((4 * p + (lane >> 4)) ^ (lane & 7))) * 16;
  });
  const int8_t *rbbase[2];
  static_for<2>([&](auto P) {
    rbbase[decltype(P)::value] = smem + BAREA + decltype(P)::value * 2 * BSTAGE + wn * NJ * 1024 + lane * 16;
  });
  auto read_a = [&](auto H, auto I) {  // A fragment i of the step at stage h
    constexpr int h = decltype(H)::value, i = decltype(I)::value;
    fa[i] = *reinterpret_cast<const i32x4 *>(rabase[h & 1] + (h & ~1) * ASTAGE + 2 * i * 1024);
  };
  auto read_b = [&](auto H, auto C, auto BUF, auto J) {
    constexpr int h = decltype(H)::value, c = decltype(C)::value, buf = decltype(BUF)::value,
                  j = decltype(J)::value;
    fb[buf][j] = *reinterpret_cast<const i32x4 *>(rbbase[h >> 1] + (h & 1) * BSTAGE + (c * NB + j) * 1024);
  };

  i32x4 acc[RCAP][MI][NJ];
  static_for<RCAP>([&](auto C) {
    static_for<MI>([&](auto I) {
      static_for<NJ>([&](auto J) {
        if constexpr (decltype(C)::value < CA)
          acc[C][I][J] = acc_zero();
        else
          acc[C][I][J] = i32x4{0, 0, 0, 0};
      });
    });
  });

  // one K step k at stage h: own loads of step k + 1 landed, then
  // everyone's (and everyone is done with step k - 1); this step's loads
  // (even steps: the A pair k + 2, k + 3 first, then B of step k + 3; odd
  // steps: B of step k + 3), spread over the (channel, row) groups; the
  // MFMAs channel by channel with the next fragments read between them
  auto step = [&](auto H, int k) {
    constexpr int h = decltype(H)::value, nxt = (h + 1) % S;
    constexpr int nl = (h & 1) ? BU : AU2 + BU;
    constexpr int slots = CA * MI;
    wait_vmcnt<BU>();
    __builtin_amdgcn_s_barrier();
    static_for<CA>([&](auto C) {
      constexpr int c = decltype(C)::value;
      constexpr int buf = (h * CA + c) & 1;
      // the next channel's B fragments (the next step's first channel)
      static_for<NJ>([&](auto J) {
        if constexpr (c + 1 < CA)
          read_b(std::integral_constant<int, h>{}, std::integral_constant<int, c + 1>{},
                 std::integral_constant<int, buf ^ 1>{}, J);
        else
          read_b(std::integral_constant<int, nxt>{}, std::integral_constant<int, 0>{},
                 std::integral_constant<int, buf ^ 1>{}, J);
      });
      static_for<MI>([&](auto I) {
        constexpr int i = decltype(I)::value, slot = c * MI + i;
        static_for<nl>([&](auto L) {
          constexpr int l = decltype(L)::value;
          if constexpr ((l * slots) / nl == slot) {
            if constexpr (!(h & 1) && l < AU2)
              dma_a(std::integral_constant<int, (h + 2) % S>{}, std::integral_constant<int, l>{}, k + 2);
            else
              dma_b(std::integral_constant<int, (h + S - 1) % S>{},
                    std::integral_constant<int, (h & 1) ? l : l - AU2>{}, k + S - 1);
          }
        });
        static_for<NJ>([&](auto J) {
          constexpr int j = decltype(J)::value;
          acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[buf][j], acc[c][i][j], 0, 0, 0);
        });
        if constexpr (c == CA - 1) read_a(std::integral_constant<int, nxt>{}, I);
        // keep the reads where they are: the scheduler otherwise sinks each
        // one to just before its first use, which exposes its latency
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  };

  // prologue: the A pair (0, 1) and B of steps 0 .. 2 in flight
  static_for<AU2>([&](auto U) { dma_a(std::integral_constant<int, 0>{}, U, 0); });
  static_for<BU>([&](auto L) { dma_b(std::integral_constant<int, 0>{}, L, 0); });
  static_for<BU>([&](auto L) { dma_b(std::integral_constant<int, 1>{}, L, 1); });
  static_for<BU>([&](auto L) { dma_b(std::integral_constant<int, 2>{}, L, 2); });
  Epi<RCAP> e;
  load_epi<RCAP>(g, e, c_act);
  pin_epi<RCAP>(e);
  int m_lim = g.m, n_lim = g.n;
  pin_sgpr(m_lim);
  pin_sgpr(n_lim);
  const int rw0 = m0 + wm * (MI * 16), cw0 = n0 + wn * (NJ * 16);
  ColScale cs[NJ];
  static_for<NJ>([&](auto J) { cs[J] = col_scale<RCAP>(e, cw0 + decltype(J)::value * 16 + (lane & 15), n_lim); });
  // step 0 landed (the column factors, when loaded, were issued after the
  // loads and are waited for too)
  wait_vmcnt<2 * BU>();
  __builtin_amdgcn_s_barrier();
  static_for<MI>([&](auto I) { read_a(std::integral_constant<int, 0>{}, I); });
  static_for<NJ>([&](auto J) {
    read_b(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, J);
  });
  __builtin_amdgcn_sched_barrier(0);

  for (int ks0 = 0; ks0 < nk; ks0 += S) {
    static_for<S>([&](auto H) { step(H, ks0 + decltype(H)::value); });
  }
  // the loads issued for steps past K land before the workgroup ends
  wait_vmcnt<0>();

  if (split >= 0 &&
      !split_exchange<RCAP, MI, NJ>(g, e, acc, static_cast<int64_t>(wu.split_tile) * NW + wave, split))
    return;
  register_epilogue<RCAP, MI, NJ>(g, e, c_act, acc, rw0, cw0, m_lim, n_lim, cs);
}

template <int RCAP>
__global__ __launch_bounds__(512) void lds_wide_kernel(const GemmArgsK<RCAP> args) {
  static_assert(RCAP == 4, "the 256 x 96 x 4 tile");
  constexpr int ASTAGE = (kLdsBM / 16) * 1024, BSTAGE = RCAP * (kLdsWBN / 16) * 1024;
  KArgs<RCAP> &g = kernel_args<GemmArgsK<RCAP>>();
  prefetch_kernel_args<kGemmArgBytes<RCAP>>();
  __shared__ __attribute__((aligned(1024))) int8_t smem[kLdsStages * (ASTAGE + BSTAGE)];
  // the adaptive check's reduction slots use the last B stage: the loads of
  // step 0 first write it, after two barriers that every wave reaches only
  // after it has read the broadcast channel count
  int8_t *spare = smem + kLdsStages * ASTAGE + (kLdsStages - 1) * BSTAGE;
  const int c_act = active_channels<RCAP>(g, reinterpret_cast<int64_t *>(spare), reinterpret_cast<int *>(spare + 64),
                                          512);
  const WorkUnit wu = work_of(g);
  if (c_act == RCAP)
    lds_wide_body<RCAP, RCAP>(g, smem, RCAP, wu);
  else if (c_act == RCAP - 1)
    lds_wide_body<RCAP, RCAP - 1>(g, smem, RCAP - 1, wu);
  else
    lds_wide_body<RCAP, RCAP>(g, smem, c_act, wu);  // every channel computed, the prefix's used
}

// ---------------------------------------------------------------------------
// LDS-staged GEMM for residue-plane activations (int16 / int32 inputs, each
// channel its own A plane), 128 x 128 tiles, 4 or 6 channels.  With raw
// int8 A one staged A tile serves every channel; here each channel has its
// own A, so the staging unit is one channel over a pair of K steps: A (128
// rows x 128 bytes, loaded as whole row segments and XOR-swizzled as in
// lds_kernel) and B (8 column blocks x 2 steps of 1 KB), 32 KB.  Four such
// slots (128 KB) form the ring; a trip runs lcm(R, 4) units (R = 6: two
// pairs of K steps, 12 units), so every unit's slot and channel are
// constants in the unrolled trip.  8 waves (2 x 4), each 64 x 32 x R
// channels: 32 R accumulator registers (192 at R = 6), fragments single-
// buffered as in lds_wide_kernel.  Per unit t, slot t % 4:
//  * wait for the own loads of unit t + 1, barrier (everyone's have landed
//    and everyone is done with unit t - 1), then the loads of unit t + 3
//    into the slot of unit t - 1, spread over the MFMAs;
//  * step 0 of the pair row by row, each A fragment of step 1 read right
//    after the last MFMA that uses its register; then the next unit's step-0
//    B fragments; step 1, each of the next unit's step-0 A fragments read
//    after its row; then the next unit's step-1 B fragments.
// A wave's LDS reads per MFMA are those of a 64 x 32 tile (6 KB per 8
// MFMAs, against 16 KB per 48 with raw int8 A): this kernel is bound by LDS
// bandwidth and the MFMAs together, not by HBM or L2.
// PK (packed weights): each channel takes two units per pair of K steps,
// (a' planes, hi plane) then (a planes, lo plane), both accumulating into
// the channel's sums (a' x hi + a x lo, as mfma_packed_kernel), so a trip is
// lcm(2 R, 4) units; the row terms are added once before the epilogue.
// ---------------------------------------------------------------------------
constexpr int kPlBM = 128, kPlBN = 128;

template <int RCAP, bool PK>
__device__ __forceinline__ void lds_planes_body(KArgs<RCAP> &g, int8_t *smem, const int c_act, const WorkUnit wu) {
  static_assert(RCAP == 4 || RCAP == 6, "32 R accumulator registers");
  // (four waves of 64 x 64, one per SIMD with 512 registers, read 25 % fewer
  // LDS bytes per MFMA, but the compiler then moves the 384 accumulators
  // between register files and scratch memory inside the loop)
  constexpr int NW = 8, S = 4, WN = NW / 2, MI = 4, NJ = 8 / WN;
  constexpr int DU = 16 / NW, LU = 2 * DU;       // A (and B) loads per wave per unit; all loads
  constexpr int UA = 16 * 1024, UB = 16 * 1024;  // A and B parts of one unit
  constexpr int BAREA = S * UA;                  // the A parts of all slots, then the B parts
  constexpr int VC = PK ? 2 * RCAP : RCAP;       // units per pair of K steps
  constexpr int TRIP = VC % S == 0 ? VC : (VC % 2 == 0 ? 2 * VC : 4 * VC);  // lcm(VC, S) units
  constexpr int PAIRS = TRIP / VC;               // pairs of K steps per trip

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = wu.mt * kPlBM, n0 = wu.nt * kPlBN;
  const KRange kr = k_range(g, wu.split);
  const int npairs = kr.nk >> 1;  // a multiple of PAIRS (the launcher requires K % 256 == 0)

  // A block b = wave + NW u (rows 8 b .. 8 b + 7 of the tile): lane l loads
  // row 8 b + (l >> 3), bytes 16 ((l & 7) ^ (l >> 3)) of the pair's 128-byte
  // row segment, into chunk l of the block.
  uint32_t aoff[DU];
  static_for<DU>([&](auto U) {
    constexpr int u = decltype(U)::value;
    const int row = min(m0 + (wave + NW * u) * 8 + (lane >> 3), g.m - 1);
    aoff[u] = static_cast<uint32_t>(row * g.a_ld + ((lane & 7) ^ (lane >> 3)) * 16);
  });
  // B fragment f = wave + NW u: step f / 8 = (NW u) / 8 of the pair, column
  // block f % 8 = wave + (NW u) % 8 (clamped to the last), 1 KB contiguous
  const int nblk = (g.n + 15) >> 4;
  const int8_t *bcol[DU];
  static_for<DU>([&](auto U) {
    constexpr int u = decltype(U)::value;
    bcol[u] = g.b + static_cast<int64_t>(min((n0 >> 4) + wave + (NW * u) % 8, nblk - 1)) * g.b_ld + kr.ks0 * 1024;
  });
  const int8_t *acol = g.a + kr.ks0 * 64;
  // the planes of unit v of a pair: channel v (or, packed, channel v / 2
  // with (a', hi) for even v and (a, lo) for odd v)
  int64_t aplane[VC], bplane[VC];
  static_for<VC>([&](auto V) {
    constexpr int v = decltype(V)::value;
    if constexpr (PK) {
      aplane[v] = packed_plane_off<RCAP>(v % 2 == 0 ? RCAP + v / 2 : v / 2, c_act, g.mods.channels, g.a_cs);
      bplane[v] = (v % 2) * g.b_cs;
    } else {
      aplane[v] = plane_off(v, c_act, g.a_cs);
      bplane[v] = plane_off(v, c_act, g.b_cs);
    }
  });
  const uint32_t boff = static_cast<uint32_t>(lane * 16);
  const uint32_t sbase = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int8_t *)(smem))) +
      wave * 1024);
  // load L (A blocks for L < DU, then B fragments) of unit (pair e,
  // channel c) into slot sl; pairs past K load the last pair again into a
  // slot never read
  auto dma = [&](auto SL, auto C, auto L, int e) {
    constexpr int sl = decltype(SL)::value, c = decltype(C)::value, l = decltype(L)::value;
    const int ec = min(e, npairs - 1);
    if constexpr (l < DU) {
      lds_dma16<sl * UA + NW * l * 1024>(acol + aplane[c] + ec * 128, aoff[l], sbase);
    } else {
      constexpr int u = l - DU, step = (NW * u) / 8;
      lds_dma16<BAREA + sl * UB + NW * u * 1024>(bcol[u] + bplane[c] + static_cast<int64_t>(2 * ec + step) * 1024,
                                                boff, sbase);
    }
  };

  // fragment reads: A fragment i of step p at slot sl (rows 16 (4 wm + i) +
  // (lane & 15): block 2 (4 wm + i) + ((lane >> 3) & 1), chunk 4 p + (lane >>
  // 4) of row lane & 7); B fragment j of step s (column block 2 wn + j)
  i32x4 fa[MI], fb[2][NJ];
  const int8_t *rabase[2];
  static_for<2>([&](auto P) {
    constexpr int p = decltype(P)::value;
    rabase[p] = smem + (2 * MI * wm) * 1024 + ((lane >> 3) & 1) * 1024 +
                ((lane & 7) * 8 + ((4 * p + (lane >> 4)) ^ (lane & 7))) * 16;
  });
  const int8_t *rbbase = smem + BAREA + wn * NJ * 1024 + lane * 16;
  auto read_a = [&](auto SL, auto P, auto I) {
    constexpr int sl = decltype(SL)::value, p = decltype(P)::value, i = decltype(I)::value;
    fa[i] = *reinterpret_cast<const i32x4 *>(rabase[p] + sl * UA + 2 * i * 1024);
  };
  auto read_b = [&](auto SL, auto ST, auto J) {
    constexpr int sl = decltype(SL)::value, st = decltype(ST)::value, j = decltype(J)::value;
    fb[st][j] = *reinterpret_cast<const i32x4 *>(rbbase + sl * UB + (st * 8 + j) * 1024);
  };

  i32x4 acc[RCAP][MI][NJ];
  static_for<RCAP>([&](auto C) {
    static_for<MI>([&](auto I) { static_for<NJ>([&](auto J) { acc[C][I][J] = acc_zero(); }); });
  });

  // unit t of the trip starting at pair e0
  auto unit = [&](auto T, int e0) {
    constexpr int t = decltype(T)::value, sl = t % S, c = PK ? (t % VC) / 2 : t % VC, nsl = (t + 1) % S;
    constexpr int t3 = t + 3, sl3 = t3 % S, c3 = t3 % VC, pe3 = t3 / VC;
    wait_vmcnt<LU>();
    __builtin_amdgcn_s_barrier();
    static_for<2>([&](auto ST) {
      constexpr int st = decltype(ST)::value;
      static_for<MI>([&](auto I) {
        constexpr int i = decltype(I)::value, grp = st * MI + i;
        // the LU loads of unit t + 3, spread over the 8 row groups
        static_for<LU>([&](auto L) {
          if constexpr ((decltype(L)::value * 2 * MI) / LU == grp)
            dma(std::integral_constant<int, sl3>{}, std::integral_constant<int, c3>{}, L, e0 + pe3);
        });
        static_for<NJ>([&](auto J) {
          constexpr int j = decltype(J)::value;
          acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[st][j], acc[c][i][j], 0, 0, 0);
        });
        // the read below reuses fa[i]'s register only if it stays after
        // the MFMAs that consume the old value
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (st == 0)
          read_a(std::integral_constant<int, sl>{}, std::integral_constant<int, 1>{}, I);
        else
          read_a(std::integral_constant<int, nsl>{}, std::integral_constant<int, 0>{}, I);
        __builtin_amdgcn_sched_barrier(0);
      });
      static_for<NJ>([&](auto J) { read_b(std::integral_constant<int, nsl>{}, ST, J); });
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // prologue: units 0, 1, 2 in flight
  static_for<3>([&](auto T) {
    constexpr int t = decltype(T)::value;
    static_for<LU>([&](auto L) {
      dma(std::integral_constant<int, t % S>{}, std::integral_constant<int, t % VC>{}, L, t / VC);
    });
  });
  // unit 0 landed
  wait_vmcnt<2 * LU>();
  __builtin_amdgcn_s_barrier();
  static_for<MI>([&](auto I) { read_a(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, I); });
  static_for<2>([&](auto ST) {
    static_for<NJ>([&](auto J) { read_b(std::integral_constant<int, 0>{}, ST, J); });
  });
  __builtin_amdgcn_sched_barrier(0);

  for (int e0 = 0; e0 < npairs; e0 += PAIRS) {
    static_for<TRIP>([&](auto T) { unit(T, e0); });
  }
  // the loads issued for units past K land before the workgroup ends
  wait_vmcnt<0>();
  const int rw0 = m0 + wm * (MI * 16), cw0 = n0 + wn * (NJ * 16);
  if constexpr (PK) {
    if (wu.split <= 0) add_packed_rows<RCAP, MI, NJ>(g, acc, rw0, c_act);
  }
  // The epilogue's constants and column factors are read only now: with
  // 6 channels they would hold some 110 scalar registers (and the column
  // factors 4 vector registers) through the loop, which the accumulators
  // leave no room for.  The scalar ones hit the constant cache (the
  // argument block was read at entry).
  Epi<RCAP> e;
  load_epi<RCAP>(g, e, c_act);
  const int m_lim = g.m, n_lim = g.n;
  if (wu.split >= 0 &&
      !split_exchange<RCAP, MI, NJ>(g, e, acc, static_cast<int64_t>(wu.split_tile) * NW + wave, wu.split))
    return;
  ColScale cs[NJ];
  static_for<NJ>([&](auto J) { cs[J] = col_scale<RCAP>(e, cw0 + decltype(J)::value * 16 + (lane & 15), n_lim); });
  register_epilogue<RCAP, MI, NJ>(g, e, c_act, acc, rw0, cw0, m_lim, n_lim, cs);
}

// Work unit of workgroup blockIdx.x for the residue-plane kernel.  Tile t
// maps to (mt, nt) in groups of 4 row tiles: t walks the 4 rows of one
// column tile, then the next column.  With each XCD's contiguous run of
// units (xcd_order) a round of 32 workgroups on one XCD reads 4 A row tiles
// and 8 B column tiles (12 x 3 MB over K at 6 channels) instead of, M-block
// fastest at M = 2048, 16 and 2 (18): each A row tile is as large as a B
// column tile here.  Tail split (as work_of): workgroups [0, split_from)
// take the whole tiles; the others take (tile, split) units split-minor,
// so both halves of a tile run on one XCD and exchange through its L2.
template <typename G>
__device__ __forceinline__ WorkUnit planes_work(G &g) {
  constexpr int RG = 4;
  const int tiles_m = g.tiles_m, tiles_n = g.tiles_n, whole = g.split_from;
  const int b = blockIdx.x;
  WorkUnit w{0, 0, -1, 0};
  int t;
  if (b < whole) {
    t = xcd_order(b, whole);
  } else {
    const int u = xcd_order(b - whole, (tiles_m * tiles_n - whole) * g.splits);
    w.split = u % g.splits;
    t = whole + u / g.splits;
  }
  w.split_tile = t - whole;
  const int grouped = tiles_m / RG * RG;  // rows in full groups
  if (t < grouped * tiles_n) {
    const int r = t % (RG * tiles_n);
    w.nt = r / RG;
    w.mt = t / (RG * tiles_n) * RG + r % RG;
  } else {
    const int r = t - grouped * tiles_n, h = tiles_m - grouped;
    w.nt = r / h;
    w.mt = grouped + r % h;
  }
  return w;
}

template <int RCAP, bool PK>
__global__ __launch_bounds__(512) void lds_planes_kernel(const GemmArgsK<RCAP> args) {
  constexpr int SLOTS = kLdsStages * 32 * 1024;
  KArgs<RCAP> &g = kernel_args<GemmArgsK<RCAP>>();
  prefetch_kernel_args<kGemmArgBytes<RCAP>>();
  __shared__ __attribute__((aligned(1024))) int8_t smem[SLOTS];
  // the adaptive check's reduction slots use the last slot's B part: the
  // loads of unit 3 first write it, after the barrier of unit 0, which every
  // wave reaches only after it has read the broadcast channel count
  int8_t *spare = smem + SLOTS - 16 * 1024;
  const int c_act = __builtin_amdgcn_readfirstlane(
      active_channels<RCAP>(g, reinterpret_cast<int64_t *>(spare), reinterpret_cast<int *>(spare + 64), 512));
  lds_planes_body<RCAP, PK>(g, smem, c_act, planes_work(g));
}

// ---------------------------------------------------------------------------
// Launchers for one channel capacity (instantiated per translation unit).
// ---------------------------------------------------------------------------
template <int RCAP, bool ARAW>
bool launch_stream(GemmArgsK<RCAP> g, int mb, int nb, int ks, int ucap, hipStream_t st) {
#define RNSMX_STREAM(MB_, NB_, UCAP_)                                                        \
  if (mb == MB_ && nb == NB_ && ucap == UCAP_) {                                            \
    g.tiles_m = (g.m + 16 * MB_ - 1) / (16 * MB_);                                          \
    g.tiles_n = (g.n + 16 * NB_ - 1) / (16 * NB_);                                          \
    const dim3 grid(static_cast<unsigned>(g.split_from + (g.tiles_m * g.tiles_n - g.split_from) * g.splits));               \
    const size_t lds = ks > 1 ? static_cast<size_t>(RCAP) * 256 * MB_ * NB_ * 4 : 0;         \
    g.threads = 64 * ks;                                                                    \
    hipLaunchKernelGGL((stream_kernel<RCAP, MB_, NB_, ARAW, UCAP_>), grid, dim3(64 * ks), lds, st, g); \
    return true;                                                                            \
  }
  RNSMX_STREAM(1, 1, 4)
  RNSMX_STREAM(2, 1, 4)
  if constexpr (RCAP <= 4) {
    RNSMX_STREAM(4, 1, 4)
    RNSMX_STREAM(1, 2, 4)
    RNSMX_STREAM(1, 1, 8)
  }
#undef RNSMX_STREAM
  return false;
}

// p_req: ring depth (K steps of A and B loads in flight), 0 = the tile's
// default.  Deeper rings than 3-4 steps cost occupancy (registers) and
// measured slower on every shape tried, also where a workgroup per CU
// leaves one wave per SIMD anyway (C2 M=256 with 64 x 64 tiles: ring of 12,
// i.e. all of K = 768 in flight, 12.1 us against 11.0 us with 3).  NBSEL: the tile widths this
// instantiation covers (0 all, 1 or 2 only NB = NBSEL).
template <int RCAP, bool ARAW, int NBSEL>
bool launch_mfma(GemmArgsK<RCAP> g, int mb, int nb, int p_req, int nwv, hipStream_t st) {
#define RNSMX_MFMA_P(MB_, NB_, P_)                                                               \
  if (p == P_ && nwv == 4) {                                                                     \
    if constexpr (!ARAW) {                                                                       \
      if (g.tiles_m == 1) {                                                                      \
        hipLaunchKernelGGL((mfma_kernel<RCAP, MB_, NB_, P_, ARAW, 4, true>), grid, dim3(256), 0, st, g); \
        return true;                                                                             \
      }                                                                                          \
    }                                                                                            \
    hipLaunchKernelGGL((mfma_kernel<RCAP, MB_, NB_, P_, ARAW>), grid, dim3(256), 0, st, g);      \
    return true;                                                                                 \
  }
#define RNSMX_MFMA_P3(MB_, NB_, P_)                                                              \
  if constexpr (ARAW) {                                                                          \
    if (p == P_ && nwv == 3) {                                                                   \
      hipLaunchKernelGGL((mfma_kernel<RCAP, MB_, NB_, P_, ARAW, 3>), grid, dim3(192), 0, st, g); \
      return true;                                                                               \
    }                                                                                            \
  }
#define RNSMX_MFMA(MB_, NB_, PDEF, ...)                                    \
  if constexpr (NBSEL == 0 || NBSEL == NB_) {                              \
    if (mb == MB_ && nb == NB_) {                                          \
      g.tiles_m = (g.m + 16 * MB_ - 1) / (16 * MB_);                       \
      g.tiles_n = (g.n + 16 * nwv * NB_ - 1) / (16 * nwv * NB_);           \
      const dim3 grid(static_cast<unsigned>(g.split_from + (g.tiles_m * g.tiles_n - g.split_from) * g.splits)); \
      const int p = p_req > 0 ? p_req : PDEF;                              \
      __VA_ARGS__                                                          \
      return false;                                                        \
    }                                                                      \
  }
  if constexpr (RCAP <= 4) {
    RNSMX_MFMA(2, 1, 3, RNSMX_MFMA_P(2, 1, 3) RNSMX_MFMA_P(2, 1, 4) RNSMX_MFMA_P3(2, 1, 4))
    RNSMX_MFMA(4, 1, 3, RNSMX_MFMA_P(4, 1, 3) RNSMX_MFMA_P(4, 1, 4) RNSMX_MFMA_P3(4, 1, 3) RNSMX_MFMA_P3(4, 1, 4))
    RNSMX_MFMA(3, 1, 3, RNSMX_MFMA_P(3, 1, 3) RNSMX_MFMA_P(3, 1, 4) RNSMX_MFMA_P3(3, 1, 4))
    RNSMX_MFMA(2, 2, 3, RNSMX_MFMA_P(2, 2, 3) RNSMX_MFMA_P(2, 2, 4))
    RNSMX_MFMA(4, 2, 3, RNSMX_MFMA_P(4, 2, 3) RNSMX_MFMA_P(4, 2, 4))
    RNSMX_MFMA(8, 2, 3, RNSMX_MFMA_P(8, 2, 3) RNSMX_MFMA_P(8, 2, 4))
  } else if constexpr (RCAP == 6) {
    RNSMX_MFMA(2, 1, 3, RNSMX_MFMA_P(2, 1, 3) RNSMX_MFMA_P(2, 1, 4))
    RNSMX_MFMA(4, 1, 3, RNSMX_MFMA_P(4, 1, 3) RNSMX_MFMA_P(4, 1, 4))
    RNSMX_MFMA(4, 2, 3, RNSMX_MFMA_P(4, 2, 3))
  } else {  // registers allow no more
    RNSMX_MFMA(2, 1, 3, RNSMX_MFMA_P(2, 1, 3))
    RNSMX_MFMA(4, 1, 3, RNSMX_MFMA_P(4, 1, 3))
    RNSMX_MFMA(2, 2, 2, RNSMX_MFMA_P(2, 2, 2))
  }
#undef RNSMX_MFMA
#undef RNSMX_MFMA_P
#undef RNSMX_MFMA_P3
  return false;
}

// The LDS-staged kernel: raw int8 A below 4 GB, K a multiple of 256 (whole
// trips of four 64-byte steps), 4-channel capacity (16 B fragments per stage
// split over 8 waves).
inline bool lds_kernel_fits(const GemmArgs &g, bool araw, int rcap) {
  // the A loads address rows through a 32-bit per-lane offset from A's base
  const bool a_offsets_fit = static_cast<int64_t>(g.m) * g.a_ld < (int64_t{1} << 32) - 256;
  return araw && rcap == 4 && g.a_k == g.kp && g.kp % (64 * kLdsStages) == 0 && a_offsets_fit;
}

// Tiles, waves per workgroup and accumulator chunks per lane of a choice
// for an m x n output (the launchers derive the same tile grid).
inline GemmGrid gemm_grid(const GemmChoice &c, int64_t m, int64_t n) {
  GemmGrid r{};
  auto cdiv = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
  if (c.kind == kStream || c.kind == kStreamWide) {
    r.tiles = cdiv(m, 16 * c.mb) * cdiv(n, 16 * c.nb);
    r.waves = c.ks < 1 ? 1 : c.ks;
    r.chunks = c.mb * c.nb;
  } else if (c.kind == kRows) {
    r.tiles = cdiv(n, 16);
    r.waves = c.ks < 1 ? 1 : c.ks;
    r.chunks = c.mb;
  } else if (c.kind == kLds || c.kind == kLdsWide) {
    const int bn = c.kind == kLds ? kLdsBN : kLdsWBN;
    r.tiles = cdiv(m, kLdsBM) * cdiv(n, bn);
    r.waves = 8;
    r.chunks = (kLdsBM / 16 / 4) * (bn / 16 / 2);
  } else if (c.kind == kLdsPlanes) {
    r.tiles = cdiv(m, kPlBM) * cdiv(n, kPlBN);
    r.waves = 8;
    r.chunks = (kPlBM / 16 / 2) * (kPlBN / 16 / 4);
  } else {
    const int nwv = c.kind == kMfma3 ? 3 : 4;
    r.tiles = cdiv(m, 16 * c.mb) * cdiv(n, 16 * nwv * c.nb);
    r.waves = nwv;
    r.chunks = c.mb * c.nb;
  }
  return r;
}

// The residue-plane LDS kernel: activations as per-channel planes (not raw
// int8), 4 or 6 channels, K a multiple of 256 (whole trips), rows addressed
// through 32-bit per-lane offsets within a plane.
template <typename G>
inline bool lds_planes_fits(const G &g, bool araw, int rcap) {
  const bool a_offsets_fit = static_cast<int64_t>(g.m) * g.a_ld < (int64_t{1} << 32) - 256;
  return !araw && (rcap == 4 || rcap == 6) && g.a_k == g.kp && g.kp % (64 * kLdsStages) == 0 && a_offsets_fit;
}

template <int RCAP>
bool launch_lds(const GemmArgs &host, bool araw, int kind, hipStream_t st) {
  if (kind == kLdsPlanes) {
    if constexpr (RCAP == 4 || RCAP == 6) {
      if (!lds_planes_fits(host, araw, RCAP)) return false;
      GemmArgsK<RCAP> g = compact_args<RCAP>(host);
      g.tiles_m = (g.m + kPlBM - 1) / kPlBM;
      g.tiles_n = (g.n + kPlBN - 1) / kPlBN;
      const dim3 grid(static_cast<unsigned>(g.split_from + (g.tiles_m * g.tiles_n - g.split_from) * g.splits));
      hipLaunchKernelGGL((lds_planes_kernel<RCAP, false>), grid, dim3(512), 0, st, g);
      return true;
    }
    return false;
  }
  const bool wide = kind == kLdsWide;
  if constexpr (RCAP != 4) {
    return false;
  } else {
    if (!lds_kernel_fits(host, araw, RCAP)) return false;
    GemmArgsK<RCAP> g = compact_args<RCAP>(host);
    const int bn = wide ? kLdsWBN : kLdsBN;
    g.tiles_m = (g.m + kLdsBM - 1) / kLdsBM;
    g.tiles_n = (g.n + bn - 1) / bn;
    const dim3 grid(static_cast<unsigned>(g.split_from + (g.tiles_m * g.tiles_n - g.split_from) * g.splits));
    if (wide)
      hipLaunchKernelGGL((lds_wide_kernel<RCAP>), grid, dim3(512), 0, st, g);
    else
      hipLaunchKernelGGL((lds_kernel<RCAP, 8>), grid, dim3(512), 0, st, g);
    return true;
  }
}

// Packed-weight kernels: stream tiles of 16 or 32 rows, MFMA tiles of 32 or
// 64 rows x 64 columns (ring depth 3 or 2: the 2R activation planes double
// the register ring of A chunks), the residue-plane LDS kernel with two
// units per channel; up to 6 channels.  Only the LDS kernel splits K over
// workgroups.
template <int RCAP>
bool launch_packed(GemmArgsK<RCAP> g, const GemmChoice &c, hipStream_t st) {
  if constexpr (RCAP != 4 && RCAP != 6) {
    return false;
  } else {
    if (c.kind == kLdsPlanes) {  // the one packed kernel that may split K
      if (!lds_planes_fits(g, false, RCAP)) return false;
      g.tiles_m = (g.m + kPlBM - 1) / kPlBM;
      g.tiles_n = (g.n + kPlBN - 1) / kPlBN;
      const dim3 grid(static_cast<unsigned>(g.split_from + (g.tiles_m * g.tiles_n - g.split_from) * g.splits));
      hipLaunchKernelGGL((lds_planes_kernel<RCAP, true>), grid, dim3(512), 0, st, g);
      return true;
    }
    if (c.splits > 1) return false;
    if (c.kind == kRows && c.ks >= 1 && c.ks <= 4) {
      g.tiles_m = 1;
      g.tiles_n = (g.n + 15) / 16;
      g.threads = 64 * c.ks;
      const dim3 grid(static_cast<unsigned>(g.tiles_n)), block(64 * c.ks);
      switch (c.mb) {
        case 1: hipLaunchKernelGGL((rows_packed_kernel<RCAP, 1>), grid, block, 0, st, g); return true;
        case 2: hipLaunchKernelGGL((rows_packed_kernel<RCAP, 2>), grid, block, 0, st, g); return true;
        case 4: hipLaunchKernelGGL((rows_packed_kernel<RCAP, 4>), grid, block, 0, st, g); return true;
        case 8: hipLaunchKernelGGL((rows_packed_kernel<RCAP, 8>), grid, block, 0, st, g); return true;
        default: return false;
      }
    }
    if (c.kind == kStream) {
#define RNSMX_STREAM_PK(MB_)                                                                           \
  if (c.mb == MB_ && c.nb == 1) {                                                                     \
    g.tiles_m = (g.m + 16 * MB_ - 1) / (16 * MB_);                                                    \
    g.tiles_n = (g.n + 15) / 16;                                                                      \
    const dim3 grid(static_cast<unsigned>(g.tiles_m * g.tiles_n));                                   \
    const size_t lds = c.ks > 1 ? static_cast<size_t>(RCAP) * 256 * MB_ * 4 : 0;                      \
    g.threads = 64 * c.ks;                                                                            \
    hipLaunchKernelGGL((stream_packed_kernel<RCAP, MB_, 1, 4>), grid, dim3(64 * c.ks), lds, st, g);   \
    return true;                                                                                      \
  }
      RNSMX_STREAM_PK(1)
      RNSMX_STREAM_PK(2)
#undef RNSMX_STREAM_PK
      return false;
    }

    if (c.kind == kMfma && c.nb == 1 && (c.mb == 2 || c.mb == 4)) {
      g.tiles_m = (g.m + 16 * c.mb - 1) / (16 * c.mb);
      g.tiles_n = (g.n + 63) / 64;
      const dim3 grid(static_cast<unsigned>(g.tiles_m * g.tiles_n));
      if (c.mb == 2)
        hipLaunchKernelGGL((mfma_packed_kernel<RCAP, 2, 1, 3>), grid, dim3(256), 0, st, g);
      else
        hipLaunchKernelGGL((mfma_packed_kernel<RCAP, 4, 1, 2>), grid, dim3(256), 0, st, g);
      return true;
    }
    return false;
  }
}

// Body of one part launcher (rnsmx_gemm_part.hip).  PART 5 is chosen only
// for packed weights (gemm_part_of), whatever the activation form.
template <int RCAP, int PART>
bool launch_gemm_part(const GemmArgs &g, bool araw, const GemmChoice &c, hipStream_t st) {
  if constexpr (PART == 5) {
    return launch_packed<RCAP>(compact_args<RCAP>(g), c, st);
  } else if constexpr (PART == 4) {
    return gemm_part_of(c, araw) == PART && launch_lds<RCAP>(g, araw, c.kind, st);
  } else {
    if (gemm_part_of(c, araw) != PART) return false;
    if constexpr (PART == 0) {
      const int ucap = c.kind == kStreamWide ? 8 : 4;
      return araw ? launch_stream<RCAP, true>(compact_args<RCAP>(g), c.mb, c.nb, c.ks, ucap, st)
                  : launch_stream<RCAP, false>(compact_args<RCAP>(g), c.mb, c.nb, c.ks, ucap, st);
    } else {
      const int nwv = c.kind == kMfma3 ? 3 : 4;
      if constexpr (PART == 1 || PART == 2)
        return launch_mfma<RCAP, true, PART>(compact_args<RCAP>(g), c.mb, c.nb, c.ks, nwv, st);
      else
        return launch_mfma<RCAP, false, 0>(compact_args<RCAP>(g), c.mb, c.nb, c.ks, nwv, st);
    }
  }
}

}  // namespace rnsmx
