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
  const int8_t *a;  // [R][M][a_ld] residue planes, or [M][a_ld] int8 (a_cs = 0)
  int64_t a_ld, a_cs;
  const int8_t *b;  // [R][N][b_ld]
  int64_t b_ld, b_cs;
  int32_t m, n, kp;  // kp: multiple of 64, <= b_ld
  int32_t a_k;       // A bytes per row that are read; 16-byte chunks at or past it load as 0
  int32_t tiles_m, tiles_n;  // output tile grid (set at launch)
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
typedef RNSMX_KARG(GemmArgs) KGemmArgs;

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
// L1 norms written by the encoder and max|B| written at weight preparation:
// bound = max_i sum_k |a_ik| * max|B| (adaptive.py:44-52); the answer is the
// smallest c >= min_channels with 2 * bound < prod_{i<c} m_i
// (adaptive.py:15-41), i.e. bound <= (P_c - 1) / 2.  When no prefix fits,
// the full set is used and meta[3] flags the overflow (the reference raises
// OverflowError on the host, which a device-side selector cannot).
template <int RCAP>
__device__ __forceinline__ int active_channels(KGemmArgs &g, int64_t *red, int *bcast) {
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

// Final value of one output element from its mixed-radix digits, centered
// about P_c / 2, written in the requested output type.  The float chain is
// ((float)x * a_scale) * w_scale[col] + bias[col], each step rounded to
// nearest even with no contraction: the op order of rns_linear.py:272-275.
template <int RCAP>
__device__ __forceinline__ void store_element(KGemmArgs &g, int c_act,
                                              const uint32_t (&d)[RCAP], int row,
                                              int col) {
  uint64_t x = 0;
#pragma unroll
  for (int c = 0; c < RCAP; ++c)
    if (c < c_act) x += static_cast<uint64_t>(d[c]) * static_cast<uint64_t>(g.mods.prefix[c]);
  const int64_t p = prefix_at<RCAP>(g.mods, c_act);
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
template <int C, typename Mods, typename DigitAt>
__device__ __forceinline__ uint32_t garner_digit(const Mods &mods, uint32_t r, DigitAt &&digit_at) {
  uint32_t s = r * mods.qinv[C];
#pragma unroll
  for (int j = 0; j < C; ++j) s += digit_at(j) * mods.ucoef[j][C];
  return mod_u32(s, static_cast<uint32_t>(mods.moduli[C]), mods.magic[C]);
}

// ---------------------------------------------------------------------------
// Workgroup -> output tile.  Workgroups are handed to the 8 XCDs round-robin
// (workgroup b runs on XCD b % 8), and each XCD has its own L2.  Tiles are
// numbered M-block fastest, so giving every XCD one contiguous run of tile
// numbers keeps the workgroups that read the same weight columns on the
// same L2.  The map is a bijection on [0, tiles) for any tile count.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void tile_of(int tiles_m, int tiles_n, int &mt, int &nt) {
  const int total = tiles_m * tiles_n;
  const int b = blockIdx.x;
  const int xcd = b & 7, local = b >> 3;
  const int base = total >> 3, rem = total & 7;
  const int t = xcd * base + min(xcd, rem) + local;
  mt = t % tiles_m;
  nt = t / tiles_m;
}

__device__ __forceinline__ i32x4 load16(const int8_t *p) {
  return *reinterpret_cast<const i32x4 *>(p);
}

// Canonical residue of one int32 accumulator of channel c (LUT or Barrett).
__device__ __forceinline__ uint32_t reduce_acc(KGemmArgs &g, int c, int32_t v) {
  const uint32_t m = static_cast<uint32_t>(g.mods.moduli[c]);
  return c < g.lut_channels ? canon_i32_lut(v, g.lut + c * 1024, m, g.mods.c31[c])
                            : canon_i32(v, m, g.mods.magic[c], g.mods.c31[c]);
}

// ---------------------------------------------------------------------------
// Stream GEMM (small and medium M: decode, continuous batches, C2 shapes).
// The bound is HBM latency: the weight residues are read once and the
// problem is a few MB, so every wave issues all the loads of its K slice
// before its first MFMA.  A workgroup owns a (16*MB) x (16*NB) output tile;
// its waves split K (wave w takes K-step chunks w, w + KS, ... of U steps)
// and each wave accumulates every channel.  Channel partial sums are reduced
// mod m_c to canonical bytes in LDS ((sum of partials) mod m = (sum of
// (partial mod m)) mod m), then each thread combines the slices of four
// adjacent outputs, runs Garner and stores them.
//
// ARAW: A is one int8 matrix shared by every channel (an int8 activation is
// its own representative mod every m_c, so the channel-c product of the raw
// activations has the same residue as the product of the centered residues);
// otherwise A holds one centered residue plane per channel.
// ---------------------------------------------------------------------------
// K steps per chunk of the stream kernel: as many as fit next to the
// accumulators in 240 registers (two waves per SIMD), at most 4.
constexpr int stream_u_of(int rcap, bool araw, int mb, int nb) {
  const int frags = (araw ? 1 : rcap) * mb + rcap * nb;  // 16-byte loads per K step
  const int u = (240 - 4 * rcap * mb * nb) / (4 * frags);
  return u < 1 ? 1 : (u > 4 ? 4 : u);
}

template <int RCAP, int MB, int NB, bool ARAW>
struct StreamCfg {
  static constexpr int AP = ARAW ? 1 : RCAP;
  static constexpr int U = stream_u_of(RCAP, ARAW, MB, NB);
  static constexpr int TILE = 16 * MB * 16 * NB;
};

template <int RCAP, int MB, int NB, bool ARAW>
__global__ __launch_bounds__(256) void gemm_stream_kernel(const GemmArgs args) {
  KGemmArgs &g = kernel_args<GemmArgs>();
  using Cfg = StreamCfg<RCAP, MB, NB, ARAW>;
  constexpr int BM = 16 * MB, BN = 16 * NB, TILE = Cfg::TILE, AP = Cfg::AP, U = Cfg::U;
  extern __shared__ __attribute__((aligned(16))) uint8_t sres[];  // [KS][RCAP][TILE]
  __shared__ int64_t red[4];
  __shared__ int bcast;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ks_n = blockDim.x >> 6;
  const int c_act = active_channels<RCAP>(g, red, &bcast);
  int mt, nt;
  tile_of(g.tiles_m, g.tiles_n, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int nk = g.kp >> 6;
  const int kofs = (lane >> 4) * 16;

  const int8_t *ap[MB];
  const int8_t *bp[NB];
  static_for<MB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    const int row = min(m0 + i * 16 + (lane & 15), g.m - 1);
    ap[i] = g.a + static_cast<int64_t>(row) * g.a_ld + kofs;
  });
  static_for<NB>([&](auto J) {
    constexpr int j = decltype(J)::value;
    const int col = min(n0 + j * 16 + (lane & 15), g.n - 1);
    bp[j] = g.b + static_cast<int64_t>(col) * g.b_ld + kofs;
  });

  const i32x4 zero = {0, 0, 0, 0};
  i32x4 acc[RCAP][MB][NB];
  static_for<RCAP>([&](auto C) {
    static_for<MB>([&](auto I) {
      static_for<NB>([&](auto J) { acc[C][I][J] = zero; });
    });
  });

  for (int q = wave * U; q < nk; q += ks_n * U) {
    i32x4 fa[U][AP][MB], fb[U][RCAP][NB];
    static_for<U>([&](auto UU) {
      constexpr int u = decltype(UU)::value;
      const int ks = q + u;
      const bool kv = ks < nk;
      const int ko = ks * 64;
      const bool av = kv && (ko + kofs < g.a_k);
      static_for<AP>([&](auto PP) {
        constexpr int p = decltype(PP)::value;
        static_for<MB>([&](auto I) {
          constexpr int i = decltype(I)::value;
          fa[u][p][i] = (av && p < c_act) ? load16(ap[i] + p * g.a_cs + ko) : zero;
        });
      });
      static_for<RCAP>([&](auto C) {
        constexpr int c = decltype(C)::value;
        static_for<NB>([&](auto J) {
          constexpr int j = decltype(J)::value;
          fb[u][c][j] = (kv && c < c_act) ? load16(bp[j] + c * g.b_cs + ko) : zero;
        });
      });
    });
    static_for<U>([&](auto UU) {
      constexpr int u = decltype(UU)::value;
      static_for<RCAP>([&](auto C) {
        constexpr int c = decltype(C)::value;
        if (c >= c_act) return;
        static_for<MB>([&](auto I) {
          constexpr int i = decltype(I)::value;
          static_for<NB>([&](auto J) {
            constexpr int j = decltype(J)::value;
            acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u][ARAW ? 0 : c][i], fb[u][c][j],
                                                                 acc[c][i][j], 0, 0, 0);
          });
        });
      });
    });
  }

  // this wave's K slice: canonical residues, one byte per (channel, element)
  uint8_t *mine = sres + wave * (RCAP * TILE);
  static_for<RCAP>([&](auto C) {
    constexpr int c = decltype(C)::value;
    if (c >= c_act) return;
    static_for<MB>([&](auto I) {
      constexpr int i = decltype(I)::value;
      static_for<NB>([&](auto J) {
        constexpr int j = decltype(J)::value;
        static_for<4>([&](auto T) {
          constexpr int t = decltype(T)::value;
          mine[c * TILE + (i * 16 + 4 * (lane >> 4) + t) * BN + j * 16 + (lane & 15)] =
              static_cast<uint8_t>(reduce_acc(g, c, acc[c][i][j][t]));
        });
      });
    });
  });
  __syncthreads();

  // combine slices, Garner, store: each thread takes 4 adjacent columns
  const int rows_here = min(BM, g.m - m0);
  for (int e = threadIdx.x * 4; e < rows_here * BN; e += blockDim.x * 4) {
    const int row = e / BN, col = e % BN;
    uint32_t d[4][RCAP];
    static_for<RCAP>([&](auto CC) {
      constexpr int cc = decltype(CC)::value;
      if (cc >= c_act) {
#pragma unroll
        for (int v = 0; v < 4; ++v) d[v][cc] = 0;
        return;
      }
      // byte sums in 16-bit lanes: even bytes and odd bytes of the 4 outputs
      uint32_t lo = 0, hi = 0;
      for (int s = 0; s < ks_n; ++s) {
        const uint32_t w = *reinterpret_cast<const uint32_t *>(sres + s * (RCAP * TILE) + cc * TILE + e);
        lo += w & 0x00FF00FFu;
        hi += (w >> 8) & 0x00FF00FFu;
      }
      const uint32_t sums[4] = {lo & 0xFFFFu, hi & 0xFFFFu, lo >> 16, hi >> 16};
      const uint32_t m = static_cast<uint32_t>(g.mods.moduli[cc]);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t r = mod_u32(sums[v], m, g.mods.magic[cc]);
        d[v][cc] = garner_digit<cc>(g.mods, r, [&](int jj) { return d[v][jj]; });
      }
    });
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (n0 + col + v < g.n) store_element<RCAP>(g, c_act, d[v], m0 + row, n0 + col + v);
  }
}

// ---------------------------------------------------------------------------
// MFMA GEMM (large M: prefill, C4/C5 shapes).  Bound by MFMA throughput, so
// operands are reused from registers and LDS.  A workgroup of 4 waves owns a
// (16*MB) x (4*16*NB) tile: the A rows (shared by all waves, and in ARAW
// mode by all channels) are staged through double-buffered LDS with rows
// padded to 80 bytes (the 16-byte fragment reads of 16 lanes hit disjoint
// banks); each wave owns 16*NB columns and streams their weight residues
// straight from global memory into a P-deep register ring.  Every K step
// feeds all channels, so all channel accumulators finish together and the
// reduction + Garner + store run from registers.
// ---------------------------------------------------------------------------
constexpr int kLdsRow = 80;

template <int RCAP, int MB, int NB, int P, bool ARAW>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const GemmArgs args) {
  KGemmArgs &g = kernel_args<GemmArgs>();
  constexpr int BM = 16 * MB, BNW = 16 * NB;
  constexpr int AP = ARAW ? 1 : RCAP;
  constexpr int PLANE = BM * kLdsRow;
  constexpr int ACH = AP * BM * 4;  // 16-byte A chunks per K step
  constexpr int AC = (ACH + 255) / 256;
  __shared__ __attribute__((aligned(16))) int8_t As[2][AP * PLANE];
  __shared__ int64_t red[4];
  __shared__ int bcast;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c_act = active_channels<RCAP>(g, red, &bcast);
  int mt, nt;
  tile_of(g.tiles_m, g.tiles_n, mt, nt);
  const int m0 = mt * BM, n0 = nt * (4 * BNW) + wave * BNW;
  const int nk = g.kp >> 6;
  const int kofs = (lane >> 4) * 16;

  // A staging: chunk q -> plane p, row, 16-byte part
  const int8_t *asrc[AC];
  int alds[AC], apart[AC];
  bool aon[AC];
  static_for<AC>([&](auto II) {
    constexpr int i = decltype(II)::value;
    const int q = tid + 256 * i;
    aon[i] = q < ACH;
    const int qq = aon[i] ? q : 0;
    const int p = qq / (BM * 4), w = qq % (BM * 4), row = w >> 2, part = w & 3;
    const int grow = min(m0 + row, g.m - 1);
    asrc[i] = g.a + p * g.a_cs + static_cast<int64_t>(grow) * g.a_ld + part * 16;
    alds[i] = p * PLANE + row * kLdsRow + part * 16;
    apart[i] = part * 16;
    aon[i] = aon[i] && (ARAW || p < c_act);
  });
  const int8_t *bp[NB];
  static_for<NB>([&](auto J) {
    constexpr int j = decltype(J)::value;
    const int col = min(n0 + j * 16 + (lane & 15), g.n - 1);
    bp[j] = g.b + static_cast<int64_t>(col) * g.b_ld + kofs;
  });

  const i32x4 zero = {0, 0, 0, 0};
  i32x4 ra[AC];
  i32x4 fb[P][RCAP][NB];
  auto gload_a = [&](int ks) {
    const int ko = ks * 64;
    static_for<AC>([&](auto II) {
      constexpr int i = decltype(II)::value;
      ra[i] = (aon[i] && ko + apart[i] < g.a_k) ? load16(asrc[i] + ko) : zero;
    });
  };
  auto lstore_a = [&](int buf) {
    static_for<AC>([&](auto II) {
      constexpr int i = decltype(II)::value;
      if (aon[i]) *reinterpret_cast<i32x4 *>(&As[buf][alds[i]]) = ra[i];
    });
  };

  i32x4 acc[RCAP][MB][NB];
  static_for<RCAP>([&](auto C) {
    static_for<MB>([&](auto I) {
      static_for<NB>([&](auto J) { acc[C][I][J] = zero; });
    });
  });

  gload_a(0);
  lstore_a(0);
  static_for<P>([&](auto SS) {
    constexpr int s = decltype(SS)::value;
    if (s < nk) {
      static_for<RCAP>([&](auto C) {
        constexpr int c = decltype(C)::value;
        static_for<NB>([&](auto J) {
          constexpr int j = decltype(J)::value;
          fb[s][c][j] = c < c_act ? load16(bp[j] + c * g.b_cs + s * 64) : zero;
        });
      });
    }
  });
  __syncthreads();

  const int a_frag = (lane & 15) * kLdsRow + kofs;
  for (int ks0 = 0; ks0 < nk; ks0 += P) {
    static_for<P>([&](auto SS) {
      constexpr int s = decltype(SS)::value;
      const int ks = ks0 + s;
      if (ks >= nk) return;
      const int buf = ks & 1;
      const bool more = ks + 1 < nk;
      if (more) gload_a(ks + 1);
      i32x4 fa[MB];
      static_for<RCAP>([&](auto C) {
        constexpr int c = decltype(C)::value;
        if (c >= c_act) return;
        if (!ARAW || c == 0) {
          static_for<MB>([&](auto I) {
            constexpr int i = decltype(I)::value;
            fa[i] = *reinterpret_cast<const i32x4 *>(
                &As[buf][(ARAW ? 0 : c) * PLANE + a_frag + i * 16 * kLdsRow]);
          });
        }
        static_for<MB>([&](auto I) {
          constexpr int i = decltype(I)::value;
          static_for<NB>([&](auto J) {
            constexpr int j = decltype(J)::value;
            acc[c][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[s][c][j], acc[c][i][j], 0, 0, 0);
          });
        });
      });
      if (ks + P < nk) {
        static_for<RCAP>([&](auto C) {
          constexpr int c = decltype(C)::value;
          static_for<NB>([&](auto J) {
            constexpr int j = decltype(J)::value;
            fb[s][c][j] = c < c_act ? load16(bp[j] + c * g.b_cs + (ks + P) * 64) : zero;
          });
        });
      }
      if (more) lstore_a(buf ^ 1);
      __syncthreads();
    });
  }

  // epilogue from registers: lane holds rows 4*(lane>>4)+t of column lane&15
  static_for<MB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    static_for<NB>([&](auto J) {
      constexpr int j = decltype(J)::value;
      const int col = n0 + j * 16 + (lane & 15);
      static_for<4>([&](auto T) {
        constexpr int t = decltype(T)::value;
        const int row = m0 + i * 16 + 4 * (lane >> 4) + t;
        uint32_t d[RCAP];
        static_for<RCAP>([&](auto CC) {
          constexpr int cc = decltype(CC)::value;
          if (cc >= c_act) {
            d[cc] = 0;
            return;
          }
          const uint32_t r = reduce_acc(g, cc, acc[cc][i][j][t]);
          d[cc] = garner_digit<cc>(g.mods, r, [&](int jj) { return d[jj]; });
        });
        if (row < g.m && col < g.n) store_element<RCAP>(g, c_act, d, row, col);
      });
    });
  });
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
    for (int c = 0; c < R && e.out != nullptr; ++c) {
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
    const int64_t p = prefix_at<RCAP>(a.mods, R);
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

enum GemmKind { kAuto = 0, kStream = 1, kMfma = 2 };

struct GemmChoice {
  int kind, mb, nb, ks;
};

// Process-wide override of the kernel choice (rnsmx_set_gemm_override).
static GemmChoice g_override = {kAuto, 0, 0, 0};

static constexpr int kStreamLdsMax = 65536;

static int stream_ks_cap(int rcap, int mb, int nb) {
  const int per_wave = rcap * 256 * mb * nb;
  return std::max(1, std::min(4, kStreamLdsMax / per_wave));
}

// Kernel family and tile for an M x N x kp problem.  Small M streams the
// weights (stream kernel, K split over waves); large M is MFMA-bound (mfma
// kernel, 128-row tiles for up to 4 channels).
static GemmChoice choose_gemm(const GemmArgs &g, bool araw) {
  const int rcap = rcap_for(g.mods.channels);
  const int nk = g.kp / 64;
  GemmChoice c{};
  if (g.m <= 256) {
    // 16- or 32-row tiles of 16 columns: the most workgroups in flight
    c.kind = kStream;
    c.mb = g.m <= 16 ? 1 : 2;
    c.nb = 1;
    const int u = stream_u_of(rcap, araw, c.mb, c.nb);
    const int want = g.m <= 16 ? 4 : (g.m < 256 ? 2 : 1);
    c.ks = std::min(std::min(want, stream_ks_cap(rcap, c.mb, c.nb)), std::max(1, (nk + u - 1) / u));
    return c;
  }
  c.kind = kMfma;
  if (rcap <= 4) {
    c.mb = 8;
    c.nb = 2;
  } else if (rcap == 6) {
    c.mb = 4;
    c.nb = 2;
  } else {
    c.mb = 2;
    c.nb = 2;
  }
  return c;
}

template <int RCAP, bool ARAW>
static bool launch_stream(GemmArgs g, int mb, int nb, int ks, hipStream_t st) {
#define RNSMX_STREAM(MB_, NB_)                                                             \
  if (mb == MB_ && nb == NB_) {                                                            \
    g.tiles_m = (g.m + 16 * MB_ - 1) / (16 * MB_);                                         \
    g.tiles_n = (g.n + 16 * NB_ - 1) / (16 * NB_);                                         \
    const dim3 grid(static_cast<unsigned>(g.tiles_m * g.tiles_n));                         \
    const size_t lds = static_cast<size_t>(ks) * RCAP * StreamCfg<RCAP, MB_, NB_, ARAW>::TILE; \
    hipLaunchKernelGGL((gemm_stream_kernel<RCAP, MB_, NB_, ARAW>), grid, dim3(64 * ks), lds, st, g); \
    return true;                                                                           \
  }
  RNSMX_STREAM(1, 1)
  RNSMX_STREAM(2, 1)
  RNSMX_STREAM(4, 1)
  if constexpr (RCAP <= 4) {
    RNSMX_STREAM(1, 2)
    RNSMX_STREAM(1, 4)
    RNSMX_STREAM(2, 2)
    RNSMX_STREAM(4, 2)
  }
#undef RNSMX_STREAM
  return false;
}

template <int RCAP, bool ARAW>
static bool launch_mfma(GemmArgs g, int mb, int nb, hipStream_t st) {
#define RNSMX_MFMA(MB_, NB_)                                                         \
  if (mb == MB_ && nb == NB_) {                                                      \
    g.tiles_m = (g.m + 16 * MB_ - 1) / (16 * MB_);                                   \
    g.tiles_n = (g.n + 64 * NB_ - 1) / (64 * NB_);                                   \
    const dim3 grid(static_cast<unsigned>(g.tiles_m * g.tiles_n));                   \
    hipLaunchKernelGGL((gemm_mfma_kernel<RCAP, MB_, NB_, 2, ARAW>), grid, dim3(256), 0, st, g); \
    return true;                                                                     \
  }
  if constexpr (RCAP <= 4) {
    RNSMX_MFMA(8, 2)
    RNSMX_MFMA(4, 2)
    RNSMX_MFMA(4, 4)
  } else if constexpr (RCAP == 6) {
    RNSMX_MFMA(4, 2)
  } else {
    RNSMX_MFMA(2, 2)
  }
#undef RNSMX_MFMA
  return false;
}

template <int RCAP>
static bool launch_rcap(const GemmArgs &g, bool araw, const GemmChoice &c, hipStream_t st) {
  if (c.kind == kStream)
    return araw ? launch_stream<RCAP, true>(g, c.mb, c.nb, c.ks, st)
                : launch_stream<RCAP, false>(g, c.mb, c.nb, c.ks, st);
  return araw ? launch_mfma<RCAP, true>(g, c.mb, c.nb, st) : launch_mfma<RCAP, false>(g, c.mb, c.nb, st);
}

// Launches the GEMM for `g`.  araw: A is one int8 matrix for all channels.
static int32_t launch_gemm(const GemmArgs &g, bool araw, hipStream_t st) {
  const int rcap = rcap_for(g.mods.channels);
  GemmChoice c = g_override.kind != kAuto ? g_override : choose_gemm(g, araw);
  if (c.kind == kStream) {
    const int cap = stream_ks_cap(rcap, c.mb, c.nb);
    if (c.ks < 1 || c.ks > cap) {
      set_error("stream GEMM needs 1 <= ks <= %d for this tile", cap);
      return RNSMX_EINVAL;
    }
  }
  bool ok = false;
  switch (rcap) {
    case 3: ok = launch_rcap<3>(g, araw, c, st); break;
    case 4: ok = launch_rcap<4>(g, araw, c, st); break;
    case 6: ok = launch_rcap<6>(g, araw, c, st); break;
    default: ok = launch_rcap<10>(g, araw, c, st); break;
  }
  if (!ok) {
    set_error("no GEMM kernel for kind %d, tile %d x %d, %d channels", c.kind, c.mb, c.nb,
              g.mods.channels);
    return RNSMX_EINVAL;
  }
  return check_launch(c.kind == kStream ? "gemm_stream" : "gemm_mfma");
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
  // room for a padded copy of A (used when K % 16 != 0 or A is not 16-byte
  // aligned) followed by B repacked to [R][N][kp]
  const int64_t a = round_up(channels * m * kp, 256);
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
  int64_t a_ld = k, a_k = k;
  int8_t *b_nk = ws + round_up(R * static_cast<int64_t>(m) * kp, 256);
  if (k % 16 != 0 || !aligned16(a_dev)) {
    // rows of 16-byte chunks are read straight from the caller's planes
    // otherwise (chunks past K load as zero)
    int8_t *a_pad = ws;
    const int64_t total = R * static_cast<int64_t>(m) * kp;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 16384));
    hipLaunchKernelGGL(pad_rows_kernel, dim3(blocks), dim3(256), 0, st, a_dev, static_cast<int64_t>(m),
                       static_cast<int64_t>(k), kp, total, a_pad);
    if (int32_t rc = check_launch("pad_rows")) return rc;
    a_use = a_pad;
    a_ld = kp;
    a_k = kp;
  }
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
  g.a_k = static_cast<int32_t>(a_k);
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
  return launch_gemm(g, false, st);
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
  if (!aligned16(a_dev)) return fail(RNSMX_EINVAL, "activations must be 16-byte aligned");

  // int8 activations with 16-byte rows feed the MFMA directly (they are
  // their own representatives mod every m_c); the encoder then only runs for
  // the adaptive row L1 norms.  Other sources are encoded to residue planes.
  const bool araw = a_dtype == RNSMX_INT8 && k % 16 == 0 && raw_accumulator_fits(*mods, k);
  EncodeArgs e{};
  e.values = a_dev;
  e.rows = m;
  e.cols = k;
  e.out_ld = kp;
  e.plane = static_cast<int64_t>(m) * kp;
  e.out = araw ? nullptr : a_res;
  e.row_l1 = min_ch != 0 ? row_l1 : nullptr;
  e.absmax = nullptr;
  e.mods = *mods;
  if (!araw || min_ch != 0)
    if (int32_t rc = launch_encode_rows(a_dtype, e, st)) return rc;

  GemmArgs g{};
  if (araw) {
    g.a = static_cast<const int8_t *>(a_dev);
    g.a_ld = k;
    g.a_cs = 0;
    g.a_k = k;
  } else {
    g.a = a_res;
    g.a_ld = kp;
    g.a_cs = kp * m;
    g.a_k = static_cast<int32_t>(kp);
  }
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
  return launch_gemm(g, araw, st);
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
  g.a_k = static_cast<int32_t>(kp);
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
  return launch_gemm(g, false, static_cast<hipStream_t>(stream));
}

int32_t rnsmx_set_gemm_override(int32_t kind, int32_t mb, int32_t nb, int32_t ks) {
  clear_error();
  if (kind == kAuto) {
    g_override = GemmChoice{kAuto, 0, 0, 0};
    return RNSMX_OK;
  }
  if (kind != kStream && kind != kMfma) return fail(RNSMX_EINVAL, "kind must be 0 (auto), 1 (stream) or 2 (mfma)");
  if (mb < 1 || nb < 1) return fail(RNSMX_EINVAL, "tile blocks must be positive");
  g_override = GemmChoice{kind, mb, nb, ks};
  return RNSMX_OK;
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
