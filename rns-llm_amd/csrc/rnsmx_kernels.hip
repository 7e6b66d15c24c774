// rnsmx device code for gfx950 (MI355X) outside the GEMM: residue
// encoders, Garner decode of residue planes, operand repacking for the
// drop-in fused op, the GEMM kernel choice and the C ABI.  The GEMM kernels
// themselves live in rnsmx_gemm.hpp (instantiated in rnsmx_gemm_part.hip,
// once per channel capacity and part).
//
// Data layout in HBM
//   residue planes   [R][rows][ld] int8, K contiguous, ld a multiple of 64
//                    and bytes [K, ld) zero, so every MFMA fragment is one
//                    aligned 16-byte load and the K loop needs no tail.
//   prepared weight  [R][N][kp]: B stored K-contiguous (the nn.Linear weight
//                    orientation); the reference keeps [R][K][N]
//                    (cuda_backend.py:68-76, rns_linear.py:185).
//   output           [M][N] int64 (exact) or float32/float16/bfloat16.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <mutex>

#include "rnsmx_gemm.hpp"

namespace rnsmx {

// ---------------------------------------------------------------------------
// Argument blocks (passed by value; kernarg memory)
// ---------------------------------------------------------------------------
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

// Sum of v over the workgroup (up to 16 waves), returned to every thread.
// sh: 16 words of LDS; uniform control flow required.
__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t *sh) {
  v = wave_sum_i64(v);
  const int nw = static_cast<int>(blockDim.x >> 6);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  int64_t t = 0;
  for (int i = 0; i < nw; ++i) t += sh[i];
  return t;
}

// Activation encoder: one workgroup per (row, channel) (blockIdx.x = row,
// blockIdx.y = channel), each thread 16 consecutive K values per pass of
// 16 * blockDim.x.  Writes the channel's centered residue plane with zero
// padding to out_ld; the channel-0 workgroup also sums the row L1 and folds
// max |v| (when asked).  With e.out null only the channel-0 workgroups run
// (row L1 alone).  Spreading one row over R x K/16 threads keeps small
// batches short: one wave per row, every channel in turn, measured 17.6 us
// for a single int16 row of K = 4096 against 6 channels.
//
// PK (packed weights): also the plane of d_c a with d_c = 256 mod m_c (at
// plane R + c) and the row term (128 sum_k a_k) mod m_c, int32, after the
// 2R planes at [R][packed_corr_ld(rows)].
constexpr int kPackedMaxChannels = 6;

template <typename T, bool PK>
__global__ __launch_bounds__(256) void encode_rows_kernel(const EncodeArgs e) {
  __shared__ int64_t sh[16];
  const int64_t row = blockIdx.x;
  const int c = static_cast<int>(blockIdx.y);
  const int R = e.mods.channels;
  const T *src = static_cast<const T *>(e.values) + row * e.cols;
  const bool vec = (e.cols % 16) == 0;
  const uint32_t m = static_cast<uint32_t>(e.mods.moduli[c]);
  const uint32_t magic = e.mods.magic[c], c31 = e.mods.c31[c];
  const int32_t d = static_cast<int32_t>(256u % m);
  const bool lead = c == 0;
  int64_t l1 = 0;
  int32_t amax = 0, s = 0;
  for (int64_t k0 = static_cast<int64_t>(threadIdx.x) * 16; k0 < e.out_ld; k0 += static_cast<int64_t>(blockDim.x) * 16) {
    int32_t v[16];
    if (vec && k0 + 16 <= e.cols) {
      load16<T>(src + k0, v);
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = (k0 + q < e.cols) ? static_cast<int32_t>(src[k0 + q]) : 0;
    }
    if (lead) {
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int32_t a = v[q] < 0 ? -v[q] : v[q];  // |INT32_MIN| wraps; widened below
        l1 += v[q] < 0 ? -static_cast<int64_t>(v[q]) : v[q];
        amax = static_cast<uint32_t>(a) > static_cast<uint32_t>(amax) ? a : amax;
      }
    }
    if (e.out == nullptr) continue;
    i32x4 w, w2;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t packed = 0, packed2 = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int32_t r = centered_i32(v[4 * g + q], m, magic, c31);
        packed |= (static_cast<uint32_t>(r) & 0xFFu) << (8 * q);
        if constexpr (PK) {
          s += r;
          packed2 |= (static_cast<uint32_t>(centered_i32(d * r, m, magic, c31)) & 0xFFu) << (8 * q);
        }
      }
      w[g] = static_cast<int32_t>(packed);
      w2[g] = static_cast<int32_t>(packed2);
    }
    *reinterpret_cast<i32x4 *>(e.out + c * e.plane + row * e.out_ld + k0) = w;
    if constexpr (PK) *reinterpret_cast<i32x4 *>(e.out + (R + c) * e.plane + row * e.out_ld + k0) = w2;
  }
  if (lead && e.row_l1 != nullptr) {
    l1 = block_sum_i64(l1, sh);
    if (threadIdx.x == 0) e.row_l1[row] = l1;
  }
  if (lead && e.absmax != nullptr) {
    const int64_t am = wave_max_i64(static_cast<int64_t>(static_cast<uint32_t>(amax)));
    if ((threadIdx.x & 63) == 0) atomicMax(e.absmax, static_cast<int32_t>(am > INT_MAX ? INT_MAX : am));
  }
  if constexpr (PK) {
    const int64_t total = block_sum_i64(s, sh);  // |sum| <= 127 K
    if (threadIdx.x == 0) {
      const int64_t t = (128 * (total % m)) % m;
      reinterpret_cast<int32_t *>(e.out + 2 * R * e.plane)[c * packed_corr_ld(e.rows) + row] =
          static_cast<int32_t>(t < 0 ? t + m : t);
    }
  }
}

// The adaptive bound's max_i sum_k |a_ik| of raw int8 rows (cols a multiple
// of 16), reduced to at most 256 words so that every GEMM wave folds those
// instead of all M norms (C5 M=2048: 2048 norms re-read by each of 1024
// workgroups before their first load).  Each wave sums whole rows (a lane
// 16 bytes per 1 KB of the row) and workgroup b writes the largest of its
// rows to row_l1[b]; the GEMM that follows reads them (the launch boundary
// orders the stores before its loads).  Folding them here into one word
// through an arrival counter cost more: the arrivals on the one counter are
// serialised at the memory side (256 of them ~2-3 us, 2048 some 20 us).
__global__ __launch_bounds__(256) void row_l1_max_kernel(const EncodeArgs e) {
  __shared__ int64_t sh[4];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int8_t *src = static_cast<const int8_t *>(e.values);
  int64_t best = 0;
  // Each wave takes two rows at a time and each lane issues its 16-byte
  // loads of both, up to 4 KB of row per pass, before it sums any: one
  // memory round trip per pass instead of one per 1 KB of row.
  constexpr int kChunks = 4;  // 1 KB row chunks per pass
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
  const i32x4 zero = {0, 0, 0, 0};
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * 4 + wv; r0 < e.rows; r0 += 2 * stride) {
    const int64_t r1 = r0 + stride;
    const bool two = r1 < e.rows;
    uint32_t sum0 = 0, sum1 = 0;  // |a| <= 128 and K < 2^24: no overflow
    for (int64_t k0 = lane * 16; k0 < e.cols; k0 += 64 * 16 * kChunks) {
      i32x4 w0[kChunks], w1[kChunks];
      static_for<kChunks>([&](auto J) {
        constexpr int j = decltype(J)::value;
        const int64_t k = k0 + j * 1024;
        w0[j] = zero;
        w1[j] = zero;
        if (k < e.cols) {
          w0[j] = *reinterpret_cast<const i32x4 *>(src + r0 * e.cols + k);
          if (two) w1[j] = *reinterpret_cast<const i32x4 *>(src + r1 * e.cols + k);
        }
      });
      static_for<kChunks>([&](auto J) {
        constexpr int j = decltype(J)::value;
        sum0 = abs_sum_i8x16(w0[j], sum0);
        sum1 = abs_sum_i8x16(w1[j], sum1);
      });
    }
    const int64_t row0 = wave_sum_i64(static_cast<int64_t>(sum0)), row1 = wave_sum_i64(static_cast<int64_t>(sum1));
    best = row0 > best ? row0 : best;
    best = row1 > best ? row1 : best;
  }
  if (lane == 0) sh[wv] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) best = sh[w] > best ? sh[w] : best;
    e.row_l1[blockIdx.x] = best;
  }
}

// Weight preparation into the fragment-major layout the GEMM kernels read:
// [R][N16][nk][64 lanes x 16 bytes] (N16 = ceil(N/16), nk = kp/64).  Lane l
// of fragment (column block jb, K step ks) holds column 16*jb + (l & 15),
// K bytes 64*ks + 16*(l >> 4) .. +16: the v_mfma_i32_16x16x64_i8 B-operand
// layout, so a fragment is one contiguous 1 KB load in which every group of
// four lanes reads 64 consecutive bytes.  One wave per column block: lane l
// reads 16 K values of source row n = 16*jb + (l & 15) per step and writes
// 16 bytes at fragment offset 16*l for every channel.  Columns past N and K
// values past K are zero; max |b| is folded into absmax.
template <typename T>
__global__ __launch_bounds__(256) void encode_frag_kernel(const EncodeArgs e) {
  const int lane = threadIdx.x & 63;
  const int64_t jb = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t n16 = (e.rows + 15) / 16;
  if (jb >= n16) return;
  const int64_t n = jb * 16 + (lane & 15);
  const bool row_ok = n < e.rows;
  const T *src = static_cast<const T *>(e.values) + (row_ok ? n : 0) * e.cols;
  const bool vec = (e.cols % 16) == 0;
  const int64_t nk = e.out_ld / 64;
  int8_t *dst = e.out + jb * nk * 1024 + lane * 16;
  int32_t amax = 0;
  const int R = e.mods.channels;
  for (int64_t ks = 0; ks < nk; ++ks) {
    const int64_t k0 = ks * 64 + (lane >> 4) * 16;
    int32_t v[16];
    if (row_ok && vec && k0 + 16 <= e.cols) {
      load16<T>(src + k0, v);
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = (row_ok && k0 + q < e.cols) ? static_cast<int32_t>(src[k0 + q]) : 0;
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int32_t a = v[q] < 0 ? -v[q] : v[q];  // |INT32_MIN| wraps to INT32_MIN: largest unsigned
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
      *reinterpret_cast<i32x4 *>(dst + c * e.plane + ks * 1024) = w;
    }
  }
  if (e.absmax != nullptr) {
    int64_t am = wave_max_i64(static_cast<int64_t>(static_cast<uint32_t>(amax)));
    if (lane == 0) atomicMax(e.absmax, static_cast<int32_t>(am > INT_MAX ? INT_MAX : am));
  }
}

template <typename T>
__device__ __forceinline__ void load4(const T *p, int32_t (&v)[4]) {
  if constexpr (sizeof(T) == 1) {
    const uint32_t w = *reinterpret_cast<const uint32_t *>(p);
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = static_cast<int8_t>((w >> (8 * q)) & 0xFFu);
  } else if constexpr (sizeof(T) == 2) {
    const uint2 w = *reinterpret_cast<const uint2 *>(p);
    v[0] = static_cast<int16_t>(w.x & 0xFFFFu);
    v[1] = static_cast<int16_t>(w.x >> 16);
    v[2] = static_cast<int16_t>(w.y & 0xFFFFu);
    v[3] = static_cast<int16_t>(w.y >> 16);
  } else {
    const i32x4 w = *reinterpret_cast<const i32x4 *>(p);
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = w[q];
  }
}

// Residue planes of a few rows (no row norm, no max |v|, no packed planes):
// one thread per 4 K values, grid (row, channel, K / 1024), so a short
// batch's encode is spread over many workgroups (its latency, not its
// bytes, is what the step pays).  Int16, 6 channels, K=4096, N=12288: M=16
// 60.1-60.9 against 61.3-61.5 us per step; M=1 and 4 within noise.
template <typename T>
__global__ __launch_bounds__(256) void encode_rows_split_kernel(const EncodeArgs e) {
  const int64_t row = blockIdx.x;
  const int c = static_cast<int>(blockIdx.y);
  const int64_t k0 = (static_cast<int64_t>(blockIdx.z) * 256 + threadIdx.x) * 4;
  if (k0 >= e.out_ld) return;
  const T *src = static_cast<const T *>(e.values) + row * e.cols;
  int32_t v[4];
  if (e.cols % 16 == 0 && k0 + 4 <= e.cols) {
    load4<T>(src + k0, v);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = (k0 + q < e.cols) ? static_cast<int32_t>(src[k0 + q]) : 0;
  }
  const uint32_t m = static_cast<uint32_t>(e.mods.moduli[c]);
  const uint32_t magic = e.mods.magic[c], c31 = e.mods.c31[c];
  uint32_t packed = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) packed |= (static_cast<uint32_t>(centered_i32(v[q], m, magic, c31)) & 0xFFu) << (8 * q);
  *reinterpret_cast<uint32_t *>(e.out + c * e.plane + row * e.out_ld + k0) = packed;
}

// Activations for rows_packed_kernel (packed weights at decode):
// [block][a' | a][kp/64][1 KB] MFMA A fragments in which row t * rpt + c of
// block b holds token b * (16 / rpt) + t, channel c (a' = centered residue
// of d_c a, d_c = 256 mod m_c); rows past the tokens or the channels and K
// past cols are zero.  Lane l of a fragment holds row l & 15, K bytes
// 64 ks + 16 (l >> 4) .. +16.  One thread per 4-byte word (word w of a
// fragment: lane w >> 2, bytes 4 (w & 3) of that lane's 16), so each
// thread forms 4 residues (8 with a'): the encode is one short dependent
// launch before the GEMM, whose latency is what counts; 16 values per lane
// (one wave per fragment) made the packed decode step ~1 us slower (M=1,
// K=4096, N=12288: 23.5 against 22.6 us).
struct TokenRowsArgs {
  const void *values;
  int64_t m, cols, nk, blocks;  // blocks: the GEMM's (blocks past the tokens are zero)
  int32_t rpt;                  // rows per token: the kernel's channel capacity
  int8_t *out;
  rnsmx_moduli_t mods;
};

template <typename T>
__global__ __launch_bounds__(256) void encode_token_rows_kernel(const TokenRowsArgs e) {
  const int64_t word = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t f = word >> 8;  // 1 KB fragment: 256 words
  if (f >= e.blocks * 2 * e.nk) return;
  const int w = static_cast<int>(word & 255), lane = w >> 2;
  const int tpb = 16 / e.rpt;
  const int64_t ks = f % e.nk, b = f / (2 * e.nk);
  const bool scaled = (f / e.nk) % 2 == 0;  // a' fragments first
  const int r = lane & 15, t = r / e.rpt, c = r % e.rpt;
  const int64_t token = b * tpb + t, k0 = ks * 64 + (lane >> 4) * 16 + 4 * (w & 3);
  uint32_t packed = 0;
  if (t < tpb && token < e.m && c < e.mods.channels) {
    const T *src = static_cast<const T *>(e.values) + token * e.cols;
    int32_t v[4];
    if (e.cols % 16 == 0 && k0 + 4 <= e.cols) {
      load4<T>(src + k0, v);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = (k0 + q < e.cols) ? static_cast<int32_t>(src[k0 + q]) : 0;
    }
    const uint32_t m = static_cast<uint32_t>(e.mods.moduli[c]);
    const uint32_t magic = e.mods.magic[c], c31 = e.mods.c31[c];
    const int32_t d = static_cast<int32_t>(256u % m);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int32_t x = centered_i32(v[q], m, magic, c31);
      if (scaled) x = centered_i32(d * x, m, magic, c31);
      packed |= (static_cast<uint32_t>(x) & 0xFFu) << (8 * q);
    }
  }
  reinterpret_cast<uint32_t *>(e.out)[word] = packed;
}

// Packed weight preparation: int8/int16 [N][K] -> two byte planes in the
// fragment-major order of encode_frag_kernel ([2][N16][nk][1024]): hi =
// v >> 8 and lo = (v & 255) - 128, so v = 256 hi + lo + 128 with both bytes
// in int8 range.  Columns past N and K values past K hold v = 0 (hi 0, lo
// -128; their activations are zero); max |v| is folded into absmax.
template <typename T>
__global__ __launch_bounds__(256) void pack_frag_kernel(const EncodeArgs e) {
  const int lane = threadIdx.x & 63;
  const int64_t jb = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t n16 = (e.rows + 15) / 16;
  if (jb >= n16) return;
  const int64_t n = jb * 16 + (lane & 15);
  const bool row_ok = n < e.rows;
  const T *src = static_cast<const T *>(e.values) + (row_ok ? n : 0) * e.cols;
  const bool vec = (e.cols % 16) == 0;
  const int64_t nk = e.out_ld / 64;
  int8_t *dst = e.out + jb * nk * 1024 + lane * 16;
  int32_t amax = 0;
  for (int64_t ks = 0; ks < nk; ++ks) {
    const int64_t k0 = ks * 64 + (lane >> 4) * 16;
    int32_t v[16];
    if (row_ok && vec && k0 + 16 <= e.cols) {
      load16<T>(src + k0, v);
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = (row_ok && k0 + q < e.cols) ? static_cast<int32_t>(src[k0 + q]) : 0;
    }
    i32x4 hi, lo;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t h = 0, l = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int32_t x = v[4 * g + q];
        amax = max(amax, x < 0 ? -x : x);
        h |= (static_cast<uint32_t>(x >> 8) & 0xFFu) << (8 * q);
        l |= ((static_cast<uint32_t>(x) & 0xFFu) ^ 0x80u) << (8 * q);
      }
      hi[g] = static_cast<int32_t>(h);
      lo[g] = static_cast<int32_t>(l);
    }
    *reinterpret_cast<i32x4 *>(dst + ks * 1024) = hi;
    *reinterpret_cast<i32x4 *>(dst + e.plane + ks * 1024) = lo;
  }
  if (e.absmax != nullptr) {
    int64_t am = wave_max_i64(static_cast<int64_t>(amax));
    if (lane == 0) atomicMax(e.absmax, static_cast<int32_t>(am));
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
  Epi<RCAP> k;
  fill_moduli<RCAP>(k, a.mods, R);
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < a.count;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    uint32_t r[RCAP];
    static_for<RCAP>([&](auto CC) {
      constexpr int c = decltype(CC)::value;
      if (c >= R) {
        r[c] = 0;
        return;
      }
      const int32_t m = a.mods.moduli[c];
      const int32_t v = a.res[c * a.count + e];  // centered residue, |v| <= m/2
      r[c] = static_cast<uint32_t>(v < 0 ? v + m : v);
    });
    a.out[e] = garner_value<RCAP>(k, r, R);
  }
}

// ---------------------------------------------------------------------------
// Repacking for the drop-in op (reference layouts -> K-contiguous, padded)
// ---------------------------------------------------------------------------
// src [R][K][N] (the reference layout) -> the fragment-major layout of
// encode_frag_kernel, zero padded: one thread per 16-byte fragment slot.
// Also clears the first `ntickets` split counters of the workspace (the
// drop-in op's workspace may hold anything before the call).
__global__ __launch_bounds__(256) void transpose_frag_kernel(const int8_t *__restrict__ src, int64_t k,
                                                             int64_t n, int64_t n16, int64_t nk,
                                                             int64_t total, int8_t *__restrict__ dst,
                                                             uint32_t *__restrict__ tickets, int64_t ntickets) {
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < ntickets;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x)
    tickets[q] = 0;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < total;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int lane = static_cast<int>(q & 63);
    int64_t t = q >> 6;
    const int64_t ks = t % nk;
    t /= nk;
    const int64_t jb = t % n16, c = t / n16;
    const int64_t nn = jb * 16 + (lane & 15), kb = ks * 64 + (lane >> 4) * 16;
    uint32_t word[4] = {0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const int64_t kk = kb + b;
      const uint32_t v = (nn < n && kk < k) ? static_cast<uint8_t>(src[(c * k + kk) * n + nn]) : 0u;
      word[b >> 2] |= v << (8 * (b & 3));
    }
    i32x4 w;
    w[0] = static_cast<int32_t>(word[0]);
    w[1] = static_cast<int32_t>(word[1]);
    w[2] = static_cast<int32_t>(word[2]);
    w[3] = static_cast<int32_t>(word[3]);
    *reinterpret_cast<i32x4 *>(dst + q * 16) = w;
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
// Scratch of rnsmx_matmul_prepared_fused_noalloc: one array per GPU, held
// until the process ends.  Its first RNSMX_SPLIT_TICKETS words are the K
// split's arrival counters, zero when the code object is loaded (the array
// is zero-initialised device memory) and cleared again by a fill kernel at
// the first call on each device; every call leaves them zero.
// ---------------------------------------------------------------------------
static __device__ __align__(256) int8_t scratch[RNSMX_NOALLOC_SCRATCH_BYTES];

__global__ __launch_bounds__(256) void fill_zero_kernel(uint32_t *p, int64_t words) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0;
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

static bool is_lds(int kind) { return kind == kLds || kind == kLdsWide || kind == kLdsPlanes; }

static int32_t check_launch(const char *what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(err));
    return RNSMX_ELAUNCH;
  }
  return RNSMX_OK;
}

static constexpr int kStreamLdsMax = 65536;

// Up to this many raw int8 rows, the adaptive prefix's row norms are summed
// inside the GEMM (every workgroup reads all the rows) instead of by a
// separate encoder launch.  Beyond it the encoder sums them; up to
// kAdaptiveFoldInGemm rows every GEMM wave folds the norms (at most 2 KB),
// beyond that row_l1_max_kernel reduces them to that many words first (C5
// M=2048: 2048 norms re-read by each of 1024 workgroups before their first
// load).
static constexpr int kAdaptiveRowsInGemm = 4;
static constexpr int kAdaptiveFoldInGemm = 256;

static int stream_ks_cap(int rcap, int mb, int nb) {
  const int per_ws = rcap * 256 * mb * nb * 4;  // int32 partial sums in LDS
  return per_ws > kStreamLdsMax ? 1 : 4;
}

// Kernel family and tile for an M x N x kp problem, from sweeps on MI355X
// (K = 768 to 4096, N = 768 to 12288).  For few rows (up to 16; up to 64
// unless K is long and N wide; up to 128 while its 32-row tiles number at
// most 512) the stream kernel (K split over 4 waves, chunks of 8 K steps
// from K = 4096) keeps the most weight loads in flight.  Beyond 128 rows the LDS-staged kernel (256 x 64 tiles)
// wherever it applies, K is at
// least 2048 (at K = 768 the MFMA kernel's 64 x 64 tiles measured faster)
// and its tiles alone give every CU a workgroup; otherwise the MFMA kernel:
// 128 x 128 tiles once they give >= 1024 workgroups (their weight reuse then
// pays for one wave per SIMD), else 32, 48 or 64 x 64 (or x 48) tiles,
// the one that leaves the fewest rows on any CU.
// packed: packed weights (packed_auto), which keep the raw-activation row
// rule of the stream kernel (their stream kernel reads two weight planes).
static GemmChoice choose_gemm(const GemmArgs &g, bool araw, bool packed = false) {
  const int rcap = rcap_for(g.mods.channels);
  const int nk = g.kp / 64;
  auto tiles = [&](int bm, int bn) {
    return static_cast<int64_t>((g.m + bm - 1) / bm) * ((g.n + bn - 1) / bn);
  };
  GemmChoice c{};
  // Stream kernel up to 16 rows; up to 64 while its 16 x 16 tiles number
  // under 1024 (K=4096, N=12288: M=64 45 us with the MFMA kernel against 79,
  // M=32 39 against 54; N=4096 M=64 28 against 33; K=768 N=8192 M=32 9.3
  // against 11.0; at K=768, N=2304, M=64 the stream kernel's 6.9 against
  // 8.7); up to 128 while its 32 x 16 tiles number at most 512 (M=128:
  // N=2304 8.8 us with the MFMA kernel against 9.6, N=4608 10.3 against
  // 14.0, K=4096 N=12288 62 against 110; at N=768, 192 tiles, 5.1 against
  // 7.4; at M=96, N=2304, 432 tiles, 7.6 against 8.7); up to 192 at K <= 2048 while its 16 x 16 tiles number at
  // most 768 (N=768: K=768 M=160 6.4 against 7.5, M=192 7.1 against 7.6;
  // K=2048 M=192 11.0 against 12.1; at K=4096 the MFMA kernel's K split
  // wins, 15.6 against 17.1).
  // Residue-plane activations (int16 / int32 inputs) make every stream wave
  // load each channel's A fragment as well (as many bytes as the weight
  // residues at M <= 16, against one shared fragment for raw int8); there
  // the stream kernel pays only up to 48 rows while the MFMA kernel's 32 x
  // 64 tiles number under 128 (K=4096, 6 channels: N=12288 M=1/16 65/68 us
  // with the MFMA kernel against 81/98, N=8192 M=16 60 against 70, N=4096
  // M=16 39 with the stream kernel against 54, M=64 60 with the MFMA kernel
  // against 105; K=768, N=2304: M=16 12.6 stream against 17.2, M=48 12.5
  // against 13.8 with 4 channels, M=64 18.9 MFMA against 24.1, M=96 19.0
  // against 30.8).  Packed weights, whose stream kernel loads 2R activation
  // planes per step, take the same rule (K=768 N=2304 M=96 29.6 us on MFMA
  // tiles against 40.7).
  const bool plane_rule = packed || !araw;
  const bool stream = plane_rule ? g.m <= 48 && tiles(32, 64) < 128
                                 : g.m <= 16 || (g.m <= 64 && tiles(16, 16) < 1024) ||
                                       (g.m > 64 && g.m <= 128 && tiles(32, 16) <= 512) ||
                                       (g.m > 128 && g.m <= 192 && nk <= 32 && tiles(16, 16) <= 768);
  // Raw int8 past 4 channels has no 8-step chunks: where they would be used
  // (K >= 4096) the MFMA kernel's 32 x 64 tiles win from 128 of them (6
  // channels, K=4096: N=12288 M=1/16 58 us against 67/72, N=8192 M=1 43.6
  // against 46.8), elsewhere the raw rule holds (N=768 M=96 7.3 against 11.3
  // at K=768, 17.2 against 33.4 at K=4096; K=768 N=8192 M=1 10.6 against
  // 12.3).
  const bool no_chunks = araw && rcap > 4 && nk >= 64 && tiles(32, 64) >= 128;
  if (stream && !no_chunks) {
    // 16-row tiles up to 64 rows, and beyond while they number at most 768
    // (raw int8, K=768: N=768 M=96 5.95 us against 6.73 with 32-row tiles,
    // M=128 6.35 against 6.87; N=2304 M=80 7.77 against 8.27; at M=96,
    // 864 tiles, 8.88 against 8.75)
    c.mb = g.m <= 64 || (!packed && tiles(16, 16) <= 768) ? 1 : 2;
    c.nb = 1;
    // chunks of 8 K steps once K >= 4096 (16-row tiles, up to 4 channels,
    // raw int8 activations): each wave then has half as many dependent round
    // trips to memory.  With residue planes the A fragments share the
    // registers and the 7-step chunks measured slower (K=4096, N=4096, 4
    // channels, M=1: 25.7 against 20.9 us with chunks of 4).
    // From K = 2048 too, up to 32 rows and 384 tiles (N=768 M=1/8/32
    // 6.25/6.67/7.28 us against 7.18/7.53/7.80 with chunks of 4; N=3072 M=1
    // 8.00 against 9.09; N=8192, 512 tiles, 23.2 against 16.5).
    const bool wide = araw && c.mb == 1 && rcap <= 4 &&
                      (nk >= 64 || (nk >= 32 && g.m <= 32 && tiles(16, 16) <= 384));
    c.kind = wide ? kStreamWide : kStream;
    const int u = stream_u_of(rcap, araw, c.mb, c.nb, wide ? 8 : 4);
    c.ks = std::min(stream_ks_cap(rcap, c.mb, c.nb), std::max(1, (nk + u - 1) / u));
    // From 16 rows the 16 x 16 tile's LDS epilogue (256 elements) runs one
    // element per thread with 4 waves, and that pays for a 4th wave even
    // where the K chunks keep only 3 busy (K=768: M=16 5.18 us against
    // 5.64 with 3 waves, M=80 5.14 against 5.76; K=512 M=16 5.05 against
    // 5.58); fewer rows go the one-element path, where the 3rd wave is
    // enough (M=1-8 0.1-0.2 us faster with 3).
    if (g.m >= 16 && c.mb == 1) c.ks = stream_ks_cap(rcap, c.mb, c.nb);
    c.splits = 1;
    return c;
  }
  // The LDS kernel's 256 x 64 tiles run one workgroup per CU (128 KB of
  // LDS each), so at short K, where a tile's prologue and epilogue weigh
  // more, it wins only when its tiles fill whole rounds of the chip's 256
  // CUs (measured at K = 768-1024: 3 and 1 full rounds faster than the
  // MFMA kernel by 7 % and 30 %; 2.25 rounds slower by 6 %).
  // Two LDS tile widths: 256 x 96 stages 25 % fewer bytes per MFMA, and a
  // round of its workgroups takes 1.38 times as long as one of 256 x 64
  // tiles at K = 4096 (C5: M=2048 6 rounds of 64 columns 358 us against 4
  // of 96 columns 328 us; M=1024 3 rounds 177 against 2 rounds 170; M=512
  // 1.5 rounds with the tail split 102 against one round 87.6; N=4096
  // M=2048 2 rounds 114 against 1.34 rounds 145).  Cost: rounds of 256
  // workgroups times that factor, a tail round the 64-column kernel splits
  // over K counted as 0.7.
  const int64_t t64 = tiles(kLdsBM, kLdsBN), t96 = tiles(kLdsBM, kLdsWBN);
  auto lds_cost = [&](int64_t t, int per_round, bool tail_split) {
    const int64_t last = t % 256;
    const int64_t last_cost = last == 0 ? 0 : (tail_split && last <= 128 && nk >= 32) ? 70 : 100;
    return (t / 256 * 100 + last_cost) * per_round;
  };
  const bool wide = lds_cost(t96, 138, false) < lds_cost(t64, 100, true);
  const int64_t lds_tiles = wide ? t96 : t64;
  const int64_t rounds = (lds_tiles + 255) / 256;
  const bool full_rounds = 8 * lds_tiles >= 7 * 256 * rounds;
  c.splits = 1;
  // One round of LDS tiles runs in about the same time however many of the
  // 256 CUs it fills (256 x 64: 18.5 us at K=768, 28.5 at K=2048, 45 at
  // K=4096), and from 144 tiles (over half a round) that beats the MFMA
  // tiles at every K measured, from 192 rows (128 at K >= 4096, where each
  // weight column's reuse over 256 rows pays however many are padding):
  // K=768 N=4608 M=512 (144 tiles) 19.1 against 21.5, N=3072 M=1024 19.0
  // against 20.8; K=2048 N=3072 M=768 28.8 against 35.4, N=768 M=3072
  // 28.8 against 35.1; K=4096 N=12288 M=128 48.8 against 62.5, M=192 53.2
  // against 80.7; with 96 tiles or fewer the MFMA tiles win (K=4096
  // N=3072 M=384 34.0 against 44.6; N=4096 M=256, 64 tiles, 31.9 against
  // 46.3; at K=4096 128 tiles win too: N=8192 M=192 48.2 against 55.6).
  // The 256 x 96 tile takes one round where the 256 x 64 one needs a
  // second (K=768 M=1536 N=3072: 192 wide tiles 25.3 us against 29.9 on
  // MFMA tiles; K=2048 43.1 against 59.2 with 288 narrow tiles, the tail
  // split; K=4096 70.7 against 87.6).
  const bool one_round = lds_tiles >= (nk >= 64 ? 128 : 144) && lds_tiles <= 256 && nk < 128 &&
                         (g.m >= 192 || (g.m >= 128 && nk >= 64));
  if (lds_kernel_fits(g, araw, rcap) &&
      ((g.m > 128 && t64 >= 256 && (g.kp >= 2048 || full_rounds)) || one_round)) {
    c.kind = wide ? kLdsWide : kLds;
    return c;
  }
  // Residue-plane activations (int16 / int32 inputs) with 4 or 6 channels:
  // the 128 x 128 LDS-staged kernel from 64 rows, given 4096 tile-steps of
  // work (int16 x int8, K = 4096, 6 channels: M=64 N=12288 81 us with K in
  // two halves against 111 with the MFMA kernel, M=128 94 against 205,
  // M=256 123 against 304, M=512 N=4096 84 against 210; 4 channels M=2048
  // N=12288 472 against 886; K = 768, N = 2304: M=4096 81 against 108, but
  // M=256 (36 tiles, 12 steps) 28.5 against 19.6, so not there).
  // From 48 rows too: K=4096 N=12288 M=48, 6 channels, 90.8 us with K in
  // two halves against 103 on 32-row MFMA tiles; and from 128 tiles at any
  // K (K=768 N=2304 M=1024, 144 tiles: 44.7 against 86.1 with 6 channels,
  // 32.9 against 42.5 with 4).
  if (g.m >= 48 && lds_planes_fits(g, araw, rcap) &&
      (tiles(kPlBM, kPlBN) * nk >= 4096 || tiles(kPlBM, kPlBN) >= 128)) {
    c.kind = kLdsPlanes;
    return c;
  }
  c.kind = kMfma;
  c.ks = 0;  // the tile's default ring depth
  c.nb = 1;
  if (g.m > 128 && rcap <= 4 && tiles(128, 128) >= 1024) {
    c.mb = 8;
    c.nb = 2;
    return c;
  }
  // Residue-plane activations stage R A planes per K step (raw int8 one),
  // so their bytes grow with the tile height: 32-row tiles up to three
  // rounds of them with 6 channels, one with 4, whatever the rows per CU (6
  // channels, K=768 N=2304: M=256 27.2 us against 32.6 with 64-row tiles,
  // M=512 39.1 against 56.6; 4 channels K=4096 N=4096 M=64 43.6 against
  // 58.6, but K=768 N=2304 M=256, 288 tiles, 23.2 against 21.7).
  if (!araw && tiles(32, 64) <= (rcap >= 6 ? 768 : 256)) {
    c.mb = 2;
    if (rcap <= 6) c.ks = 4;
    return c;
  }
  // 32, 48 or 64 rows x 64 (or 48) columns: among the tiles that give at
  // most 512 workgroups, the one with the fewest rows per CU, counted as
  // rounds of 256 workgroups times the tile height; 64 x 64 when none does
  // (more tiles then re-read every weight column more often).
  // Swept on MI355X at K = 768 (N = 768-4608, M = 96-448), K = 2048 and
  // K = 4096 (N = 12288, M = 16-256), this picks the fastest height at
  // every shape: C2 M=256 (N=2304) 48 rows, 216 tiles, 9.9 us against 11.0
  // with 64 and 11.1 with 32; M=160-224 32 rows (8.98-9.20 against 9.6-9.8
  // and 10.8-10.9); M=384-448 64 rows (11.3-11.6 against 11.7-12.0 and
  // 12.6-12.9); N=4608 M=256 48 rows (13.6 against 15.2 and 15.7); C5
  // M=128 64 rows (62 us against 68 with 32 rows, 768 tiles); C5 M=32 32
  // rows (38 against 42).  The 48-row tile is built for up to 4 channels.
  // At K <= 1024 tiles of 48 columns (three waves) are candidates too
  // (raw int8 activations, up to 4 channels): on a tie in rows per CU the
  // choice that fits one round of 256 workgroups with the most of them wins
  // (C2 M=128 32 x 48, 192 tiles, 8.3 us against 8.8 with 32 x 64; N=1536
  // M=256 8.5 against 9.0; K=1024 N=3072 M=256 64 x 48, 12.9 against 13.5),
  // past one round the one whose last round is fuller (K=768 N=3072 M=384:
  // 48 x 48, 512 tiles, 12.4 against 14.0 with 384 of 48 x 64; N=768
  // M=1536 12.1 against 13.2), then the taller, then the wider tile.  48 x 48 and 64 x 48 never beat
  // 48 x 64 on the headline (10.9 against 9.9 us).  At K = 2048-4096 the
  // same tie-break gains 2-10 % (K=4096: N=12288 M=48 40.2 us against 41.0,
  // M=64 43.2 against 46.4; N=4096 M=64 25.6 against 28.1; N=6144 M=64
  // 28.4 against 30.3; K=2048 N=4096 M=64 13.6 against 15.1).
  c.mb = 4;
  int best_w = 4;
  int64_t best_rows = -1, best_fill = 0;
  for (int w = 4; w >= 3; --w) {
    if (w == 3 && !(araw && rcap <= 4)) continue;
    for (int mb = 4; mb >= 2; --mb) {
      if (mb == 3 && rcap > 4) continue;
      // past K = 1024 a three-wave tile only where the four-wave one of its
      // height already gives 128 workgroups and K is under 8192 (so neither
      // would split K over workgroups)
      if (w == 3 && nk > 16 && !(nk < 128 && tiles(16 * mb, 64) >= 128)) continue;
      const int64_t t = tiles(16 * mb, 16 * w);
      if (t > 512) continue;
      const int64_t rows = (t + 255) / 256 * (16 * mb);
      // a single round first (by its workgroups), then the fuller last round
      const int64_t fill = t <= 256 ? 256 + t : t - (t - 1) / 256 * 256;
      const bool better = best_rows < 0 || rows < best_rows ||
                          (rows == best_rows && fill > best_fill) ||
                          (rows == best_rows && fill == best_fill && mb > c.mb);
      if (better) {
        best_rows = rows;
        best_fill = fill;
        c.mb = mb;
        best_w = w;
      }
    }
  }
  // From K = 2048, where that choice needs more than one round of 256, the
  // rows per CU mislead (the small MFMA workgroups run several to a CU):
  // there a grid of at most 320 tiles wins, else the one closest to 512
  // (K=4096 N=3072 M=384: 64 x 64, 288 tiles, 34.0 us against 44.5 with
  // 384 tiles of 48 x 64 and 39.7 with 512 of 48 x 48; N=768 M=1536 33.6
  // against 42.6; K=2048 N=3072 M=512: 64 x 48, 512 tiles, 27.0 against
  // 29.2 with 384 of 64 x 64).
  if (nk >= 32 && best_rows >= 0 && tiles(16 * c.mb, 16 * best_w) > 256) {
    int64_t pick = -1;
    for (int w = 4; w >= 3; --w) {
      if (w == 3 && !(araw && rcap <= 4)) continue;
      for (int mb = 4; mb >= 2; --mb) {
        if (mb == 3 && rcap > 4) continue;
        if (w == 3 && !(nk < 128 && tiles(16 * mb, 64) >= 128)) continue;
        const int64_t t = tiles(16 * mb, 16 * w);
        if (t > 512) continue;
        // class 0 (at most 320 tiles) before class 1, then the most tiles
        const int64_t score = (t <= 320 ? 1024 : 0) + t;
        if (score > pick) {
          pick = score;
          c.mb = mb;
          best_w = w;
        }
      }
    }
  }
  // a ring of 4 K steps measured 1-3 % faster than 3 for 32- and 48-row
  // tiles and for three-wave tiles (and slower for 64 x 64 ones); past 6
  // channels the registers hold a ring of 3 only (the tile's default)
  if (best_w == 3) c.kind = kMfma3;
  if ((c.mb < 4 || best_w == 3) && rcap <= 6) c.ks = 4;
  return c;
}

// ---------------------------------------------------------------------------
// K split over workgroups (split_exchange in rnsmx_gemm.hpp)
// ---------------------------------------------------------------------------
// Bytes of the arrival counters at the start of every workspace.
static constexpr int64_t kTicketBytes = int64_t{RNSMX_SPLIT_TICKETS} * 4;

// Steps per split for `splits` workgroups over nk K steps (the LDS kernel
// runs whole trips of its stages), and the split count that leaves no
// split empty.
static void split_steps(const GemmChoice &c, int nk, int &splits, int &kchunk) {
  const int unit = is_lds(c.kind) ? kLdsStages : 1;
  const int s = std::max(1, std::min(c.splits, nk / unit));
  kchunk = ((nk + s - 1) / s + unit - 1) / unit * unit;
  splits = (nk + kchunk - 1) / kchunk;
}

// Tiles that run whole (workgroups [0, whole) of the launch): all of them
// without a split, none with a uniform split, and with a tail split those of
// the full rounds of 256 (one workgroup per CU: the LDS kernel).
static int64_t whole_tiles(const GemmChoice &c, int64_t tiles) {
  if (c.splits <= 1) return tiles;
  if (!c.tail) return 0;
  return (tiles - 1) / 256 * 256;
}

// Whether `c` may split K: a tile built with the exchange (stream_splits,
// mfma_splits: up to 4 channels, one residue byte per channel in the
// exchange word), one wave per stream workgroup (the waves of a larger one
// already meet in LDS), and every (tile, wave) counter inside the
// workspace's fixed counter block.
static bool split_fits(const GemmChoice &c, const GemmArgs &g) {
  const int rcap = rcap_for(g.mods.channels);
  const GemmGrid gr = gemm_grid(c, g.m, g.n);
  bool built;
  if (c.kind == kStream || c.kind == kStreamWide)
    built = stream_splits(rcap, c.mb, c.nb) && c.ks == 1;
  else if (c.kind == kLdsPlanes)
    built = rcap == 4 || rcap == 6;
  else if (is_lds(c.kind))
    built = rcap <= 4;
  else
    built = mfma_splits(rcap, c.mb, c.nb);
  return built && (gr.tiles - whole_tiles(c, gr.tiles)) * gr.waves <= RNSMX_SPLIT_TICKETS;
}

// Exchange-area bytes of a choice (0 without a split).
static int64_t xchg_bytes(const GemmChoice &c, const GemmArgs &g) {
  if (c.splits <= 1) return 0;
  int splits, kchunk;
  split_steps(c, g.kp / 64, splits, kchunk);
  if (splits <= 1) return 0;
  const GemmGrid gr = gemm_grid(c, g.m, g.n);
  const int64_t parted = gr.tiles - whole_tiles(c, gr.tiles);
  const int words = (rcap_for(g.mods.channels) + 3) / 4;  // residue words per element (xchg_words)
  return round_up(parted * gr.waves * splits * gr.chunks * words * 1024, 256);
}

// The automatic split count for a choice of kernel and tile, from sweeps on
// MI355X.  A split pays only where the K loop of each tile is long and the
// grid leaves CUs idle: every split adds a fixed cost per workgroup (entry,
// first loads, a second epilogue-sized pass over the residues) and an
// exchange of R bytes per output element through the device-coherent level.
// Measured (us, 4 channels, automatic kernel unsplit -> split):
//   M=1    N=768  K=16384  57.3 -> 15.6 (8 splits)   M=256 N=256 K=8192  48.3 -> 16.4 (8)
//   M=16   N=512  K=8192   30.2 -> 10.2 (8)          M=512 N=512 K=8192  46.5 -> 25.6 (4)
//   M=256  N=768  K=4096   25.9 -> 17.9 (4)          M=128 N=4096 K=16384 104.5 -> 94.6 (2)
//   M=2048 N=768  K=16384 148 -> 128 (2)
// and it loses on the BASELINE shapes: C2 M=256 (216 tiles, 12 K steps)
// 10.3 -> 15.9 (2), C3 M=1 4.3 -> 5.5, C5 M=64 (192 tiles, 64 steps) 44.8
// -> 48.2, C5 M=512 (384 LDS tiles) 107 -> 127 (and 114 even with the
// exchange data left out: the extra workgroups' fixed cost alone).
// A split stream kernel runs one wave per workgroup, against the unsplit
// one's four waves sharing K through LDS; at decode (M=1) the one-wave
// split wins from 4 splits (N=768: K=4096 9.35 -> 8.33, K=8192 16.4 ->
// 11.1, K=16384 28.7 -> 15.7; N=256 K=4096 7.07 -> 6.53) and never with 2
// (N=768 K=2048 7.39 against 9.76).
// Rule: under 128 tiles, the largest power of two up to 8 that keeps at
// least 16 K steps per split and at most 512 workgroups (for the stream
// kernel only when that is 4 or more); 128-511 tiles of the MFMA or LDS
// kernel, 2 splits once K >= 8192; otherwise none.
// The LDS kernel runs one workgroup per CU, so its tiles go in rounds of
// 256; when the last round holds at most half that (and K is long), only
// that round's tiles are split (tail), over the CUs it would leave idle:
// C5 M=512 (384 tiles, 1.5 rounds) runs 256 whole tiles, then 128 tiles in
// two halves of K.
static int choose_splits(const GemmChoice &c, const GemmArgs &g) {
  const int nk = g.kp / 64;
  const int64_t tiles = gemm_grid(c, g.m, g.n).tiles;
  const bool stream = c.kind == kStream || c.kind == kStreamWide;
  int s = 1;
  if (c.kind == kLdsWide) return 1;  // chosen only where no tail split pays
  if (c.kind == kLdsPlanes && tiles < 256) {
    // fewer tiles than CUs: split K over as many workgroups as one round
    // holds, keeping 16 K steps per split (M=512 N=4096 K=4096: 128 tiles,
    // 84 us in two halves against 114 whole; 192 tiles split in two, 1.5
    // rounds, lose: 156 against 123)
    while (2 * s * tiles <= 256 && nk / (2 * s) >= 16 && s < 8) s *= 2;
    return s;
  }
  if (is_lds(c.kind) && tiles >= 256) {
    const int64_t last = tiles - (tiles - 1) / 256 * 256;  // tiles of the last round
    if (last <= 128 && nk >= 32) {
      const int64_t cap = std::min<int64_t>(4, 256 / last);
      while (2 * s <= cap) s *= 2;
    }
    return s;
  }
  if (tiles < 128) {
    const int64_t cap = std::min<int64_t>(std::min<int64_t>(8, 512 / tiles), nk / 16);
    while (2 * s <= cap) s *= 2;
    if (stream && s < 4) s = 1;
  } else if (!stream && tiles < 512 && nk >= 128) {
    s = 2;
  }
  return s;
}

// The automatic plan: kernel and tile (choose_gemm), then the split.  A
// stream choice that splits over workgroups runs one wave per workgroup.
static GemmChoice auto_plan(const GemmArgs &g, bool araw, bool allow_split) {
  GemmChoice c = choose_gemm(g, araw);
  if (!allow_split || (rcap_for(g.mods.channels) > 4 && c.kind != kLdsPlanes)) return c;
  GemmChoice t = c;
  if (t.kind == kStream || t.kind == kStreamWide) t.ks = 1;
  t.splits = choose_splits(c, g);
  t.tail = is_lds(t.kind) && gemm_grid(t, g.m, g.n).tiles >= 256;
  if (t.splits > 1 && split_fits(t, g)) return t;
  return c;
}

static int32_t plan_from(const rnsmx_plan_t *plan, const GemmArgs &g, bool araw, bool allow_split,
                         GemmChoice &c) {
  if (plan == nullptr || plan->kind == kAuto) {
    c = auto_plan(g, araw, allow_split);
    return RNSMX_OK;
  }
  const int k = plan->kind;
  if (k != kStream && k != kMfma && k != kLds && k != kStreamWide && k != kMfma3 && k != kLdsWide &&
      k != kLdsPlanes)
    return fail(RNSMX_EINVAL,
                "plan kind must be 0 (auto), 1 (stream), 2 (mfma), 3 (lds), 4 (wide stream), 5 (3-wave mfma), "
                "7 (wide lds) or 8 (residue-plane lds)");
  if (!is_lds(k) && (plan->mb < 1 || plan->nb < 1)) return fail(RNSMX_EINVAL, "tile blocks must be positive");
  c = GemmChoice{k, plan->mb, plan->nb, plan->ks, std::max(1, plan->splits), plan->tail != 0};
  if (c.splits > 1 && (!allow_split || !split_fits(c, g)))
    return fail(RNSMX_EINVAL, "this plan cannot split K over workgroups (channels, stream waves, or counters)");
  return RNSMX_OK;
}

// Launches the GEMM for `g` with choice `c`.  araw: A is one int8 matrix for
// all channels.  tickets / xchg: the split counters and exchange area (only
// read when c splits K).
static int32_t launch_gemm(GemmArgs g, bool araw, const GemmChoice &c, uint32_t *tickets, int8_t *xchg,
                           hipStream_t st, bool packed = false) {
  // packed weights run the capacity-4 or capacity-6 kernels only
  const int rcap = packed ? (g.mods.channels <= 4 ? 4 : 6) : rcap_for(g.mods.channels);
  if (c.kind == kStream || c.kind == kStreamWide) {
    const int cap = stream_ks_cap(rcap, c.mb, c.nb);
    if (c.ks < 1 || c.ks > cap) {
      set_error("stream GEMM needs 1 <= ks <= %d for this tile", cap);
      return RNSMX_EINVAL;
    }
  }
  g.splits = 1;
  g.kchunk = g.kp / 64;
  g.tickets = tickets;
  g.xchg = xchg;
  const int64_t tiles = gemm_grid(c, g.m, g.n).tiles;
  g.split_from = static_cast<int32_t>(tiles);
  if (c.splits > 1) {
    if (is_lds(c.kind) &&
        !(c.kind == kLdsPlanes ? lds_planes_fits(g, araw, rcap) : lds_kernel_fits(g, araw, rcap))) {
      set_error("no GEMM kernel for kind %d, tile %d x %d, %d channels", c.kind, c.mb, c.nb, g.mods.channels);
      return RNSMX_EINVAL;
    }
    split_steps(c, g.kp / 64, g.splits, g.kchunk);
    if (g.splits > 1 && (tickets == nullptr || xchg == nullptr))
      return fail(RNSMX_EINVAL, "a K split needs the workspace's counters and exchange area");
    if (g.splits > 1) g.split_from = static_cast<int32_t>(whole_tiles(c, tiles));
  }
  using PartFn = bool (*)(const GemmArgs &, bool, const GemmChoice &, hipStream_t);
#define RNSMX_PARTS(R)                                                                      \
  {                                                                                         \
    RNSMX_GEMM_PART_NAME(R, 0), RNSMX_GEMM_PART_NAME(R, 1), RNSMX_GEMM_PART_NAME(R, 2),     \
        RNSMX_GEMM_PART_NAME(R, 3), RNSMX_GEMM_PART_NAME(R, 4), RNSMX_GEMM_PART_NAME(R, 5)  \
  }
  static const PartFn parts[4][kGemmParts] = {RNSMX_PARTS(3), RNSMX_PARTS(4), RNSMX_PARTS(6),
                                              RNSMX_PARTS(10)};
#undef RNSMX_PARTS
  const int ri = rcap == 3 ? 0 : rcap == 4 ? 1 : rcap == 6 ? 2 : 3;
  if (!parts[ri][gemm_part_of(c, araw, packed)](g, araw, c, st)) {
    set_error("no GEMM kernel for kind %d, tile %d x %d, %d channels", c.kind, c.mb, c.nb,
              g.mods.channels);
    return RNSMX_EINVAL;
  }
  return check_launch(c.kind == kStream || c.kind == kStreamWide ? "gemm_stream"
                      : is_lds(c.kind)                           ? "gemm_lds"
                                                                 : "gemm_mfma");
}

// Activation encoder launch: one workgroup per (row, channel), or per row
// for the row L1 alone (e.out null), with a thread per 16 K values up to
// 256 threads (one pass up to K = 4096).
// Up to this many rows the plain residue-plane encode runs split over K.
static constexpr int64_t kEncodeSplitRows = 16;

static int32_t launch_encode_rows(int32_t dtype, const EncodeArgs &e, hipStream_t st, bool packed = false) {
  if (e.rows == 0) return RNSMX_OK;
  if (!packed && e.out != nullptr && e.row_l1 == nullptr && e.absmax == nullptr && e.rows <= kEncodeSplitRows) {
    const dim3 grid(static_cast<unsigned>(e.rows), static_cast<unsigned>(e.mods.channels),
                    static_cast<unsigned>((e.out_ld + 1023) / 1024));
    switch (dtype) {
      case RNSMX_INT8: hipLaunchKernelGGL(encode_rows_split_kernel<int8_t>, grid, dim3(256), 0, st, e); break;
      case RNSMX_INT16: hipLaunchKernelGGL(encode_rows_split_kernel<int16_t>, grid, dim3(256), 0, st, e); break;
      case RNSMX_INT32: hipLaunchKernelGGL(encode_rows_split_kernel<int32_t>, grid, dim3(256), 0, st, e); break;
      default: return fail(RNSMX_EINVAL, "encoder supports int8, int16 and int32");
    }
    return check_launch("encode_rows_split");
  }
  const int64_t chunks = (e.out_ld + 15) / 16;
  const unsigned threads = static_cast<unsigned>(std::min<int64_t>(256, (chunks + 63) / 64 * 64));
  const dim3 grid(static_cast<unsigned>(e.rows), e.out != nullptr ? static_cast<unsigned>(e.mods.channels) : 1u);
  const dim3 block(threads);
#define RNSMX_ENCODE_ROWS(T)                                                            \
  if (packed)                                                                           \
    hipLaunchKernelGGL((encode_rows_kernel<T, true>), grid, block, 0, st, e);          \
  else                                                                                  \
    hipLaunchKernelGGL((encode_rows_kernel<T, false>), grid, block, 0, st, e);
  switch (dtype) {
    case RNSMX_INT8: RNSMX_ENCODE_ROWS(int8_t) break;
    case RNSMX_INT16: RNSMX_ENCODE_ROWS(int16_t) break;
    case RNSMX_INT32: RNSMX_ENCODE_ROWS(int32_t) break;
    default: return fail(RNSMX_EINVAL, "encoder supports int8, int16 and int32");
  }
#undef RNSMX_ENCODE_ROWS
  return check_launch("encode_rows");
}

// Kernel choice for packed weights: the stream kernel wherever the
// automatic choice takes it (tiles of 16 or 32 rows, K over up to 4
// waves), else the MFMA kernel with 32- or 64-row tiles, whichever leaves
// fewer rows on a CU (rounds of 256 workgroups times the tile height;
// 64 rows on a tie); never split over workgroups.
// Packed weights at decode: rows_packed_kernel for up to 8 blocks of
// 16 / R tokens (R = 4 or 6 channel rows each; the fewest blocks, a power
// of two, that hold M) while its sums fit int32 (K * 384 * 127 for moduli
// up to 255).
static constexpr int kRowsMaxKp = 44032;
static constexpr int kRowsMaxBlocks = 8;

static int rows_steps_of(int nblk) { return nblk == 1 ? 8 : nblk == 2 ? 4 : 2; }

static GemmChoice packed_auto(const GemmArgs &g) {
  const int rcap = g.mods.channels <= 4 ? 4 : 6;
  const int tpb = 16 / rcap;
  if (g.m <= kRowsMaxBlocks * tpb && g.kp <= kRowsMaxKp) {
    int nblk = 1;
    while (nblk * tpb < g.m) nblk *= 2;
    const int u = rows_steps_of(nblk);
    return GemmChoice{kRows, nblk, 1, std::min(4, std::max(1, (g.kp / 64 + u - 1) / u)), 1, 0};
  }
  GemmChoice c = choose_gemm(g, false, true);
  c.splits = 1;
  c.tail = 0;
  // the residue-plane LDS kernel with two units per channel (a' x hi, a x
  // lo) under the rule and split of residue-plane weights
  const int64_t pl_tiles = static_cast<int64_t>((g.m + kPlBM - 1) / kPlBM) * ((g.n + kPlBN - 1) / kPlBN);
  if (g.m >= 64 && lds_planes_fits(g, false, rcap) && (pl_tiles * (g.kp / 64) >= 4096 || pl_tiles >= 128)) {
    const int64_t tiles = pl_tiles;
    GemmChoice t{kLdsPlanes, 0, 0, 0, 1, tiles >= 256};
    t.splits = choose_splits(t, g);
    if (t.splits > 1 && split_fits(t, g)) return t;
    return GemmChoice{kLdsPlanes, 0, 0, 0, 1, 0};
  }
  c.nb = 1;
  if (c.kind == kStream || c.kind == kStreamWide) {
    c.kind = kStream;
    // past 16 rows 32-row tiles: the 2R activation planes of a step serve
    // twice the rows (K=4096 N=4096 M=32, 6 channels: 64.0 us against 83.8)
    c.mb = g.m > 16 ? 2 : 1;
    const int u = stream_u_of(rcap, false, c.mb, 1, 4, true);
    c.ks = std::min(stream_ks_cap(rcap, c.mb, 1), std::max(1, (g.kp / 64 + u - 1) / u));
    return c;
  }
  auto rows_per_cu = [&](int mb) {
    const int64_t t = static_cast<int64_t>((g.m + 16 * mb - 1) / (16 * mb)) * ((g.n + 63) / 64);
    return (t + 255) / 256 * 16 * mb;
  };
  // 32-row tiles on a tie in rows per CU up to three rounds of them (6
  // channels, K=768 N=2304 M=256: 36.0 us against 50.3 with 64-row tiles)
  const bool few = static_cast<int64_t>((g.m + 31) / 32) * ((g.n + 63) / 64) <= 768;
  c.kind = kMfma;
  c.mb = rows_per_cu(2) < rows_per_cu(4) || (few && rows_per_cu(2) == rows_per_cu(4)) ? 2 : 4;
  c.ks = 0;
  return c;
}

static int32_t packed_plan_from(const rnsmx_plan_t *plan, const GemmArgs &g, GemmChoice &c) {
  if (plan == nullptr || plan->kind == kAuto) {
    c = packed_auto(g);
    return RNSMX_OK;
  }
  const bool stream = plan->kind == kStream && (plan->mb == 1 || plan->mb == 2) && plan->nb == 1;
  const bool mfma = plan->kind == kMfma && (plan->mb == 2 || plan->mb == 4) && plan->nb == 1;
  const bool rows = plan->kind == kRows && (plan->mb == 1 || plan->mb == 2 || plan->mb == 4 || plan->mb == 8) &&
                    plan->nb == 1 && plan->ks >= 1 && plan->ks <= 4;
  const bool lds = plan->kind == kLdsPlanes;
  if (!(stream || mfma || rows || lds) || (!lds && (plan->splits > 1 || plan->tail != 0)))
    return fail(RNSMX_EINVAL, "packed weights run the stream kernel (16- or 32-row tiles), the MFMA kernel "
                              "(32- or 64-row tiles), the channel-row kernel (1, 2, 4 or 8 token blocks) or the "
                              "residue-plane LDS kernel (kind 8), one column block, K split over "
                              "workgroups only by the LDS kernel");
  if (rows) {
    const int tpb = 16 / (g.mods.channels <= 4 ? 4 : 6);
    if (g.m > plan->mb * tpb) return fail(RNSMX_EINVAL, "channel-row plan: more tokens than its blocks hold");
    if (g.kp * int64_t{384} * max_half(g.mods) > INT32_MAX)
      return fail(RNSMX_ERANGE, "channel-row plan: K * 384 * max(floor(m/2)) exceeds the int32 sums");
  }
  c = GemmChoice{plan->kind, plan->mb, 1, stream || rows ? plan->ks : 0, std::max(1, plan->splits), plan->tail != 0};
  if (c.splits > 1 && !split_fits(c, g))
    return fail(RNSMX_EINVAL, "this plan cannot split K over workgroups (channels or counters)");
  return RNSMX_OK;
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

// ---------------------------------------------------------------------------
// Per-tensor symmetric quantization of activations: RNSLinear's
// _symmetric_scale + _quantize (src/rns_llm/layers/rns_linear.py:154-166)
// in two launches instead of a chain of elementwise and reduction ops.
//   scale = max(amax|x| * fl32(1 / qmax), eps_f32)   (the GPU reference
//           divides by the Python float qmax as a multiply by its float
//           reciprocal)
//   q     = clamp(rint(x / scale), -qmax, qmax)      (correctly rounded
//           division: tensor / tensor)
// The amax pass writes one maximum per block (at most 256 blocks) into the
// scratch; every block of the quantize pass folds them
// again (a few hundred floats from L2) and derives the same scale, so no
// atomics or last-block logic are needed and the scratch carries nothing
// from one call to the next.  Both passes read 16 bytes per lane when the
// activations are 16-byte aligned.
// ---------------------------------------------------------------------------
// Inputs up to this many elements are quantized by one workgroup in one
// launch (quant_one_block_kernel); larger ones take two launches.  One
// workgroup is bound by the correctly rounded divisions (measured on
// MI355X, fp16: 768 values 2.2 us, 12 K 3.7 us, 98 K 16.5 us, against
// 5.5 us for 393 K in two launches), while a launch costs the host about
// 3 us: below this size the saved launch is worth more.
static constexpr int64_t kQuantOneBlockMax = 16384;

struct QuantArgs {
  const void *x;
  int64_t count;
  int32_t vec;      // 1: x is 16-byte aligned, read in 16-byte vectors
  int32_t nparts;   // blocks of the amax pass
  float qmax, rcp;  // rcp = fl32(1 / qmax)
  float *partial;
  float *scale;
  void *q;
};

// Input element decoding: float32, or the bits of a float16 / bfloat16.
template <typename T>
struct QuantIn;
template <>
struct QuantIn<float> {
  __device__ static float get(float v) { return v; }
};
struct Bf16Bits {
  uint16_t bits;
};
template <>
struct QuantIn<__half> {
  __device__ static float get(uint16_t v) { return __half2float(__ushort_as_half(v)); }
};
template <>
struct QuantIn<Bf16Bits> {
  __device__ static float get(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }
};
template <typename T>
using QuantRaw = typename std::conditional<std::is_same<T, float>::value, float, uint16_t>::type;



// max(a, b) that propagates NaN, as torch's amax does (fmaxf drops it).
__device__ __forceinline__ float max_nan(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}

// max |x| over the elements this thread visits (tid, tid + stride, ...);
// NaN when any of them is NaN.
template <typename T>
__device__ __forceinline__ float quant_thread_amax(const QuantArgs &a, int64_t tid, int64_t stride) {
  using R = QuantRaw<T>;
  constexpr int V = 16 / sizeof(R);
  const R *x = static_cast<const R *>(a.x);
  const int64_t nvec = a.vec ? a.count / V : 0;
  float m = 0.0f;
  bool nan = false;
  auto visit = [&](float v) {
    m = fmaxf(m, fabsf(v));
    nan |= v != v;
  };
  for (int64_t i = tid; i < nvec; i += stride) {
    R v[V];
    *reinterpret_cast<uint4 *>(v) = reinterpret_cast<const uint4 *>(x)[i];
    static_for<V>([&](auto E) { visit(QuantIn<T>::get(v[decltype(E)::value])); });
  }
  for (int64_t i = nvec * V + tid; i < a.count; i += stride) visit(QuantIn<T>::get(x[i]));
  return nan ? __builtin_nanf("") : m;
}

// q = clamp(rint(x / s), -qmax, qmax) over the elements of (tid, stride).
template <typename T, typename Q>
__device__ __forceinline__ void quant_thread_apply(const QuantArgs &a, float s, int64_t tid, int64_t stride) {
  using R = QuantRaw<T>;
  constexpr int V = 16 / sizeof(R);
  const R *x = static_cast<const R *>(a.x);
  Q *q = static_cast<Q *>(a.q);
  // a NaN quotient (x NaN, s NaN, or x and s infinite) quantizes to 0, the
  // value the hardware's float-to-integer conversion gives NaN
  auto quant = [&](R raw) {
    const float r = rintf(QuantIn<T>::get(raw) / s);
    return static_cast<Q>(r != r ? 0.0f : fminf(fmaxf(r, -a.qmax), a.qmax));
  };
  const int64_t nvec = a.vec ? a.count / V : 0;
  for (int64_t i = tid; i < nvec; i += stride) {
    R v[V];
    *reinterpret_cast<uint4 *>(v) = reinterpret_cast<const uint4 *>(x)[i];
    Q o[V];
    static_for<V>([&](auto E) { o[decltype(E)::value] = quant(v[decltype(E)::value]); });
    // V outputs: 4-16 bytes, aligned to their size (q is 16-byte aligned)
    if constexpr (sizeof(o) == 16)
      reinterpret_cast<uint4 *>(q)[i] = *reinterpret_cast<const uint4 *>(o);
    else if constexpr (sizeof(o) == 8)
      reinterpret_cast<uint2 *>(q)[i] = *reinterpret_cast<const uint2 *>(o);
    else
      reinterpret_cast<uint32_t *>(q)[i] = *reinterpret_cast<const uint32_t *>(o);
  }
  for (int64_t i = nvec * V + tid; i < a.count; i += stride) q[i] = quant(x[i]);
}

// Block-wide max of non-negative floats or NaN (256 threads; NaN wins).
__device__ __forceinline__ float block_max256(float m, float *wmax) {
  for (int off = 32; off > 0; off >>= 1) m = max_nan(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  return max_nan(max_nan(wmax[0], wmax[1]), max_nan(wmax[2], wmax[3]));
}

template <typename T>
__global__ __launch_bounds__(256) void quant_amax_kernel(const QuantArgs a) {
  __shared__ float wmax[4];
  float m = quant_thread_amax<T>(a, static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x,
                                 static_cast<int64_t>(gridDim.x) * blockDim.x);
  m = block_max256(m, wmax);
  if (threadIdx.x == 0) a.partial[blockIdx.x] = m;
}

template <typename T, typename Q>
__global__ __launch_bounds__(256) void quant_apply_kernel(const QuantArgs a) {
  __shared__ float wmax[4];
  float t = 0.0f;
  for (int b = threadIdx.x; b < a.nparts; b += blockDim.x) t = max_nan(t, a.partial[b]);
  const float amax = block_max256(t, wmax);
  // clamp at FLT_EPSILON; NaN stays NaN (torch.clamp keeps it, fmaxf would not)
  const float s = amax != amax ? amax : fmaxf(amax * a.rcp, 1.1920928955078125e-07f);
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale = s;
  quant_thread_apply<T, Q>(a, s, static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x,
                           static_cast<int64_t>(gridDim.x) * blockDim.x);
}

// Small inputs in one launch: one workgroup of 1024 threads takes the
// maximum over every element, then quantizes them (a second launch costs
// more host time than these few kilobytes cost the one workgroup).
template <typename T, typename Q>
__global__ __launch_bounds__(1024) void quant_one_block_kernel(const QuantArgs a) {
  __shared__ float wmax[16];
  float m = quant_thread_amax<T>(a, threadIdx.x, blockDim.x);
  for (int off = 32; off > 0; off >>= 1) m = max_nan(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  float amax = 0.0f;
  for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) amax = max_nan(amax, wmax[w]);
  // clamp at FLT_EPSILON; NaN stays NaN (torch.clamp keeps it, fmaxf would not)
  const float s = amax != amax ? amax : fmaxf(amax * a.rcp, 1.1920928955078125e-07f);
  if (threadIdx.x == 0) *a.scale = s;
  quant_thread_apply<T, Q>(a, s, threadIdx.x, blockDim.x);
}

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
  if (rows > INT32_MAX) return fail(RNSMX_EINVAL, "padded encode takes fewer than 2^31 rows");
  e.rows = rows;
  e.cols = cols;
  e.out_ld = out_ld;
  e.plane = rows * out_ld;
  return launch_encode_rows(dtype, e, st);
}

// The fields of GemmArgs the kernel choice reads, for an M x N x K product
// (raw int8 activations read in place with row stride K, or residue planes
// padded to kp).
static GemmArgs plan_args(int64_t m, int64_t n, int64_t k, int32_t channels, bool araw) {
  GemmArgs g{};
  g.m = static_cast<int32_t>(m);
  g.n = static_cast<int32_t>(n);
  g.kp = static_cast<int32_t>(round_up(std::max<int64_t>(k, 1), RNSMX_K_ALIGN));
  g.a_k = araw ? static_cast<int32_t>(k) : g.kp;
  g.a_ld = araw ? k : g.kp;
  g.mods.channels = channels;
  return g;
}

// Drop-in op workspace: [split counters][A padded to kp (when needed)]
// [B repacked fragment-major][split exchange].
struct FusedLayout {
  int64_t a_pad, b_nk, xchg, total;
};

static FusedLayout fused_layout(int64_t m, int64_t kp, int64_t n, int32_t channels, int64_t xchg) {
  FusedLayout l{};
  l.a_pad = kTicketBytes;
  l.b_nk = l.a_pad + round_up(channels * m * kp, 256);
  l.xchg = l.b_nk + round_up(channels * ((n + 15) / 16) * 16 * kp, 256);
  l.total = l.xchg + xchg;
  return l;
}

int64_t rnsmx_fused_workspace_bytes(int64_t m, int64_t k, int64_t n, int32_t channels) {
  if (m < 0 || k < 0 || n < 0 || channels < 1 || channels > RNSMX_MAX_CHANNELS) return -1;
  const int64_t kp = round_up(std::max<int64_t>(k, 1), RNSMX_K_ALIGN);
  int64_t xchg = 0;
  if (m > 0 && n > 0 && m <= INT32_MAX && n <= INT32_MAX) {
    const GemmArgs g = plan_args(m, n, k, channels, false);
    xchg = xchg_bytes(auto_plan(g, false, true), g);
  }
  return fused_layout(m, kp, n, channels, xchg).total;
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
  GemmArgs g = plan_args(m, n, k, R, false);
  g.mods = *mods;
  const GemmChoice c = auto_plan(g, false, true);
  const FusedLayout l = fused_layout(m, kp, n, R, xchg_bytes(c, g));
  int8_t *ws = static_cast<int8_t *>(workspace_dev);
  uint32_t *tickets = reinterpret_cast<uint32_t *>(ws);
  const int8_t *a_use = a_dev;
  int64_t a_ld = k, a_k = k;
  int8_t *b_nk = ws + l.b_nk;
  if (k % 16 != 0 || !aligned16(a_dev)) {
    // rows of 16-byte chunks are read straight from the caller's planes
    // otherwise (chunks past K load as zero)
    int8_t *a_pad = ws + l.a_pad;
    const int64_t total = R * static_cast<int64_t>(m) * kp;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 16384));
    hipLaunchKernelGGL(pad_rows_kernel, dim3(blocks), dim3(256), 0, st, a_dev, static_cast<int64_t>(m),
                       static_cast<int64_t>(k), kp, total, a_pad);
    if (int32_t rc = check_launch("pad_rows")) return rc;
    a_use = a_pad;
    a_ld = kp;
    a_k = kp;
  }
  const int64_t n16 = (n + 15) / 16, nk = kp / 64;
  {
    const int64_t total = R * n16 * nk * 64;
    const GemmGrid gr = gemm_grid(c, m, n);
    const int64_t ntickets = c.splits > 1 ? (gr.tiles - whole_tiles(c, gr.tiles)) * gr.waves : 0;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 16384));
    hipLaunchKernelGGL(transpose_frag_kernel, dim3(blocks), dim3(256), 0, st, b_dev, static_cast<int64_t>(k),
                       static_cast<int64_t>(n), n16, nk, total, b_nk, tickets, ntickets);
    if (int32_t rc = check_launch("transpose_frag")) return rc;
  }
  g.a = a_use;
  g.a_ld = a_ld;
  g.a_cs = a_ld * m;
  g.a_k = static_cast<int32_t>(a_k);
  g.b = b_nk;
  g.b_ld = kp * 16;
  g.b_cs = kp * 16 * n16;
  g.min_channels = 0;
  g.out = out_dev;
  g.out_ld = n;
  g.out_dtype = RNSMX_INT64;
  return launch_gemm(g, false, c, tickets, ws + l.xchg, st);
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
  const int64_t n16 = (static_cast<int64_t>(n) + 15) / 16;
  EncodeArgs e{};
  e.values = b_nk_dev;
  e.rows = n;
  e.cols = k;
  e.out_ld = kp;
  e.plane = n16 * kp * 16;
  e.out = packed_dev;
  e.row_l1 = nullptr;
  e.absmax = absmax_dev;
  e.mods = *mods;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((n16 + 3) / 4)), block(256);
  switch (dtype) {
    case RNSMX_INT8: hipLaunchKernelGGL(encode_frag_kernel<int8_t>, grid, block, 0, st, e); break;
    case RNSMX_INT16: hipLaunchKernelGGL(encode_frag_kernel<int16_t>, grid, block, 0, st, e); break;
    default: hipLaunchKernelGGL(encode_frag_kernel<int32_t>, grid, block, 0, st, e); break;
  }
  return check_launch("encode_frag");

}

int32_t rnsmx_prepare_weight_packed(const void *b_nk_dev, int32_t dtype, int32_t n, int32_t k, int8_t *packed_dev,
                                    int32_t *absmax_dev, void *stream) {
  clear_error();
  if (n < 0 || k < 1) return fail(RNSMX_EINVAL, "bad weight shape");
  if (dtype != RNSMX_INT8 && dtype != RNSMX_INT16) return fail(RNSMX_EINVAL, "packed weights take int8 or int16 values");
  if (n == 0) return RNSMX_OK;
  if (!b_nk_dev || !packed_dev) return fail(RNSMX_EINVAL, "null tensor pointer");
  if (!aligned16(b_nk_dev) || !aligned16(packed_dev))
    return fail(RNSMX_EINVAL, "weight buffers must be 16-byte aligned");
  const int64_t kp = round_up(k, RNSMX_K_ALIGN);
  const int64_t n16 = (static_cast<int64_t>(n) + 15) / 16;
  EncodeArgs e{};
  e.values = b_nk_dev;
  e.rows = n;
  e.cols = k;
  e.out_ld = kp;
  e.plane = n16 * kp * 16;
  e.out = packed_dev;
  e.absmax = absmax_dev;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((n16 + 3) / 4)), block(256);
  if (dtype == RNSMX_INT8)
    hipLaunchKernelGGL(pack_frag_kernel<int8_t>, grid, block, 0, st, e);
  else
    hipLaunchKernelGGL(pack_frag_kernel<int16_t>, grid, block, 0, st, e);
  return check_launch("pack_frag");
}

// Prepared-path workspace: [split counters][activation residue planes
// (only when A is not read in place)][row L1 norms][split exchange].  Only
// the counters sit at a fixed place; the rest is rewritten by every call.
struct PreparedLayout {
  int64_t a_res, row_l1, xchg, total;
};

static PreparedLayout prepared_layout(bool araw, int64_t m, int64_t kp, int32_t channels, int64_t xchg) {
  PreparedLayout l{};
  l.a_res = kTicketBytes;
  l.row_l1 = l.a_res + (araw ? 0 : round_up(channels * m * kp, 256));
  l.xchg = l.row_l1 + round_up(8 * (m + 1), 256);  // the norms, then their maximum
  l.total = l.xchg + xchg;
  return l;
}

// Packed-weight workspace: [split counters (unused: never split)][2R
// activation planes, then the int32 row terms [R][packed_corr_ld(M)]; or
// (up to 32 tokens) 8 blocks of channel-row fragments][row L1 norms].
static PreparedLayout packed_layout(int64_t m, int64_t kp, int32_t channels, int64_t xchg) {
  PreparedLayout l{};
  l.a_res = kTicketBytes;
  // per-channel planes, or (up to 8 tokens) two blocks of channel-row fragments
  const int64_t planes = 2 * channels * m * kp + 4 * channels * packed_corr_ld(m);
  const int64_t rows = m <= kRowsMaxBlocks * 4 ? int64_t{kRowsMaxBlocks} * 2 * kp * 16 : 0;
  l.row_l1 = l.a_res + round_up(std::max(planes, rows), 256);
  l.xchg = l.row_l1 + round_up(8 * (m + 1), 256);  // the norms, then their maximum
  l.total = l.xchg + xchg;
  return l;
}

// Workspace bytes of one prepared-path call shape and plan, for A read in
// place (araw) or as residue planes.
static int64_t prepared_need(bool araw, int64_t m, int64_t k, int64_t n, int32_t channels,
                             const rnsmx_plan_t *plan) {
  const int64_t kp = round_up(std::max<int64_t>(k, 1), RNSMX_K_ALIGN);
  int64_t xchg = 0;
  if (m > 0 && n > 0) {
    const GemmArgs g = plan_args(m, n, k, channels, araw);
    GemmChoice c{};
    if (plan_from(plan, g, araw, true, c) == RNSMX_OK) xchg = xchg_bytes(c, g);
  }
  return prepared_layout(araw, m, kp, channels, xchg).total;
}

int64_t rnsmx_prepared_workspace_bytes(int64_t m, int64_t k, int64_t n, int32_t channels,
                                       const rnsmx_plan_t *plan) {
  if (m < 0 || k < 0 || n < 0 || channels < 1 || channels > RNSMX_MAX_CHANNELS || m > INT32_MAX ||
      n > INT32_MAX || k > INT32_MAX - 63)
    return -1;
  return std::max(prepared_need(true, m, k, n, channels, plan), prepared_need(false, m, k, n, channels, plan));
}

// The prepared-weight product for both weight forms: residue planes
// (rnsmx_prepare_weight) or packed bytes (rnsmx_prepare_weight_packed).
static int32_t run_prepared(const void *a_dev, int32_t a_dtype, int32_t m, int32_t k, int32_t n,
                            const int8_t *packed_dev, const rnsmx_moduli_t *mods, const int16_t *lut_dev,
                            int32_t lut_channels, const rnsmx_adaptive_t *adaptive,
                            const rnsmx_epilogue_t *epilogue, const rnsmx_plan_t *plan, void *workspace_dev,
                            int64_t workspace_bytes, void *out_dev, void *stream, bool packed) {
  clear_error();
  if (!mods || mods->channels < 1) return fail(RNSMX_EINVAL, "moduli are not initialised");
  if (m < 0 || k < 1 || n < 0) return fail(RNSMX_EINVAL, "bad GEMM shape");
  if (dtype_size(a_dtype) == 0) return fail(RNSMX_EINVAL, "a must be int8/int16/int32");
  if (lut_channels < 0 || lut_channels > 2 || lut_channels > mods->channels)
    return fail(RNSMX_EINVAL, "lut_channels must be 0, 1 or 2 and <= channel count");
  if (lut_channels > 0 && !lut_dev) return fail(RNSMX_EINVAL, "lut_channels > 0 needs the LUT");
  if (packed && mods->channels > kPackedMaxChannels)
    return fail(RNSMX_EINVAL, "packed weights take at most 6 channels");
  if (packed ? !packed_accumulator_fits(*mods, k) : !accumulator_fits(*mods, k))
    return fail(RNSMX_ERANGE, packed ? "2 * K * 128 * max(floor(m/2)) exceeds the int32 accumulator"
                                     : "K * max(floor(m/2))^2 exceeds the int32 accumulator");
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
  if (!aligned16(a_dev)) return fail(RNSMX_EINVAL, "activations must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int R = mods->channels;
  const int64_t kp = round_up(k, RNSMX_K_ALIGN);

  // int8 activations with 16-byte rows feed the MFMA directly (they are
  // their own representatives mod every m_c); the encoder then only runs for
  // the adaptive row L1 norms.  Other sources are encoded to residue planes.
  const bool araw = !packed && a_dtype == RNSMX_INT8 && k % 16 == 0 && raw_accumulator_fits(*mods, k);
  GemmArgs g = plan_args(m, n, k, R, araw);
  g.mods = *mods;
  GemmChoice c{};
  if (int32_t rc = packed ? packed_plan_from(plan, g, c) : plan_from(plan, g, araw, true, c)) return rc;
  const PreparedLayout l = packed ? packed_layout(m, kp, R, xchg_bytes(c, g))
                                  : prepared_layout(araw, m, kp, R, xchg_bytes(c, g));
  if (workspace_bytes < l.total) {
    set_error("workspace too small: %lld < %lld bytes", static_cast<long long>(workspace_bytes),
              static_cast<long long>(l.total));
    return RNSMX_ESPACE;
  }
  int8_t *ws = static_cast<int8_t *>(workspace_dev);
  int8_t *a_res = ws + l.a_res;
  int64_t *row_l1 = reinterpret_cast<int64_t *>(ws + l.row_l1);
  // With a few raw rows the GEMM workgroups sum the adaptive row norms
  // themselves (each reads the rows: a few KB from L2), which saves the
  // encoder launch: C5 adaptive M=1 44 -> 39 us.
  const bool l1_in_gemm = araw && min_ch != 0 && m <= kAdaptiveRowsInGemm;
  const bool l1_fold = araw && min_ch != 0 && !l1_in_gemm && m > kAdaptiveFoldInGemm;
  // row_l1_max_kernel's workgroups: their maxima are the words the GEMM folds
  const int l1_groups = static_cast<int>(std::min<int64_t>((m + 3) / 4, kAdaptiveFoldInGemm));
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
  const bool rows = packed && c.kind == kRows;
  if (rows) {
    TokenRowsArgs t{};
    t.values = a_dev;
    t.m = m;
    t.cols = k;
    t.nk = kp / 64;
    t.rpt = R <= 4 ? 4 : 6;
    t.blocks = c.mb;
    t.out = a_res;
    t.mods = *mods;
    const int64_t frags = t.blocks * 2 * t.nk;  // one workgroup per 1 KB fragment
    const dim3 grid(static_cast<unsigned>(frags)), block(256);
    switch (a_dtype) {
      case RNSMX_INT8: hipLaunchKernelGGL(encode_token_rows_kernel<int8_t>, grid, block, 0, st, t); break;
      case RNSMX_INT16: hipLaunchKernelGGL(encode_token_rows_kernel<int16_t>, grid, block, 0, st, t); break;
      default: hipLaunchKernelGGL(encode_token_rows_kernel<int32_t>, grid, block, 0, st, t); break;
    }
    if (int32_t rc = check_launch("encode_token_rows")) return rc;
    if (min_ch != 0) {  // the row norms of the adaptive bound
      EncodeArgs l1 = e;
      l1.out = nullptr;
      if (int32_t rc = launch_encode_rows(a_dtype, l1, st)) return rc;
    }
  } else if (packed) {
    if (int32_t rc = launch_encode_rows(a_dtype, e, st, true)) return rc;
  } else if (l1_fold) {
    hipLaunchKernelGGL(row_l1_max_kernel, dim3(static_cast<unsigned>(l1_groups)), dim3(256), 0, st, e);
    if (int32_t rc = check_launch("row_l1_max")) return rc;
  } else if (!araw || (min_ch != 0 && !l1_in_gemm)) {
    if (int32_t rc = launch_encode_rows(a_dtype, e, st)) return rc;
  }

  if (araw) {
    g.a = static_cast<const int8_t *>(a_dev);
    g.a_cs = 0;
  } else {
    g.a = a_res;
    g.a_cs = rows ? 2 * kp * 16 : kp * m;  // channel-row fragments: bytes per token block
  }
  g.b = packed_dev;
  g.b_ld = kp * 16;
  g.b_cs = kp * 16 * ((n + 15) / 16);  // per channel, or per byte plane of packed weights
  g.min_channels = min_ch;
  // the norms, or the maximum the encoder folded
  g.row_l1 = l1_in_gemm ? nullptr : row_l1;
  g.l1_rows = l1_fold ? l1_groups : m;
  g.w_absmax = min_ch != 0 ? adaptive->w_absmax_dev : nullptr;
  g.meta = min_ch != 0 ? adaptive->meta_dev : nullptr;
  g.out = out_dev;
  g.out_ld = n;
  g.out_dtype = out_dtype;
  g.a_scale = epilogue ? epilogue->a_scale_dev : nullptr;
  g.w_scale = epilogue ? epilogue->w_scale_dev : nullptr;
  g.bias = epilogue ? epilogue->bias_dev : nullptr;
  return launch_gemm(g, araw, c, reinterpret_cast<uint32_t *>(ws), ws + l.xchg, st, packed);
}

int64_t rnsmx_packed_workspace_bytes(int64_t m, int64_t k, int64_t n, int32_t channels,
                                     const rnsmx_plan_t *plan) {
  if (m < 0 || k < 0 || n < 0 || channels < 1 || channels > kPackedMaxChannels || m > INT32_MAX ||
      n > INT32_MAX || k > INT32_MAX - 63)
    return -1;
  const GemmArgs g = plan_args(std::max<int64_t>(m, 1), std::max<int64_t>(n, 1), std::max<int64_t>(k, 1), channels,
                               false);
  GemmChoice c{};
  if (packed_plan_from(plan, g, c) != RNSMX_OK) return -1;
  return packed_layout(m, g.kp, channels, xchg_bytes(c, g)).total;
}

int32_t rnsmx_matmul_prepared_fused(const void *a_dev, int32_t a_dtype, int32_t m, int32_t k, int32_t n,
                                    const int8_t *packed_dev, const rnsmx_moduli_t *mods,
                                    const int16_t *lut_dev, int32_t lut_channels,
                                    const rnsmx_adaptive_t *adaptive, const rnsmx_epilogue_t *epilogue,
                                    const rnsmx_plan_t *plan, void *workspace_dev, int64_t workspace_bytes,
                                    void *out_dev, void *stream) {
  return run_prepared(a_dev, a_dtype, m, k, n, packed_dev, mods, lut_dev, lut_channels, adaptive, epilogue, plan,
                      workspace_dev, workspace_bytes, out_dev, stream, false);
}

int32_t rnsmx_matmul_packed_fused(const void *a_dev, int32_t a_dtype, int32_t m, int32_t k, int32_t n,
                                  const int8_t *packed_dev, const rnsmx_moduli_t *mods,
                                  const int16_t *lut_dev, int32_t lut_channels,
                                  const rnsmx_adaptive_t *adaptive, const rnsmx_epilogue_t *epilogue,
                                  const rnsmx_plan_t *plan, void *workspace_dev, int64_t workspace_bytes,
                                  void *out_dev, void *stream) {
  return run_prepared(a_dev, a_dtype, m, k, n, packed_dev, mods, lut_dev, lut_channels, adaptive, epilogue, plan,
                      workspace_dev, workspace_bytes, out_dev, stream, true);
}

// Device address of `scratch` on the current device, resolved once per
// device (each GPU holds its own copy of the array at its own address; the
// host-side name is only a stand-in and is never passed to a kernel).  The
// first resolution on a device also clears the counters on `st`.
static int32_t static_scratch(hipStream_t st, int8_t **out) {
  constexpr int kMaxDevices = 64;
  static std::mutex lock;
  static int8_t *ptr[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(RNSMX_ELAUNCH, "no current HIP device for the static scratch");
  std::lock_guard<std::mutex> guard(lock);
  if (ptr[dev] == nullptr) {
    void *p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(err));
      return RNSMX_ELAUNCH;
    }
    hipLaunchKernelGGL(fill_zero_kernel, dim3(16), dim3(256), 0, st, static_cast<uint32_t *>(p),
                       static_cast<int64_t>(RNSMX_SPLIT_TICKETS));
    if (int32_t rc = check_launch("fill_zero")) return rc;
    ptr[dev] = static_cast<int8_t *>(p);
  }
  *out = ptr[dev];
  return RNSMX_OK;
}

int32_t rnsmx_matmul_prepared_fused_noalloc(const void *a_dev, int32_t a_dtype, int32_t m, int32_t k, int32_t n,
                                            const int8_t *packed_dev, const rnsmx_moduli_t *mods,
                                            const int16_t *lut_dev, int32_t lut_channels,
                                            const rnsmx_adaptive_t *adaptive, const rnsmx_epilogue_t *epilogue,
                                            const rnsmx_plan_t *plan, void *out_dev, void *stream) {
  clear_error();
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (m == 0 || n == 0 || m < 0 || n < 0 || k < 1 || !mods || mods->channels < 1 ||
      mods->channels > RNSMX_MAX_CHANNELS || dtype_size(a_dtype) == 0)
    // nothing to launch, or an argument error: the workspace entry point
    // returns it (an empty call, or the same status) without touching the GPU
    return rnsmx_matmul_prepared_fused(a_dev, a_dtype, m, k, n, packed_dev, mods, lut_dev, lut_channels,
                                       adaptive, epilogue, plan, nullptr, 0, out_dev, stream);
  // The plan this call runs, checked on the host.  The automatic plan may
  // split K over workgroups, whose exchange area can outgrow the static
  // scratch where the same product unsplit fits (an LDS-kernel tail split
  // at K = 4096, N = 12288 needs 16 MiB of exchange); it then runs unsplit.
  const bool araw = a_dtype == RNSMX_INT8 && k % 16 == 0 && raw_accumulator_fits(*mods, k);
  const GemmArgs g = plan_args(m, n, k, mods->channels, araw);
  const int64_t kp = round_up(k, RNSMX_K_ALIGN);
  GemmChoice c{};
  if (int32_t rc = plan_from(plan, g, araw, true, c)) return rc;
  rnsmx_plan_t own{};
  const rnsmx_plan_t *run_plan = plan;
  int64_t need = prepared_layout(araw, m, kp, mods->channels, xchg_bytes(c, g)).total;
  if (need > RNSMX_NOALLOC_SCRATCH_BYTES && (plan == nullptr || plan->kind == kAuto)) {
    c = auto_plan(g, araw, false);
    own = rnsmx_plan_t{c.kind, c.mb, c.nb, c.ks, 1, 0};
    run_plan = &own;
    need = prepared_layout(araw, m, kp, mods->channels, 0).total;
  }
  if (need > RNSMX_NOALLOC_SCRATCH_BYTES) {
    set_error("this call needs %lld bytes of scratch; the static scratch holds %lld (use "
              "rnsmx_matmul_prepared_fused with a workspace)",
              static_cast<long long>(need), static_cast<long long>(RNSMX_NOALLOC_SCRATCH_BYTES));
    return RNSMX_ESPACE;
  }
  int8_t *ws = nullptr;
  if (int32_t rc = static_scratch(st, &ws)) return rc;
  return rnsmx_matmul_prepared_fused(a_dev, a_dtype, m, k, n, packed_dev, mods, lut_dev, lut_channels, adaptive,
                                     epilogue, run_plan, ws, RNSMX_NOALLOC_SCRATCH_BYTES, out_dev, stream);
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
  g.b_ld = kp * 16;
  g.b_cs = kp * 16 * ((n + 15) / 16);
  g.m = m;
  g.n = n;
  g.kp = static_cast<int32_t>(kp);
  g.min_channels = 0;
  g.out = out_dev;
  g.out_ld = n;
  g.out_dtype = out_dtype;
  g.a_scale = epilogue ? epilogue->a_scale_dev : nullptr;
  g.w_scale = epilogue ? epilogue->w_scale_dev : nullptr;
  g.bias = epilogue ? epilogue->bias_dev : nullptr;
  g.mods = *mods;
  return launch_gemm(g, false, auto_plan(g, false, false), nullptr, nullptr, static_cast<hipStream_t>(stream));
}

int32_t rnsmx_gemm_plan(int64_t m, int64_t n, int64_t k, int32_t channels, int32_t raw_a, rnsmx_plan_t *out) {
  clear_error();
  if (out == nullptr) return fail(RNSMX_EINVAL, "gemm plan needs an output");
  if (m < 1 || n < 1 || k < 1 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX - 63)
    return fail(RNSMX_EINVAL, "gemm plan needs 1 <= M, N, K < 2^31");
  if (channels < 2 || channels > RNSMX_MAX_CHANNELS)
    return fail(RNSMX_EINVAL, "gemm plan needs 2..10 channels");
  const GemmArgs g = plan_args(m, n, k, channels, raw_a != 0);
  GemmChoice c = auto_plan(g, raw_a != 0, true);
  if (c.splits > 1) {
    int kchunk;
    split_steps(c, g.kp / 64, c.splits, kchunk);
  }
  out->kind = c.kind;
  out->mb = c.mb;
  out->nb = c.nb;
  out->ks = c.ks;
  out->splits = c.splits;
  out->tail = c.splits > 1 ? c.tail : 0;
  return RNSMX_OK;
}

int32_t rnsmx_packed_plan(int64_t m, int64_t n, int64_t k, int32_t channels, rnsmx_plan_t *out) {
  clear_error();
  if (out == nullptr) return fail(RNSMX_EINVAL, "gemm plan needs an output");
  if (m < 1 || n < 1 || k < 1 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX - 63)
    return fail(RNSMX_EINVAL, "gemm plan needs 1 <= M, N, K < 2^31");
  if (channels < 2 || channels > kPackedMaxChannels) return fail(RNSMX_EINVAL, "packed plan needs 2..6 channels");
  const GemmChoice c = packed_auto(plan_args(m, n, k, channels, false));
  *out = rnsmx_plan_t{c.kind, c.mb, c.nb, c.ks, c.splits, c.tail};
  return RNSMX_OK;
}

int32_t rnsmx_quantize_symmetric(const void *x_dev, int32_t x_dtype, int64_t count,
                                 int32_t quant_bits, int32_t *scratch_dev, float *scale_dev,
                                 void *q_dev, void *stream) {
  clear_error();
  if (x_dtype != RNSMX_FLOAT32 && x_dtype != RNSMX_FLOAT16 && x_dtype != RNSMX_BFLOAT16)
    return fail(RNSMX_EINVAL, "activations must be float32, float16 or bfloat16");
  if (quant_bits != 8 && quant_bits != 12 && quant_bits != 16)
    return fail(RNSMX_EINVAL, "quant_bits must be 8, 12 or 16");
  if (count < 0) return fail(RNSMX_EINVAL, "bad element count");
  if (!scratch_dev || !scale_dev || (count > 0 && (!x_dev || !q_dev)))
    return fail(RNSMX_EINVAL, "null pointer");
  QuantArgs a{};
  a.x = x_dev;
  a.count = count;
  const int32_t qmax = (1 << (quant_bits - 1)) - 1;
  a.qmax = static_cast<float>(qmax);
  a.rcp = 1.0f / a.qmax;
  a.partial = reinterpret_cast<float *>(scratch_dev);
  a.scale = scale_dev;
  a.q = q_dev;
  // vector reads need x and q 16-byte aligned (q holds V outputs per vector)
  a.vec = aligned16(x_dev) && aligned16(q_dev);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // ~32 KB of input per block, at most 256 blocks (the chip's CU count)
  const int64_t bytes = count * (x_dtype == RNSMX_FLOAT32 ? 4 : 2);
  const unsigned blocks =
      static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((bytes + 32767) / 32768, 256)));
  static_assert(256 < RNSMX_QUANT_SCRATCH, "the scratch holds one maximum per block");
  a.nparts = static_cast<int32_t>(blocks);
  const int vlen = x_dtype == RNSMX_FLOAT32 ? 4 : 8;
  const unsigned qblocks = static_cast<unsigned>(
      std::max<int64_t>(1, std::min<int64_t>((count / vlen + 255) / 256 + 1, 2048)));
  const bool out16 = quant_bits != 8;
  const bool one_block = count <= kQuantOneBlockMax;
#define RNSMX_QUANT(T)                                                                               \
  if (one_block) {                                                                                   \
    if (out16)                                                                                       \
      hipLaunchKernelGGL((quant_one_block_kernel<T, int16_t>), dim3(1), dim3(1024), 0, st, a);       \
    else                                                                                             \
      hipLaunchKernelGGL((quant_one_block_kernel<T, int8_t>), dim3(1), dim3(1024), 0, st, a);        \
    return check_launch("quant_one_block");                                                          \
  }                                                                                                  \
  hipLaunchKernelGGL(quant_amax_kernel<T>, dim3(blocks), dim3(256), 0, st, a);                       \
  if (int32_t rc = check_launch("quant_amax")) return rc;                                            \
  if (out16)                                                                                         \
    hipLaunchKernelGGL((quant_apply_kernel<T, int16_t>), dim3(qblocks), dim3(256), 0, st, a);        \
  else                                                                                               \
    hipLaunchKernelGGL((quant_apply_kernel<T, int8_t>), dim3(qblocks), dim3(256), 0, st, a);         \
  return check_launch("quant_apply");
  switch (x_dtype) {
    case RNSMX_FLOAT16: { RNSMX_QUANT(__half) }
    case RNSMX_BFLOAT16: { RNSMX_QUANT(Bf16Bits) }
    default: { RNSMX_QUANT(float) }
  }
#undef RNSMX_QUANT
}

// ---------------------------------------------------------------------------
// RNSLinear.forward's device part in one call: [prepared-path workspace
// (split counters first)][quantizer block maxima][activation scale]
// [quantized activations].
// ---------------------------------------------------------------------------
struct LinearLayout {
  int64_t gemm, quant, scale, q, total;
};

static LinearLayout linear_layout(int64_t rows, int64_t k, int64_t n, int32_t channels, int32_t quant_bits) {
  LinearLayout l{};
  l.gemm = rnsmx_prepared_workspace_bytes(rows, k, n, channels, nullptr);
  if (l.gemm < 0) {
    l.total = -1;
    return l;
  }
  l.quant = round_up(l.gemm, 256);
  l.scale = l.quant + round_up(4 * RNSMX_QUANT_SCRATCH, 256);
  l.q = l.scale + 256;
  l.total = l.q + round_up(rows * k * (quant_bits == 8 ? 1 : 2), 256);
  return l;
}

int64_t rnsmx_linear_workspace_bytes(int64_t rows, int64_t k, int64_t n, int32_t channels, int32_t quant_bits) {
  if (quant_bits != 8 && quant_bits != 12 && quant_bits != 16) return -1;
  return linear_layout(rows, k, n, channels, quant_bits).total;
}

int32_t rnsmx_linear_forward(const void *x_dev, int32_t x_dtype, int32_t rows, int32_t k, int32_t n,
                             int32_t quant_bits, const int8_t *packed_dev, const rnsmx_moduli_t *mods,
                             const float *w_scale_dev, const float *bias_dev, const rnsmx_adaptive_t *adaptive,
                             void *workspace_dev, int64_t workspace_bytes, void *out_dev, void *stream) {
  clear_error();
  if (x_dtype != RNSMX_FLOAT32 && x_dtype != RNSMX_FLOAT16 && x_dtype != RNSMX_BFLOAT16)
    return fail(RNSMX_EINVAL, "activations must be float32, float16 or bfloat16");
  if (quant_bits != 8 && quant_bits != 12 && quant_bits != 16)
    return fail(RNSMX_EINVAL, "quant_bits must be 8, 12 or 16");
  if (!mods || mods->channels < 1) return fail(RNSMX_EINVAL, "moduli are not initialised");
  if (rows < 0 || k < 1 || n < 0) return fail(RNSMX_EINVAL, "bad linear shape");
  if (!w_scale_dev) return fail(RNSMX_EINVAL, "the weight scales are missing");
  const LinearLayout l = linear_layout(rows, k, n, mods->channels, quant_bits);
  if (l.total < 0) return fail(RNSMX_EINVAL, "bad linear shape");
  if (!workspace_dev) return fail(RNSMX_EINVAL, "null workspace");
  if (workspace_bytes < l.total) {
    set_error("workspace too small: %lld < %lld bytes", static_cast<long long>(workspace_bytes),
              static_cast<long long>(l.total));
    return RNSMX_ESPACE;
  }
  int8_t *ws = static_cast<int8_t *>(workspace_dev);
  float *scale = reinterpret_cast<float *>(ws + l.scale);
  void *q = ws + l.q;
  if (int32_t rc = rnsmx_quantize_symmetric(x_dev, x_dtype, static_cast<int64_t>(rows) * k, quant_bits,
                                            reinterpret_cast<int32_t *>(ws + l.quant), scale, q, stream))
    return rc;
  rnsmx_epilogue_t epi{x_dtype, scale, w_scale_dev, bias_dev};
  return rnsmx_matmul_prepared_fused(q, quant_bits == 8 ? RNSMX_INT8 : RNSMX_INT16, rows, k, n, packed_dev, mods,
                                     nullptr, 0, adaptive, &epi, nullptr, ws, l.gemm, out_dev, stream);
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
