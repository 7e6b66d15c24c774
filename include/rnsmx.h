/*
 * rnsmx: MI355X (gfx950) native RNS linear / fused-QKV backend, C ABI.
 *
 * The boundary replaces the pybind11 module `rns_llm._C` of Nek1tt/rns-llm
 * (csrc/bindings.cpp:45-75) and the host-side constant cache of
 * `CudaRNSBackend` (src/rns_llm/backends/cuda_backend.py:48-66, 137-166).
 *
 * Conventions
 *   - Every pointer named *_dev is a device pointer on the current HIP device;
 *     everything else is host memory.
 *   - Every call that launches work is asynchronous on `stream` and never
 *     synchronises, allocates, or frees memory.  Scratch memory is always
 *     caller-owned (`workspace`, sized by the *_workspace_bytes queries).
 *   - A workspace starts with RNSMX_SPLIT_TICKETS 32-bit arrival counters of
 *     the K split over workgroups (rnsmx_plan_t.splits).  For
 *     rnsmx_matmul_prepared_fused they must be zero when the workspace is
 *     first used (allocate it zero-filled); every call leaves them zero, for
 *     any shape, so one workspace serves any sequence of calls.  Calls that
 *     share a workspace must not overlap (keep one per stream).
 *   - Return value: RNSMX_OK (0) on success, otherwise an RNSMX_E* code and a
 *     thread-local message readable through rnsmx_last_error().
 *   - Integer results are exact: bit-identical to A.astype(int64) @ B for any
 *     input whose product fits the moduli's centered range.
 */
#ifndef RNSMX_H
#define RNSMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RNSMX_MAX_CHANNELS 10
#define RNSMX_K_ALIGN 64 /* K padding of residue planes, bytes */
/* Arrival counters at the start of every workspace (64 KiB): a K split runs
 * only when its (tile, wave) count fits. */
#define RNSMX_SPLIT_TICKETS 16384

enum rnsmx_status {
  RNSMX_OK = 0,
  RNSMX_EINVAL = 1,  /* bad argument: shape, dtype, pointer, moduli */
  RNSMX_ERANGE = 2,  /* arithmetic range: product or accumulator bound */
  RNSMX_ELAUNCH = 3, /* HIP runtime reported an error */
  RNSMX_ESPACE = 4   /* caller-provided workspace too small */
};

enum rnsmx_dtype {
  RNSMX_INT8 = 0,
  RNSMX_INT16 = 1,
  RNSMX_INT32 = 2,
  RNSMX_INT64 = 3,
  RNSMX_FLOAT32 = 4,
  RNSMX_FLOAT16 = 5,
  RNSMX_BFLOAT16 = 6
};

/*
 * Moduli set plus every constant the kernels need, built on the host and
 * passed to kernels by value (kernel-argument memory, read through scalar
 * loads).  Replaces `_host_constants` / `_DeviceConstants`
 * (cuda_backend.py:48-66): Barrett reciprocals, Garner inverses and the
 * modulus product.
 */
typedef struct rnsmx_moduli {
  int32_t channels;
  int32_t moduli[RNSMX_MAX_CHANNELS];
  uint32_t magic[RNSMX_MAX_CHANNELS];  /* floor(2^32 / m_i)                   */
  uint32_t c31[RNSMX_MAX_CHANNELS];    /* 2^31 mod m_i                        */
  uint32_t qinv[RNSMX_MAX_CHANNELS];   /* (prod_{j<i} m_j)^-1 mod m_i         */
  uint32_t ucoef[RNSMX_MAX_CHANNELS][RNSMX_MAX_CHANNELS];
                                       /* [j][i], j<i: -(prod_{l<j} m_l)*qinv_i mod m_i */
  int64_t prefix[RNSMX_MAX_CHANNELS + 1]; /* prod_{j<i} m_j, i = 0..channels  */
  int32_t qk16[RNSMX_MAX_CHANNELS];    /* 2^16 * qinv_i mod m_i, centered (|.| <= m_i/2) */
  uint32_t qk8[RNSMX_MAX_CHANNELS];    /* 2^8 * qinv_i mod m_i                */
} rnsmx_moduli_t;

/*
 * Kernel plan of one GEMM launch.  kind 0 = the library's automatic choice
 * (the other fields are then ignored); 1 = stream kernel (tile 16*mb x
 * 16*nb, ks waves splitting K inside a workgroup), 2 = MFMA kernel (tile
 * 16*mb x 64*nb, ks = K steps of loads in flight, 0 = the tile's default),
 * 3 = LDS-staged kernel (256 x 64 tiles; int8 activations, 4-channel
 * capacity, K a multiple of 256; mb, nb, ks ignored), 4 = the stream kernel
 * loading chunks of up to 8 K steps per wave (16 x 16 tiles, up to 4
 * channels), 5 = the MFMA kernel with three column waves (tile 16*mb x
 * 48*nb; int8 activations read in place, up to 4 channels), 7 = the
 * LDS-staged kernel with 256 x 96 tiles (same conditions as 3), 8 = the
 * LDS-staged kernel for residue-plane activations (int16 / int32 inputs,
 * and packed weights; 128 x 128 tiles, 4- or 6-channel capacity, K a
 * multiple of 256; mb, nb, ks ignored; splits and tail as for kind 3).
 * splits: workgroups splitting K per output tile (0 or 1 = none; up to 4
 * channels, 6 for kind 8, and for the stream kernel ks = 1): each reduces its partial
 * sums to residues, and the last to finish a tile reconstructs it.  tail:
 * split only the tiles past the last full round of 256 (the others run
 * whole, first).  A plan
 * that names a kernel that is not built, or does not fit the call, makes the
 * call fail with RNSMX_EINVAL.  Results never depend on the plan.  No
 * counterpart in the reference (cuBLAS picks its own kernels there); for
 * tuning and for tests that run every kernel on the same inputs.
 */
typedef struct rnsmx_plan {
  int32_t kind;
  int32_t mb, nb, ks;
  int32_t splits;
  int32_t tail;
} rnsmx_plan_t;

/* Thread-local text of the last error (empty string when none). */
const char *rnsmx_last_error(void);

/* ABI version; bumped on any signature or struct change. */
int32_t rnsmx_abi_version(void);

/*
 * Host only.  Validates the set (each m in [2,255], pairwise coprime,
 * product < 2^63) and fills `out`.
 * Replaces reference.py:11-23 (validate_moduli), reference.py:43-67
 * (crt_constants, garner_pairwise_inverses) and cuda_backend.py:48-55.
 */
int32_t rnsmx_moduli_init(const int32_t *moduli, int32_t channels,
                          rnsmx_moduli_t *out);

/*
 * Host only.  Fills `lut` (int16 [channels][4][256]) with b*256^p mod m_c:
 * the compact byte-decomposition table of reference.py:70-88.
 */
int32_t rnsmx_compact_lut(const rnsmx_moduli_t *mods, int16_t *lut);

/*
 * Centered residue encode: values [rows][cols] (RNSMX_INT8/16/32,
 * contiguous) -> out_dev [channels][rows][out_ld] int8 with
 * r = v mod m in [-floor(m/2), floor(m/2)], and zero bytes in columns
 * [cols, out_ld).  out_ld >= cols.  When row_l1_dev is non-null it receives
 * int64 sum_k |v[row][k]| per row; when absmax_dev is non-null the maximum
 * |v| is folded into it with an atomic max (the caller zeroes it first).
 * Replaces _C.encode_centered (csrc/rns_cuda.cu:584-626, kernel 98-124);
 * the plain reference form is rows=1, cols=numel, out_ld=numel.
 */
int32_t rnsmx_encode_centered(const void *values_dev, int32_t dtype,
                              int64_t rows, int64_t cols, int64_t out_ld,
                              const rnsmx_moduli_t *mods, int8_t *out_dev,
                              int64_t *row_l1_dev, int32_t *absmax_dev,
                              void *stream);

/* Bytes of workspace rnsmx_matmul_centered_fused_out needs (its counters
 * are cleared by the call itself, so any buffer of this size serves). */
int64_t rnsmx_fused_workspace_bytes(int64_t m, int64_t k, int64_t n,
                                    int32_t channels);

/*
 * Drop-in fused op: a_dev [R][M][K] and b_dev [R][K][N] centered int8
 * residue planes (contiguous, the reference layout) -> out_dev [M][N] int64.
 * Per-channel int8 GEMM on MFMA, modular reduction, Garner mixed radix and
 * signed correction, all in one GEMM epilogue.  `lut_dev` / `lut_channels`
 * are the reference's byte-table arguments: validated as the reference
 * does (lut_channels in {0, 1, 2}, <= R, table present when > 0); the
 * residue is unique, so results do not depend on them and every channel
 * uses the 24-bit arithmetic reduction.  No K%4 / N%4
 * restriction.  `workspace_dev` holds the repacked operands (B in the
 * fragment-major order of rnsmx_prepare_weight).
 * Replaces _C.matmul_centered_fused_out (csrc/rns_cuda.cu:887-980: cuBLAS
 * site 478-523 + fused_reduce_garner_kernel 442-476).
 */
int32_t rnsmx_matmul_centered_fused_out(
    const int8_t *a_dev, const int8_t *b_dev, int32_t m, int32_t k, int32_t n,
    const rnsmx_moduli_t *mods, const int16_t *lut_dev, int32_t lut_channels,
    void *workspace_dev, int64_t workspace_bytes, int64_t *out_dev,
    void *stream);

/*
 * Weight preparation: b_nk_dev [N][K] (int8/16/32, i.e. the quantized
 * nn.Linear weight, or B transposed) -> packed_dev, centered residues in
 * fragment-major order [R][ceil(N/16)][kp/64][1024], kp = round_up(K,
 * RNSMX_K_ALIGN): byte 16*l + b of the fragment of column block jb and K
 * step ks is the residue of column 16*jb + (l % 16), K index
 * 64*ks + 16*(l / 16) + b (zero past N and past K).  That is the B-operand
 * layout of the gfx950 int8 MFMA, so each operand load is one contiguous
 * 1 KB.  absmax_dev (nullable, zeroed by the caller) receives max |b| for
 * the adaptive bound.
 * Replaces CudaRNSBackend.prepare_weight (cuda_backend.py:464-487), whose
 * storage is [R][K][N].
 */
int32_t rnsmx_prepare_weight(const void *b_nk_dev, int32_t dtype, int32_t n,
                             int32_t k, const rnsmx_moduli_t *mods,
                             int8_t *packed_dev, int32_t *absmax_dev,
                             void *stream);

/* Bytes of workspace rnsmx_matmul_prepared_fused needs for an M x N x K
 * product with `channels` moduli under `plan` (NULL: the automatic plan),
 * whatever the activation dtype. */
int64_t rnsmx_prepared_workspace_bytes(int64_t m, int64_t k, int64_t n,
                                       int32_t channels,
                                       const rnsmx_plan_t *plan);

/* Epilogue selector of rnsmx_matmul_prepared_fused. */
typedef struct rnsmx_epilogue {
  int32_t out_dtype;            /* RNSMX_INT64 (exact) or FLOAT32/16/BFLOAT16 */
  const float *a_scale_dev;     /* [1] activation scale (float outputs)      */
  const float *w_scale_dev;     /* [N] per-output-channel scale              */
  const float *bias_dev;        /* [N] or null                               */
} rnsmx_epilogue_t;

/* Adaptive channel prefix, decided on the device. */
typedef struct rnsmx_adaptive {
  int32_t min_channels;         /* 0 = off (all channels)                    */
  const int32_t *w_absmax_dev;  /* [1] max |B| from rnsmx_prepare_weight     */
  int64_t *meta_dev;            /* [4] out: channels, bound, capacity, overflow */
} rnsmx_adaptive_t;

/*
 * Hot path: a_dev [M][K] (int8/16/32 activations) x prepared weight
 * (packed_dev from rnsmx_prepare_weight, n x k) -> out_dev [M][N].
 * Encodes activations (fused row-L1 bound), runs the per-channel MFMA GEMM
 * with the reduction + Garner (+ optional dequant) epilogue.  With
 * adaptive.min_channels > 0 the GEMM picks, on the device and without any
 * host synchronisation, the shortest moduli prefix c >= min_channels with
 * 2 * max_i(sum_k |a_ik|) * max|B| < prod(prefix); if none fits it uses the
 * full set and sets meta[3] = 1.  plan: NULL for the automatic kernel
 * choice.  The workspace's counters must be zero at its first use (see
 * the conventions above).
 * Replaces matmul_prepared_fused (cuda_backend.py:514-539) and
 * matmul_prepared_adaptive_fused (cuda_backend.py:577-622, whose selector
 * synchronises at :591).
 */
int32_t rnsmx_matmul_prepared_fused(
    const void *a_dev, int32_t a_dtype, int32_t m, int32_t k, int32_t n,
    const int8_t *packed_dev, const rnsmx_moduli_t *mods,
    const int16_t *lut_dev, int32_t lut_channels,
    const rnsmx_adaptive_t *adaptive, const rnsmx_epilogue_t *epilogue,
    const rnsmx_plan_t *plan, void *workspace_dev, int64_t workspace_bytes,
    void *out_dev, void *stream);

/* Bytes of the static scratch of rnsmx_matmul_prepared_fused_noalloc (16 MiB
 * per GPU, held until the process ends). */
#define RNSMX_NOALLOC_SCRATCH_BYTES (16 << 20)

/*
 * rnsmx_matmul_prepared_fused without a workspace argument: the call uses a
 * library-owned static device array of RNSMX_NOALLOC_SCRATCH_BYTES per GPU
 * instead, and allocates nothing (no hipMalloc, no hipFree, no allocating
 * library call).  Same arguments, results and errors otherwise.  With the
 * automatic plan (plan NULL or kind 0) a K split whose exchange area does
 * not fit the static scratch is dropped: the call then runs the automatic
 * kernel unsplit (same results).  A call whose scratch need for the plan it
 * runs still exceeds the maximum fails with RNSMX_ESPACE; that check, and
 * those of the shape, moduli, activation type and plan, come before the
 * GPU is touched.
 * The first call on each device resolves the array's address there and
 * clears its counters with one small kernel on `stream`; make that call
 * outside graph capture.  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other threads) race and
 * must be serialised by the caller.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation).
 */
int32_t rnsmx_matmul_prepared_fused_noalloc(
    const void *a_dev, int32_t a_dtype, int32_t m, int32_t k, int32_t n,
    const int8_t *packed_dev, const rnsmx_moduli_t *mods,
    const int16_t *lut_dev, int32_t lut_channels,
    const rnsmx_adaptive_t *adaptive, const rnsmx_epilogue_t *epilogue,
    const rnsmx_plan_t *plan, void *out_dev, void *stream);

/*
 * GEMM stage of rnsmx_matmul_prepared_fused on activations already encoded
 * by rnsmx_encode_centered into a_res_dev [R][M][a_ld] (a_ld a multiple of
 * RNSMX_K_ALIGN, zero bytes in [K, a_ld)), against a prepared weight.  Same
 * epilogue options, no adaptive prefix (all channels), no workspace (so no
 * K split over workgroups).  Lets a caller
 * encode once and reuse the residues (e.g. one activation against several
 * weights) and times the GEMM kernel on its own.
 * Replaces the cuBLAS + fused_reduce_garner half of _C.matmul_centered_fused_out
 * (csrc/rns_cuda.cu:949-976) for a prepared weight.
 */
int32_t rnsmx_matmul_residues_prepared(
    const int8_t *a_res_dev, int64_t a_ld, int32_t m, int32_t k, int32_t n,
    const int8_t *packed_dev, const rnsmx_moduli_t *mods,
    const int16_t *lut_dev, int32_t lut_channels,
    const rnsmx_epilogue_t *epilogue, void *out_dev, void *stream);

/*
 * Packed weights: 2 bytes per weight value whatever the channel count, for
 * int16 (quant_bits 12 or 16) or int8 weights.  The reference stores one
 * byte per residue channel and names packed residues, or residues made
 * inside the GEMM, as the way to a real memory saving (README.md:26-36,
 * docs/RELEASE_V05.md:81-91); it has no such entry point.
 *
 * rnsmx_prepare_weight_packed: b_nk_dev [N][K] int8 or int16 -> packed_dev,
 * two byte planes [2][ceil(N/16)][kp/64][1024] in the fragment-major order
 * of rnsmx_prepare_weight: plane 0 holds hi = v >> 8 (arithmetic shift),
 * plane 1 lo = (v & 255) - 128, so v = 256 hi + lo + 128 (zero past N and
 * K).  No moduli: one packed weight serves any moduli set.  absmax_dev as
 * in rnsmx_prepare_weight.
 *
 * rnsmx_matmul_packed_fused: rnsmx_matmul_prepared_fused against a packed
 * weight, with the same arguments, results and errors, for 2 to 6
 * channels.  Channel c's weight residue is never stored: with
 * d_c = 256 mod m_c, v = d_c hi + lo + 128 (mod m_c), so the kernels run
 * two MFMAs per channel (activation residues of d_c a against hi, of a
 * against lo) and add 128 sum_k a_k per row.  Accumulators: 2 K 128
 * max(floor(m/2)) + 255 < 2^31 (else RNSMX_ERANGE).  Plans: kind 1 (stream,
 * mb 1 or 2, nb 1, ks 1-4), 2 (MFMA, mb 2 or 4, nb 1) or 6 (channel rows,
 * mb 1, 2, 4 or 8 token blocks), never split, or 8 (the residue-plane LDS
 * kernel, K a multiple of 256, split as for the residue-plane entry); NULL
 * for the automatic one (rnsmx_packed_plan).  The workspace holds the
 * encoded activations and the split exchange of the automatic plan
 * (rnsmx_packed_workspace_bytes).
 */
int32_t rnsmx_prepare_weight_packed(const void *b_nk_dev, int32_t dtype,
                                    int32_t n, int32_t k, int8_t *packed_dev,
                                    int32_t *absmax_dev, void *stream);

/* Bytes of workspace rnsmx_matmul_packed_fused needs for an M x N x K
 * product with `channels` moduli under `plan` (NULL: the automatic plan);
 * -1 for a bad shape or a plan the call would reject. */
int64_t rnsmx_packed_workspace_bytes(int64_t m, int64_t k, int64_t n,
                                     int32_t channels,
                                     const rnsmx_plan_t *plan);

int32_t rnsmx_matmul_packed_fused(
    const void *a_dev, int32_t a_dtype, int32_t m, int32_t k, int32_t n,
    const int8_t *packed_dev, const rnsmx_moduli_t *mods,
    const int16_t *lut_dev, int32_t lut_channels,
    const rnsmx_adaptive_t *adaptive, const rnsmx_epilogue_t *epilogue,
    const rnsmx_plan_t *plan, void *workspace_dev, int64_t workspace_bytes,
    void *out_dev, void *stream);

/* The plan rnsmx_matmul_packed_fused chooses by itself (host only). */
int32_t rnsmx_packed_plan(int64_t m, int64_t n, int64_t k, int32_t channels,
                          rnsmx_plan_t *out);

/*
 * The plan rnsmx_matmul_prepared_fused chooses by itself for an M x N x K
 * product with `channels` moduli (kind 1-8, tile, ks, splits as in
 * rnsmx_plan_t).  raw_a != 0: int8 activations read in place, as the fused
 * entry points do for int8 sources with K a multiple of 16 whose
 * accumulators fit int32; 0: residue planes.  Host code only (no GPU call,
 * no stream).  No counterpart in the reference (cuBLAS picks its own
 * kernels there); for tests and tuning.
 */
int32_t rnsmx_gemm_plan(int64_t m, int64_t n, int64_t k, int32_t channels,
                        int32_t raw_a, rnsmx_plan_t *out);

/* 32-bit scratch words rnsmx_quantize_symmetric needs (per-block maxima). */
#define RNSMX_QUANT_SCRATCH 1025

/*
 * Per-tensor symmetric quantization of activations, two launches:
 * scale_dev[0] = max(amax|x| * fl32(1 / qmax), FLT_EPSILON) and
 * q_dev[i] = clamp(rint(x[i] / scale), -qmax, qmax) with qmax =
 * 2^(quant_bits-1) - 1, int8 for 8 bits, int16 for 12 or 16.  x_dev is
 * float32, float16 or bfloat16 [count], contiguous.  scratch_dev holds
 * RNSMX_QUANT_SCRATCH 32-bit words of per-block maxima passed from the
 * first launch to the second; its contents before a call do not matter,
 * and calls that share one scratch must not overlap (keep one per stream).
 * Non-finite inputs follow the reference chain's float operations: a NaN
 * anywhere makes the scale NaN (torch's amax propagates it) and an infinity
 * (without NaN) makes it +inf; an element whose quotient x / scale is NaN
 * quantizes to 0 (what the reference leaves to the float-to-integer cast),
 * so the dequantized outputs of such a call are all NaN, as the reference's
 * are.
 * Replaces RNSLinear._symmetric_scale + _quantize on activations
 * (src/rns_llm/layers/rns_linear.py:154-166, called at 249-250).
 */
int32_t rnsmx_quantize_symmetric(const void *x_dev, int32_t x_dtype, int64_t count,
                                 int32_t quant_bits, int32_t *scratch_dev, float *scale_dev,
                                 void *q_dev, void *stream);

/* Bytes of workspace rnsmx_linear_forward needs (-1 for a bad shape). */
int64_t rnsmx_linear_workspace_bytes(int64_t rows, int64_t k, int64_t n,
                                     int32_t channels, int32_t quant_bits);

/*
 * The device part of RNSLinear.forward in one call: per-tensor symmetric
 * quantization of x_dev [rows][k] (float32, float16 or bfloat16, as
 * rnsmx_quantize_symmetric), then the prepared-weight GEMM whose epilogue
 * writes ((float)y * s_x) * w_scale[col] + bias[col] in x's dtype into
 * out_dev [rows][n].  w_scale_dev [n] float32 (per output channel), bias_dev
 * [n] float32 or NULL; adaptive as in rnsmx_matmul_prepared_fused.  The
 * quantized activations, their scale and the GEMM scratch live in the
 * workspace (rnsmx_linear_workspace_bytes; the counter rule of the
 * conventions above applies).  Three launches, no host synchronisation.
 * Replaces RNSLinear.forward's quantize -> backend -> dequantize chain
 * (src/rns_llm/layers/rns_linear.py:238-275) on a prepared weight.
 */
int32_t rnsmx_linear_forward(const void *x_dev, int32_t x_dtype, int32_t rows,
                             int32_t k, int32_t n, int32_t quant_bits,
                             const int8_t *packed_dev, const rnsmx_moduli_t *mods,
                             const float *w_scale_dev, const float *bias_dev,
                             const rnsmx_adaptive_t *adaptive,
                             void *workspace_dev, int64_t workspace_bytes,
                             void *out_dev, void *stream);

/*
 * Garner reconstruction of centered residues [R][count] int8 -> int64.
 * Replaces _C.decode_garner (csrc/rns_cuda.cu:818-885, kernel 416-440).
 */
int32_t rnsmx_decode_garner(const int8_t *residues_dev, int64_t count,
                            const rnsmx_moduli_t *mods, int64_t *out_dev,
                            void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RNSMX_H */
