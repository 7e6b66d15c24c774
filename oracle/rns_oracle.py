"""CPU oracle for the RNS linear / fused-QKV path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this module;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or as the timed CPU baseline).

This is a NumPy restatement of the reference's integer algorithm
(``src/rns_llm/reference.py`` and ``src/rns_llm/adaptive.py`` of Nek1tt/rns-llm
v0.5), written from its behaviour, plus the semantics of the fused CUDA path
(``csrc/rns_cuda.cu`` reduction + Garner) and of the backend's adaptive prefix
and continuous batching (``src/rns_llm/backends/cuda_backend.py``).

How each function is pinned (tests/test_oracle.py):
  * encode / decode: exhaustive int8 and a large int16/int32 sample against the
    closed form ``v mod m`` and the CRT identity; reference known answers
    (``tests/test_reference.py:11-14`` round trip over [-10000, 10000];
    ``:49-57`` Garner over +-1e6 with seed 123).
  * residue matmul + reconstruction: equal to ``A.astype(int64) @ B`` (the
    reference's own oracle, ``docs/CORRECTNESS_GUARDS.md:5-9``) and to a
    brute-force triple loop on tiny inputs.
  * Garner vs CRT: both decoders agree with each other and with the integer.
  * moduli selection: reference known answer (255, 253, 251, 247) for K=768,
    int8; product covers 2*K*127^2 (``tests/test_reference.py:60-66``);
    12-bit case (``:40-46``).
  * adaptive prefix: ``tests/test_reference.py:69-81`` (bound 5e6 -> 3
    channels); the 3-channel capacity 8,096,632 recorded in
    ``results/v0.5/adaptive_channels.json:20``; brute force over every prefix;
    ``adaptive_select`` on hand-built activations whose largest row L1
    differs from their largest column L1 (the reference sums each row,
    ``cuda_backend.py:591``), with the bound, prefix and capacity worked out
    by hand.
  * compact LUT: every entry equals b * 256**p mod m and byte decomposition
    reproduces ``%`` for sampled 32-bit values.
"""
from __future__ import annotations

from math import gcd, prod
from typing import Iterable

import numpy as np

INT64_MAX = (1 << 63) - 1


# ---------------------------------------------------------------------------
# Moduli tables and validation
# ---------------------------------------------------------------------------
# Candidate orders are data fixed by the reference (``reference.py:190-230``);
# the selection result for a given K depends on the exact order, so the order
# is kept identical.
LARGE_PRIME_MODULI = (
    251, 241, 239, 233, 229, 227, 223, 211, 199, 197, 193, 191, 181, 179, 173,
    167, 163, 157, 151, 149, 139, 137, 131, 127,
)
DENSE_COPRIME_MODULI = (
    255, 253, 251, 247, 241, 239, 233, 229, 227, 223, 211, 199, 197, 193, 191,
    181, 179, 173, 167, 163, 157, 151, 149, 139, 137, 131, 127, 125, 121,
)
SMALL_PRIME_MODULI = (
    3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37, 41, 43, 47, 53, 59, 61, 67, 71,
    73, 79, 83, 89, 97, 101, 103, 107, 109, 113, 127, 131, 137, 139, 149, 151,
    157, 163, 167, 173, 179, 181, 191, 193, 197, 199, 211, 223, 227, 229, 233,
    239, 241, 251,
)


def validate_moduli(moduli: Iterable[int]) -> tuple[int, ...]:
    """Every modulus in [2, 255], pairwise coprime (``reference.py:11-23``)."""
    mods = tuple(int(m) for m in moduli)
    if len(mods) == 0:
        raise ValueError("moduli must not be empty")
    for m in mods:
        if not 2 <= m <= 255:
            raise ValueError("every modulus must be in [2, 255]")
    for i in range(len(mods)):
        for j in range(i + 1, len(mods)):
            if gcd(mods[i], mods[j]) != 1:
                raise ValueError(
                    f"moduli are not pairwise coprime: {mods[i]}, {mods[j]}")
    return mods


def candidates_for_strategy(strategy: str) -> tuple[int, ...]:
    """``reference.py:226-235``."""
    table = {
        "large_primes": LARGE_PRIME_MODULI,
        "dense_coprime": DENSE_COPRIME_MODULI,
        "small_primes": SMALL_PRIME_MODULI,
    }
    if strategy not in table:
        raise ValueError(f"unknown moduli strategy: {strategy}")
    return table[strategy]


def dot_product_bound(k: int, max_abs_a: int, max_abs_b: int) -> int:
    """``reference.py:238-243``: |sum_k a*b| <= K * max|a| * max|b|."""
    if k <= 0:
        raise ValueError("k must be positive")
    if max_abs_a < 0 or max_abs_b < 0:
        raise ValueError("absolute bounds must be non-negative")
    return int(k) * int(max_abs_a) * int(max_abs_b)


def choose_moduli_for_dot(k, max_abs_a, max_abs_b, *, candidates=None,
                          strategy="large_primes") -> tuple[int, ...]:
    """Greedy coprime prefix until prod >= 2*bound + 1 (``reference.py:246-275``)."""
    need = 2 * dot_product_bound(k, max_abs_a, max_abs_b) + 1
    pool = tuple(candidates) if candidates is not None else candidates_for_strategy(strategy)
    chosen: list[int] = []
    running = 1
    for m in pool:
        m = int(m)
        if m < 2 or m > 255 or any(gcd(m, c) != 1 for c in chosen):
            continue
        chosen.append(m)
        running *= m
        if running >= need:
            return tuple(chosen)
    raise ValueError(f"candidate moduli cannot cover required range {need}")


# ---------------------------------------------------------------------------
# Encoding
# ---------------------------------------------------------------------------
def encode_canonical(values, moduli) -> np.ndarray:
    """[R, *shape] uint8 residues in [0, m) (``reference.py:26-29``)."""
    mods = validate_moduli(moduli)
    v = np.asarray(values, dtype=np.int64)
    out = np.empty((len(mods),) + v.shape, dtype=np.uint8)
    for c, m in enumerate(mods):
        out[c] = np.mod(v, m)
    return out


def encode_centered(values, moduli) -> np.ndarray:
    """[R, *shape] int8 residues in [-floor(m/2), floor(m/2)].

    Canonical residue r in [0, m); r > floor(m/2) maps to r - m
    (``reference.py:32-40``; device form ``csrc/rns_cuda.cu:98-124``).
    """
    mods = validate_moduli(moduli)
    v = np.asarray(values, dtype=np.int64)
    out = np.empty((len(mods),) + v.shape, dtype=np.int8)
    for c, m in enumerate(mods):
        r = np.mod(v, m)
        out[c] = (r - m * (r > m // 2)).astype(np.int8)
    return out


# ---------------------------------------------------------------------------
# Constants
# ---------------------------------------------------------------------------
def crt_constants(moduli) -> tuple[int, tuple[int, ...]]:
    """P and the CRT basis e_i = (P/m_i) * ((P/m_i)^-1 mod m_i) mod P
    (``reference.py:43-54``)."""
    mods = validate_moduli(moduli)
    big_p = prod(mods)
    if big_p > INT64_MAX:
        raise OverflowError("product(moduli) must fit signed int64 for this decoder")
    basis = []
    for m in mods:
        cofactor = big_p // m
        basis.append((cofactor * pow(cofactor % m, -1, m)) % big_p)
    return big_p, tuple(basis)


def garner_pairwise_inverses(moduli) -> tuple[tuple[int, ...], ...]:
    """Table [j][i] = m_j^-1 mod m_i for j < i, zero elsewhere
    (``reference.py:57-67``)."""
    mods = validate_moduli(moduli)
    n = len(mods)
    return tuple(
        tuple(pow(mods[j], -1, mods[i]) if j < i else 0 for i in range(n))
        for j in range(n)
    )


def compact_byte_mod_lut(moduli) -> np.ndarray:
    """int16 [R, 4, 256]: entry [c, p, b] = b * 256**p mod m_c
    (``reference.py:70-88``)."""
    mods = validate_moduli(moduli)
    b = np.arange(256, dtype=np.int64)
    lut = np.empty((len(mods), 4, 256), dtype=np.int16)
    for c, m in enumerate(mods):
        for p in range(4):
            lut[c, p] = (b * pow(256, p, m)) % m
    return lut


def signed_capacity(moduli) -> int:
    """``adaptive.py:9-12``: (P - 1) // 2."""
    return (prod(validate_moduli(moduli)) - 1) // 2


# ---------------------------------------------------------------------------
# Decoding
# ---------------------------------------------------------------------------
def _center(x: np.ndarray, big_p: int) -> np.ndarray:
    return np.where(x > big_p // 2, x - big_p, x)


def decode_crt(residues, moduli, *, signed=True) -> np.ndarray:
    """CRT reconstruction, accumulating mod P one channel at a time
    (``reference.py:91-116``).  Accepts canonical or centered residues."""
    mods = validate_moduli(moduli)
    r = np.asarray(residues, dtype=np.int64)
    if r.shape[0] != len(mods):
        raise ValueError("residue channel count does not match moduli")
    big_p, basis = crt_constants(mods)
    acc = np.zeros(r.shape[1:], dtype=np.int64)
    for c, e in enumerate(basis):
        # r mod m (< 256) times e (< P) can exceed int64 when P is large, so
        # the product is formed as exact Python integers for object safety.
        term = (np.mod(r[c], mods[c]).astype(object) * e) % big_p
        acc = ((acc.astype(object) + term) % big_p).astype(np.int64)
    return _center(acc, big_p) if signed else acc


def decode_garner(residues, moduli, *, signed=True) -> np.ndarray:
    """Mixed-radix (Garner) reconstruction (``reference.py:119-147``;
    device form ``csrc/rns_cuda.cu:380-414``).

    digit_i = ((r_i - d_0) m_0^-1 - d_1) m_1^-1 ... mod m_i, then
    x = sum_i d_i * prod_{j<i} m_j, centered about P // 2.
    """
    mods = validate_moduli(moduli)
    r = np.asarray(residues, dtype=np.int64)
    if r.shape[0] != len(mods):
        raise ValueError("residue channel count does not match moduli")
    inv = garner_pairwise_inverses(mods)
    digits = []
    for i, m in enumerate(mods):
        d = np.mod(r[i], m)
        for j in range(i):
            d = np.mod((d - digits[j]) * inv[j][i], m)
        digits.append(d)
    x = np.zeros(r.shape[1:], dtype=np.int64)
    radix = 1
    for m, d in zip(mods, digits):
        x = x + d * radix
        radix *= m
    return _center(x, radix) if signed else x


# ---------------------------------------------------------------------------
# Residue GEMMs and the fused path
# ---------------------------------------------------------------------------
def matmul_residues(a_res, b_res, moduli) -> np.ndarray:
    """Canonical residue GEMM: per channel int64 (A_c @ B_c) mod m_c
    (``reference.py:150-170``)."""
    mods = validate_moduli(moduli)
    a = np.asarray(a_res)
    b = np.asarray(b_res)
    if a.ndim != 3 or b.ndim != 3:
        raise ValueError("expected [R, M, K] and [R, K, N]")
    if a.shape[0] != len(mods) or b.shape[0] != len(mods):
        raise ValueError("residue channel count does not match moduli")
    if a.shape[2] != b.shape[1]:
        raise ValueError("K dimensions do not match")
    out = np.empty((len(mods), a.shape[1], b.shape[2]), dtype=np.int64)
    for c, m in enumerate(mods):
        out[c] = np.mod(a[c].astype(np.int64) @ b[c].astype(np.int64), m)
    return out


def channel_accumulators(a_res, b_res) -> np.ndarray:
    """int32-exact per-channel products [R, M, N] of centered residue planes
    (what ``run_cublas_int8_batched``, ``csrc/rns_cuda.cu:478-523``, writes)."""
    a = np.asarray(a_res, dtype=np.int64)
    b = np.asarray(b_res, dtype=np.int64)
    return np.stack([a[c] @ b[c] for c in range(a.shape[0])])


def canonical_mod_byte_lut(values, modulus, lut_row) -> np.ndarray:
    """Canonical residue of int32 values through a [4, 256] byte table: the
    sum over the four bytes of |v| of table[p][byte_p], reduced below m, and
    negated for negative v (``csrc/rns_cuda.cu:69-96``)."""
    v = np.asarray(values, dtype=np.int64)
    mag = np.abs(v)
    s = np.zeros_like(mag)
    for p in range(4):
        s += lut_row[p][(mag >> (8 * p)) & 0xFF].astype(np.int64)
    s = np.mod(s, modulus)
    return np.where((v < 0) & (s != 0), modulus - s, s)


def fused_reduce_garner(acc, moduli, *, lut_channels=0) -> np.ndarray:
    """Reduction of [R, M, N] int32 accumulators to int64 [M, N]: channels
    below ``lut_channels`` reduce through the byte LUT, the rest with plain
    modulo (Barrett on the device); then Garner and the signed correction
    (``csrc/rns_cuda.cu:442-476``).  Both reductions give the same canonical
    residue; the LUT path is exercised to prove it."""
    mods = validate_moduli(moduli)
    a = np.asarray(acc, dtype=np.int64)
    lut = compact_byte_mod_lut(mods)
    canon = np.empty_like(a)
    for c, m in enumerate(mods):
        if c < lut_channels:
            canon[c] = canonical_mod_byte_lut(a[c], m, lut[c])
        else:
            canon[c] = np.mod(a[c], m)
    return decode_garner(canon, mods)


def rns_matmul(a, b, moduli, *, decode=True) -> np.ndarray:
    """Canonical pipeline encode -> residue GEMM -> CRT
    (``reference.py:173-185``)."""
    ar = encode_canonical(a, moduli)
    br = encode_canonical(b, moduli)
    out = matmul_residues(ar, br, moduli)
    return decode_crt(out, moduli) if decode else out


def rns_matmul_centered(a, b, moduli, *, lut_channels=0) -> np.ndarray:
    """The fused fast path on CPU: centered encode of both operands, exact
    per-channel products, modular reduction, Garner, signed correction
    (``cuda_backend.py:514-539`` -> ``csrc/rns_cuda.cu:887-980``)."""
    ar = encode_centered(a, moduli)
    br = encode_centered(b, moduli)
    return fused_reduce_garner(channel_accumulators(ar, br), moduli,
                               lut_channels=lut_channels)


def exact_matmul(a, b) -> np.ndarray:
    """The closed form every RNS result must equal (``tests/test_cuda_backend.py:17-18``)."""
    return np.asarray(a, dtype=np.int64) @ np.asarray(b, dtype=np.int64)


# ---------------------------------------------------------------------------
# Adaptive channel prefix (``adaptive.py:15-52``, ``cuda_backend.py:541-622``)
# ---------------------------------------------------------------------------
def minimal_prefix_channels(moduli, absolute_bound: int, *, min_channels=2) -> int:
    """Smallest prefix length c >= min_channels with 2*bound < prod(prefix)."""
    mods = validate_moduli(moduli)
    if absolute_bound < 0:
        raise ValueError("absolute_bound must be non-negative")
    if not 2 <= min_channels <= len(mods):
        raise ValueError("min_channels must be between 2 and len(moduli)")
    running = 1
    for c, m in enumerate(mods, start=1):
        running *= m
        if c >= min_channels and 2 * absolute_bound < running:
            return c
    raise OverflowError(
        f"full moduli set cannot represent bound {absolute_bound}; "
        f"capacity={signed_capacity(mods)}")


def safe_l1_dot_bound(max_row_l1: int, max_abs_weight: int) -> int:
    """max_i sum_k |a_ik| * max|B| dominates every |(A@B)_ij|."""
    if max_row_l1 < 0 or max_abs_weight < 0:
        raise ValueError("bounds must be non-negative")
    return int(max_row_l1) * int(max_abs_weight)


def adaptive_select(a, max_abs_weight: int, moduli, *, min_channels=3):
    """(channels, bound, capacity) as ``select_adaptive_variant`` and the
    metadata of ``matmul_prepared_adaptive_fused`` compute them
    (``cuda_backend.py:577-622``)."""
    a64 = np.asarray(a, dtype=np.int64)
    row_l1 = int(np.abs(a64).sum(axis=1).max()) if a64.size else 0
    bound = safe_l1_dot_bound(row_l1, max_abs_weight)
    c = minimal_prefix_channels(moduli, bound, min_channels=min_channels)
    prefix = tuple(moduli)[:c]
    return c, bound, signed_capacity(prefix)


def adaptive_matmul(a, b, moduli, *, min_channels=3, lut_channels=2):
    """Adaptive fused product: the chosen prefix's centered reconstruction."""
    max_abs_w = int(np.abs(np.asarray(b, dtype=np.int64)).max())
    c, bound, cap = adaptive_select(a, max_abs_w, moduli, min_channels=min_channels)
    prefix = tuple(moduli)[:c]
    out = rns_matmul_centered(a, b, prefix, lut_channels=min(lut_channels, c))
    return out, {"channels": c, "bound": bound, "capacity": cap}


# ---------------------------------------------------------------------------
# Packed weights (no counterpart in the reference: its prepared weights keep
# one byte per channel, ``README.md:26-36``).  Pinned in tests/test_oracle.py
# by the round trip over every int16 value, the congruence for every
# candidate modulus, and packed_channel_residues against the residues of the
# exact product.
# ---------------------------------------------------------------------------
def pack16_split(values) -> tuple[np.ndarray, np.ndarray]:
    """(hi, lo) with hi = v >> 8 and lo = (v & 255) - 128, both in int8
    range for int16 v, so v = 256 hi + lo + 128."""
    v = np.asarray(values, dtype=np.int64)
    if v.size and (v.min() < -(1 << 15) or v.max() >= (1 << 15)):
        raise ValueError("packed weights hold int16 values")
    return v >> 8, (v & 255) - 128


def packed_channel_residues(a, b, moduli) -> np.ndarray:
    """Canonical residues [R, M, N] of A @ B computed the way the packed
    kernels do, channel by channel: with d = 256 mod m, a_c the centered
    residues of A and a'_c those of d * a_c, the sum
    a'_c @ hi + a_c @ lo + 128 * rowsum(a_c), reduced mod m."""
    mods = validate_moduli(moduli)
    hi, lo = pack16_split(b)
    a_c = encode_centered(a, mods).astype(np.int64)
    out = []
    for c, m in enumerate(mods):
        d = 256 % m
        r = np.mod(d * a_c[c], m)
        a2 = r - m * (r > m // 2)
        s = a2 @ hi + a_c[c] @ lo + 128 * a_c[c].sum(axis=1, keepdims=True)
        out.append(np.mod(s, m))
    return np.stack(out)
