"""Host-side moduli logic of the RNS path: validation, candidate orders,
greedy selection for a dot product, and the adaptive-prefix bounds.

Mirrors the public functions of the reference's ``src/rns_llm/reference.py``
(``validate_moduli`` 11-23, candidate tables 190-230, ``choose_moduli_for_dot``
238-265) and ``src/rns_llm/adaptive.py`` (9-52) with the same names, argument
meaning and exception types.  The device constants themselves (Barrett
reciprocals, Garner coefficients, prefix products) are built natively by
``rnsmx_moduli_init``.
"""
from __future__ import annotations

from itertools import accumulate, combinations
from math import gcd, prod
from typing import Iterable

LARGE_PRIME_MODULI: tuple[int, ...] = (
    251, 241, 239, 233, 229, 227, 223, 211, 199, 197, 193, 191, 181, 179, 173,
    167, 163, 157, 151, 149, 139, 137, 131, 127,
)
DENSE_COPRIME_MODULI: tuple[int, ...] = (
    255, 253, 251, 247, 241, 239, 233, 229, 227, 223, 211, 199, 197, 193, 191,
    181, 179, 173, 167, 163, 157, 151, 149, 139, 137, 131, 127, 125, 121,
)
SMALL_PRIME_MODULI: tuple[int, ...] = (
    3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37, 41, 43, 47, 53, 59, 61, 67, 71,
    73, 79, 83, 89, 97, 101, 103, 107, 109, 113, 127, 131, 137, 139, 149, 151,
    157, 163, 167, 173, 179, 181, 191, 193, 197, 199, 211, 223, 227, 229, 233,
    239, 241, 251,
)
HARDWARE_FRIENDLY_MODULI = LARGE_PRIME_MODULI

_STRATEGIES = {
    "large_primes": LARGE_PRIME_MODULI,
    "dense_coprime": DENSE_COPRIME_MODULI,
    "small_primes": SMALL_PRIME_MODULI,
}


def validate_moduli(moduli: Iterable[int]) -> tuple[int, ...]:
    """The moduli as a tuple of ints, each in [2, 255] (one residue byte) and
    coprime to every other; ValueError otherwise."""
    mods = tuple(map(int, moduli))
    if len(mods) == 0:
        raise ValueError("an RNS needs at least one modulus")
    out_of_range = [m for m in mods if m < 2 or m > 255]
    if out_of_range:
        raise ValueError(f"moduli must lie in [2, 255] (residues are bytes): {out_of_range}")
    shared = next(((x, y) for x, y in combinations(mods, 2) if gcd(x, y) > 1), None)
    if shared is not None:
        raise ValueError(f"moduli {shared[0]} and {shared[1]} share a factor; they must be pairwise coprime")
    return mods


def candidates_for_strategy(strategy: str) -> tuple[int, ...]:
    try:
        return _STRATEGIES[strategy]
    except KeyError:
        raise ValueError(f"unknown moduli strategy: {strategy}") from None


def dot_product_bound(k: int, max_abs_a: int, max_abs_b: int) -> int:
    if k <= 0:
        raise ValueError("k must be positive")
    if max_abs_a < 0 or max_abs_b < 0:
        raise ValueError("absolute bounds must be non-negative")
    return int(k) * int(max_abs_a) * int(max_abs_b)


def choose_moduli_for_dot(k: int, max_abs_a: int, max_abs_b: int, *,
                          candidates: Iterable[int] | None = None,
                          strategy: str = "large_primes") -> tuple[int, ...]:
    """Greedy pairwise-coprime prefix of the candidates whose product reaches
    2 * K * max|a| * max|b| + 1 (exact signed reconstruction)."""
    target = 2 * dot_product_bound(k, max_abs_a, max_abs_b) + 1
    pool = tuple(candidates) if candidates is not None else candidates_for_strategy(strategy)
    chosen: list[int] = []
    running = 1
    for m in pool:
        m = int(m)
        if not 2 <= m <= 255 or any(gcd(m, c) != 1 for c in chosen):
            continue
        chosen.append(m)
        running *= m
        if running >= target:
            return tuple(chosen)
    raise ValueError(f"candidate moduli cannot cover required range {target}")


def signed_capacity(moduli: Iterable[int]) -> int:
    """Largest |x| the centered range of the moduli set holds: (P - 1) // 2."""
    return (prod(validate_moduli(moduli)) - 1) // 2


def minimal_prefix_channels(moduli: Iterable[int], absolute_bound: int, *,
                            min_channels: int = 2) -> int:
    """Length of the shortest prefix, at least ``min_channels`` long, whose
    product P_c holds every value of magnitude up to ``absolute_bound``
    exactly (strictly: 2 * bound < P_c); OverflowError when the whole set
    does not."""
    mods = validate_moduli(moduli)
    if absolute_bound < 0:
        raise ValueError("absolute_bound cannot be negative")
    if min_channels < 2 or min_channels > len(mods):
        raise ValueError(f"min_channels must be in [2, {len(mods)}]")
    products = list(accumulate(mods, lambda p, m: p * m))
    for c in range(min_channels, len(mods) + 1):
        if products[c - 1] > 2 * absolute_bound:
            return c
    raise OverflowError(
        f"bound {absolute_bound} exceeds what the full moduli set represents "
        f"(capacity={signed_capacity(mods)})")


def safe_l1_dot_bound(max_row_l1: int, max_abs_weight: int) -> int:
    """|sum_k a_k b_k| <= (sum_k |a_k|) * max|b|: the bound the adaptive
    prefix must hold."""
    if min(max_row_l1, max_abs_weight) < 0:
        raise ValueError("max_row_l1 and max_abs_weight cannot be negative")
    return int(max_row_l1) * int(max_abs_weight)


def centered_accumulator_bound(k: int, moduli: Iterable[int]) -> int:
    """Largest |int32 accumulator| of one channel: K * max(floor(m/2))^2
    (``cuda_backend.py:210-214``)."""
    mods = validate_moduli(moduli)
    return int(k) * max(m // 2 for m in mods) ** 2
