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
    mods = tuple(int(m) for m in moduli)
    if not mods:
        raise ValueError("moduli must not be empty")
    if any(not 2 <= m <= 255 for m in mods):
        raise ValueError("every modulus must be in [2, 255]")
    for i, left in enumerate(mods):
        for right in mods[i + 1:]:
            if gcd(left, right) != 1:
                raise ValueError(f"moduli are not pairwise coprime: {left}, {right}")
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
    return (prod(validate_moduli(moduli)) - 1) // 2


def minimal_prefix_channels(moduli: Iterable[int], absolute_bound: int, *,
                            min_channels: int = 2) -> int:
    mods = validate_moduli(moduli)
    if absolute_bound < 0:
        raise ValueError("absolute_bound must be non-negative")
    if not 2 <= min_channels <= len(mods):
        raise ValueError("min_channels must be between 2 and len(moduli)")
    running = 1
    for count, m in enumerate(mods, start=1):
        running *= m
        if count >= min_channels and 2 * absolute_bound < running:
            return count
    raise OverflowError(
        f"full moduli set cannot represent bound {absolute_bound}; "
        f"capacity={signed_capacity(mods)}")


def safe_l1_dot_bound(max_row_l1: int, max_abs_weight: int) -> int:
    if max_row_l1 < 0 or max_abs_weight < 0:
        raise ValueError("bounds must be non-negative")
    return int(max_row_l1) * int(max_abs_weight)


def centered_accumulator_bound(k: int, moduli: Iterable[int]) -> int:
    """Largest |int32 accumulator| of one channel: K * max(floor(m/2))^2
    (``cuda_backend.py:210-214``)."""
    mods = validate_moduli(moduli)
    return int(k) * max(m // 2 for m in mods) ** 2
