"""Torch-CPU restatement of the reference's readable torch backend.

TEST INFRASTRUCTURE ONLY (see ``oracle/rns_oracle.py``): used by
``bench.py``'s CPU baseline (the reference CPU path at all host threads)
and checked by ``tests/test_oracle.py``.

Restates ``TorchReferenceBackend.matmul_int8``
(``src/rns_llm/backends/torch_reference.py:72-84``) with its three steps:

  * ``encode`` (``:17-23``): canonical residues ``remainder(v, m)`` in
    [0, m), one plane per modulus, as uint8;
  * ``matmul_residues`` (``:25-43``): per channel an int64 matrix product of
    the residue planes, reduced ``remainder(., m)`` to uint8;
  * ``decode`` (``:45-70``): CRT, ``sum_c r_c * coefficient_c`` accumulated
    modulo P, then the signed correction ``x > P // 2 -> x - P``.

The CRT coefficients are ``(P / m_c) * ((P / m_c)^-1 mod m_c)``, the
reference's ``crt_constants`` (``reference.py:43-55``), computed here with
Python integers.  Pinned against the exact int64 product and the NumPy
oracle's CRT decoder.
"""
from __future__ import annotations

from math import prod

import torch


def crt_coefficients(moduli) -> tuple[int, tuple[int, ...]]:
    big_p = prod(moduli)
    coeffs = []
    for m in moduli:
        cofactor = big_p // m
        coeffs.append(cofactor * pow(cofactor % m, -1, m) % big_p)
    return big_p, tuple(coeffs)


def encode(values: torch.Tensor, moduli) -> torch.Tensor:
    mods = torch.tensor(tuple(moduli), dtype=torch.int64)
    shape = (len(moduli),) + (1,) * values.ndim
    return torch.remainder(values.to(torch.int64).unsqueeze(0), mods.view(shape)).to(torch.uint8)


def matmul_residues(a_res: torch.Tensor, b_res: torch.Tensor, moduli) -> torch.Tensor:
    planes = [torch.remainder(a_res[c].to(torch.int64) @ b_res[c].to(torch.int64), m).to(torch.uint8)
              for c, m in enumerate(moduli)]
    return torch.stack(planes, dim=0)


def decode(residues: torch.Tensor, moduli) -> torch.Tensor:
    big_p, coeffs = crt_coefficients(moduli)
    if big_p > (2**63 - 1) // max(moduli):
        raise OverflowError("CRT product too large for an int64 decoder")
    acc = torch.zeros(residues.shape[1:], dtype=torch.int64)
    for c, coeff in enumerate(coeffs):
        acc = torch.remainder(acc + residues[c].to(torch.int64) * coeff, big_p)
    return torch.where(acc > big_p // 2, acc - big_p, acc)


def matmul_int8(a: torch.Tensor, b: torch.Tensor, moduli) -> torch.Tensor:
    """int8 A [M, K] x int8 B [K, N] -> exact int64 [M, N] through residues."""
    return decode(matmul_residues(encode(a, moduli), encode(b, moduli), moduli), moduli)
