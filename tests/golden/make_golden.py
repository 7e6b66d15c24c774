"""Writes the golden vectors under tests/golden/ (committed .npz fixtures).

Every expected output is the exact int64 product A @ B computed with plain
NumPy integer matmul: the closed form the reference's own tests use as their
oracle (tests/test_cuda_backend.py:17-18, docs/CORRECTNESS_GUARDS.md:5-9).
Inputs are seeded so the files can be regenerated bit for bit:

    python tests/golden/make_golden.py

Cases follow the reference tests and BASELINE configs at sizes the CPU
finishes instantly:
  ref_residue_matmul   tests/test_reference.py:17-26   (seed 4, 13x29x17)
  ref_end_to_end       tests/test_reference.py:29-37   (seed 5, 7x19x11, |v|<=32)
  ref_garner_values    tests/test_reference.py:49-57   (seed 123, +-1e6 values)
  c1_slice             config C1 rows 0..15 (M=16, K=N=768 -> N=64 slice)
  c2_qkv_small         config C2 quantisation recipe at K=768, N=3x32, M=16
  c3_decode            config C3: 4 requests of M=1, K=768, N=96
  int12_wide           tests/test_cuda_backend.py:73-94 (int16 +-2047, 24x64x32)
  adversarial_k4096    config C5 all +-127 inputs at K=4096 (M=2, N=16)
  ragged_k100          K=100, N=37 (no multiple-of-4/16/64 shape)
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
DENSE4 = (255, 253, 251, 247)


def exact(a, b):
    return np.asarray(a, dtype=np.int64) @ np.asarray(b, dtype=np.int64)


def quantize_per_row(w: np.ndarray) -> np.ndarray:
    """Symmetric int8 per output channel (rows of W [N, K]), float32 math."""
    w = w.astype(np.float32)
    amax = np.abs(w).max(axis=1, keepdims=True)
    scale = np.maximum(amax / np.float32(127.0), np.finfo(np.float32).eps).astype(np.float32)
    return np.clip(np.rint(w / scale), -127, 127).astype(np.int8)


def cases():
    out = {}
    rng = np.random.default_rng(4)
    a = rng.integers(-127, 128, (13, 29), dtype=np.int16).astype(np.int8)
    b = rng.integers(-127, 128, (29, 17), dtype=np.int16).astype(np.int8)
    out["ref_residue_matmul"] = dict(a=a, b=b, moduli=np.array((251, 241, 239, 233)))

    rng = np.random.default_rng(5)
    a = rng.integers(-32, 33, (7, 19), dtype=np.int16).astype(np.int8)
    b = rng.integers(-32, 33, (19, 11), dtype=np.int16).astype(np.int8)
    out["ref_end_to_end"] = dict(a=a, b=b, moduli=np.array((251, 241, 239, 233)))

    rng = np.random.default_rng(2025)
    a = rng.integers(-127, 128, (16, 768), dtype=np.int16).astype(np.int8)
    b = rng.integers(-127, 128, (768, 64), dtype=np.int16).astype(np.int8)
    out["c1_slice"] = dict(a=a, b=b, moduli=np.array(DENSE4))

    rng = np.random.default_rng(17)
    w = rng.normal(0.0, 0.02, (96, 768)).astype(np.float16)  # q|k|v rows, 32 each
    x = rng.normal(0.0, 1.0, (16, 768)).astype(np.float32)
    xs = np.maximum(np.abs(x).max(axis=1, keepdims=True) / np.float32(127.0),
                    np.finfo(np.float32).eps).astype(np.float32)
    xq = np.clip(np.rint(x / xs), -127, 127).astype(np.int8)
    out["c2_qkv_small"] = dict(a=xq, b=quantize_per_row(w).T.copy(), moduli=np.array(DENSE4))

    rng = np.random.default_rng(3)
    a = rng.integers(-127, 128, (4, 768), dtype=np.int16).astype(np.int8)
    b = rng.integers(-127, 128, (768, 96), dtype=np.int16).astype(np.int8)
    out["c3_decode"] = dict(a=a, b=b, moduli=np.array(DENSE4))

    rng = np.random.default_rng(12)
    a = rng.integers(-2047, 2048, (24, 64), dtype=np.int16)
    b = rng.integers(-2047, 2048, (64, 32), dtype=np.int16)
    # choose_moduli_for_dot(64, 2047, 2047, strategy="dense_coprime")
    out["int12_wide"] = dict(a=a, b=b, moduli=np.array((255, 253, 251, 247)))

    signs_a = np.where(np.random.default_rng(9).random((2, 4096)) < 0.5, -127, 127)
    a = np.concatenate([np.full((1, 4096), 127), signs_a[:1]], axis=0).astype(np.int8)
    b = np.concatenate([np.full((4096, 8), 127), -np.full((4096, 8), 127)], axis=1).astype(np.int8)
    out["adversarial_k4096"] = dict(a=a, b=b, moduli=np.array(DENSE4))

    rng = np.random.default_rng(100)
    a = rng.integers(-127, 128, (5, 100), dtype=np.int16).astype(np.int8)
    b = rng.integers(-127, 128, (100, 37), dtype=np.int16).astype(np.int8)
    out["ragged_k100"] = dict(a=a, b=b, moduli=np.array((255, 253, 251)))

    for case in out.values():
        case["expected"] = exact(case["a"], case["b"])

    rng = np.random.default_rng(123)
    out["ref_garner_values"] = dict(
        values=rng.integers(-1_000_000, 1_000_001, size=(17, 13), dtype=np.int64),
        moduli=np.array(DENSE4))
    return out


def main():
    for name, arrays in cases().items():
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        print("wrote", name)


if __name__ == "__main__":
    main()
