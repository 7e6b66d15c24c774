"""Pins the CPU oracle (oracle/) before anything is compared with it.

Each check is chosen so a plausible slip in the oracle (dropped term, wrong
sign or index, transposed operand, off-by-one centering) fails it: closed
forms (the exact int64 product, v mod m), brute force on tiny inputs,
exhaustive small domains, and the reference's own known answers
(tests/test_reference.py, results/v0.5/adaptive_channels.json).
"""
import glob
import os
from math import prod

import numpy as np
import pytest
import torch

from oracle import c_oracle, linear_oracle
from oracle import rns_oracle as ro

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
DENSE4 = (255, 253, 251, 247)
SETS = [DENSE4, (251, 241, 239, 233), (127, 125, 121, 113), (3, 5, 7, 11), (2, 3, 5, 7, 11, 13),
        (254, 253, 251), (255, 253, 251, 247, 241, 239)]


# --------------------------------------------------------------------------
# encode
# --------------------------------------------------------------------------
@pytest.mark.parametrize("moduli", SETS)
def test_encode_centered_exhaustive_int8(moduli):
    v = np.arange(-128, 128, dtype=np.int64)
    r = ro.encode_centered(v, moduli).astype(np.int64)
    for c, m in enumerate(moduli):
        assert np.all((r[c] - v) % m == 0)              # congruent
        assert np.all(2 * r[c] <= m)                     # r <= m/2
        assert np.all(2 * r[c] > -m)                     # r > -m/2 (m/2 itself stays positive)


@pytest.mark.parametrize("moduli", SETS[:3])
def test_encode_centered_wide_sample(moduli):
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.integers(-2**31, 2**31, 20000, dtype=np.int64),
                        np.array([-2**31, 2**31 - 1, -32768, 32767, 0, -1, 1])])
    r = ro.encode_centered(v, moduli).astype(np.int64)
    for c, m in enumerate(moduli):
        assert np.all((r[c] - v) % m == 0)
        assert np.all((2 * r[c] <= m) & (2 * r[c] > -m))


def test_encode_canonical_range():
    v = np.arange(-300, 300)
    r = ro.encode_canonical(v, DENSE4).astype(np.int64)
    for c, m in enumerate(DENSE4):
        assert np.all((r[c] >= 0) & (r[c] < m) & ((r[c] - v) % m == 0))


# --------------------------------------------------------------------------
# decoders (reference known answers + exhaustive small range)
# --------------------------------------------------------------------------
def test_reference_signed_roundtrip():
    # tests/test_reference.py:11-14
    mods = (251, 241, 239, 233)
    v = np.arange(-10000, 10001, dtype=np.int64)
    np.testing.assert_array_equal(ro.decode_crt(ro.encode_canonical(v, mods), mods), v)


def test_reference_garner_known_answer():
    # tests/test_reference.py:49-57, fixture ref_garner_values.npz
    g = np.load(os.path.join(GOLDEN, "ref_garner_values.npz"))
    mods = tuple(int(m) for m in g["moduli"])
    np.testing.assert_array_equal(ro.decode_garner(ro.encode_centered(g["values"], mods), mods),
                                  g["values"])


@pytest.mark.parametrize("moduli", [(3, 5, 7), (2, 3, 5, 7), (4, 9, 25), (11, 13)])
def test_decoders_exhaustive_centered_range(moduli):
    p = prod(moduli)
    lo = -((p - 1) // 2) if p % 2 else -(p // 2) + 1
    v = np.arange(lo, p // 2 + 1, dtype=np.int64)           # every representable value
    for dec in (ro.decode_crt, ro.decode_garner):
        np.testing.assert_array_equal(dec(ro.encode_centered(v, moduli), moduli), v)
    # the value just outside the range wraps to the other end
    for dec in (ro.decode_crt, ro.decode_garner):
        assert int(dec(ro.encode_centered(np.array([p // 2 + 1]), moduli), moduli)[0]) == p // 2 + 1 - p


@pytest.mark.parametrize("moduli", SETS)
def test_garner_equals_crt_on_random_residues(moduli):
    rng = np.random.default_rng(7)
    r = np.stack([rng.integers(0, m, 500) for m in moduli])
    np.testing.assert_array_equal(ro.decode_garner(r, moduli), ro.decode_crt(r, moduli))


def test_garner_prefix_digits_are_a_prefix():
    # Reconstructing with the first c channels equals the full reconstruction
    # whenever the value fits the prefix range (what the adaptive prefix uses).
    v = np.arange(-8_096_632, 8_096_633, 40_507, dtype=np.int64)
    res = ro.encode_centered(v, DENSE4)
    np.testing.assert_array_equal(ro.decode_garner(res[:3], DENSE4[:3]), v)


# --------------------------------------------------------------------------
# residue GEMM / fused path
# --------------------------------------------------------------------------
def brute_force(a, b):
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), dtype=np.int64)
    for i in range(m):
        for j in range(n):
            s = 0
            for t in range(k):
                s += int(a[i, t]) * int(b[t, j])
            out[i, j] = s
    return out


def test_exact_matmul_is_brute_force():
    rng = np.random.default_rng(0)
    a = rng.integers(-127, 128, (3, 7))
    b = rng.integers(-127, 128, (7, 5))
    np.testing.assert_array_equal(ro.exact_matmul(a, b), brute_force(a, b))
    assert ro.exact_matmul(a, b).shape == (3, 5)


@pytest.mark.parametrize("lut", [0, 1, 2])
def test_centered_pipeline_matches_brute_force(lut):
    rng = np.random.default_rng(11 + lut)
    a = rng.integers(-127, 128, (5, 9)).astype(np.int8)
    b = rng.integers(-127, 128, (9, 4)).astype(np.int8)
    got = ro.rns_matmul_centered(a, b, DENSE4, lut_channels=lut)
    np.testing.assert_array_equal(got, brute_force(a, b))


def test_byte_lut_reduction_equals_modulo():
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.integers(-2**31, 2**31, 50000, dtype=np.int64),
                        np.array([-2**31, -2**31 + 1, 2**31 - 1, 0, -1])])
    lut = ro.compact_byte_mod_lut(DENSE4 + (2,))
    for c, m in enumerate(DENSE4 + (2,)):
        assert lut[c].max() < m and lut[c].min() >= 0
        np.testing.assert_array_equal(ro.canonical_mod_byte_lut(v, m, lut[c]), np.mod(v, m))


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))))
def test_golden_vectors(path):
    g = np.load(path)
    if "expected" not in g:
        return
    mods = tuple(int(m) for m in g["moduli"])
    np.testing.assert_array_equal(g["expected"], ro.exact_matmul(g["a"], g["b"]))
    np.testing.assert_array_equal(ro.rns_matmul_centered(g["a"], g["b"], mods), g["expected"])
    np.testing.assert_array_equal(ro.rns_matmul(g["a"], g["b"], mods), g["expected"])


def test_matmul_residues_channels_are_independent():
    # transposed or swapped operands would change this per-channel identity
    rng = np.random.default_rng(21)
    a = rng.integers(-100, 100, (4, 6))
    b = rng.integers(-100, 100, (6, 3))
    res = ro.matmul_residues(ro.encode_canonical(a, DENSE4), ro.encode_canonical(b, DENSE4), DENSE4)
    for c, m in enumerate(DENSE4):
        np.testing.assert_array_equal(res[c], np.mod(a @ b, m))


def test_c_oracle_matches_numpy_oracle():
    rng = np.random.default_rng(5)
    for (m, k, n), mods in [((9, 100, 13), DENSE4), ((1, 768, 64), DENSE4),
                            ((17, 64, 20), (3, 5, 7, 11, 13, 17, 19, 23, 29, 31))]:
        amax = 127 if prod(mods) > 2 * k * 127 * 127 else 2
        a = rng.integers(-amax, amax + 1, (m, k)).astype(np.int8)
        b = rng.integers(-amax, amax + 1, (k, n)).astype(np.int8)
        got = c_oracle.rns_matmul_centered(a, b, mods)
        np.testing.assert_array_equal(got, ro.rns_matmul_centered(a, b, mods))
        np.testing.assert_array_equal(got, ro.exact_matmul(a, b))


def test_overflowing_product_wraps_identically():
    # outside the range both oracles reduce mod P the same way (no silent
    # disagreement between the C and NumPy restatements)
    mods = (3, 5, 7, 11)
    rng = np.random.default_rng(8)
    a = rng.integers(-127, 128, (4, 16)).astype(np.int8)
    b = rng.integers(-127, 128, (16, 5)).astype(np.int8)
    exact = ro.exact_matmul(a, b)
    p = prod(mods)
    wrapped = np.mod(exact + p // 2, p) - p // 2
    np.testing.assert_array_equal(ro.rns_matmul_centered(a, b, mods), wrapped)
    np.testing.assert_array_equal(c_oracle.rns_matmul_centered(a, b, mods), wrapped)


# --------------------------------------------------------------------------
# moduli selection and adaptive prefix
# --------------------------------------------------------------------------
def test_dense_moduli_known_answer():
    # greedy dense prefix until the product reaches 2*K*127^2 + 1 (reference.py:238-265):
    # 255*253*251 = 16,193,265 holds K <= 501 (2*501*127^2 + 1 = 16,161,259), K = 502 needs 4
    for k in (502, 768, 4096, 123_992):
        assert ro.choose_moduli_for_dot(k, 127, 127, strategy="dense_coprime") == DENSE4
    assert ro.choose_moduli_for_dot(501, 127, 127, strategy="dense_coprime") == DENSE4[:3]
    assert len(ro.choose_moduli_for_dot(123_993, 127, 127, strategy="dense_coprime")) == 5


def test_reference_12bit_and_dense_cover():
    # tests/test_reference.py:40-46, 60-66
    mods = ro.choose_moduli_for_dot(768, 2047, 2047)
    assert prod(mods) > 2 * 768 * 2047 * 2047 and max(mods) <= 255
    mods = ro.choose_moduli_for_dot(768, 127, 127, strategy="dense_coprime")
    assert prod(mods) > 2 * 768 * 127 * 127


def test_validate_moduli_errors():
    with pytest.raises(ValueError):
        ro.validate_moduli(())
    with pytest.raises(ValueError):
        ro.validate_moduli((256, 3))
    with pytest.raises(ValueError):
        ro.validate_moduli((255, 253, 15))   # gcd(255, 15) = 15


def test_minimal_prefix_known_answers():
    # tests/test_reference.py:69-81 and adaptive_channels.json:20 (capacity 8,096,632)
    assert ro.minimal_prefix_channels(DENSE4, 5_000_000, min_channels=3) == 3
    assert ro.signed_capacity(DENSE4[:3]) == 8_096_632
    assert ro.minimal_prefix_channels(DENSE4, 8_096_632, min_channels=3) == 3
    assert ro.minimal_prefix_channels(DENSE4, 8_096_633, min_channels=3) == 4
    assert ro.minimal_prefix_channels(DENSE4, 0, min_channels=2) == 2
    with pytest.raises(OverflowError):
        ro.minimal_prefix_channels(DENSE4, ro.signed_capacity(DENSE4) + 1)
    with pytest.raises(ValueError):
        ro.minimal_prefix_channels(DENSE4, 10, min_channels=1)


def test_minimal_prefix_is_minimal_brute_force():
    rng = np.random.default_rng(2)
    for bound in rng.integers(0, 2_000_000_000, 200):
        c = ro.minimal_prefix_channels(DENSE4, int(bound), min_channels=2)
        ok = [cc for cc in range(2, 5) if all(abs(x) <= (prod(DENSE4[:cc]) - 1) // 2
                                              for x in (int(bound), -int(bound)))]
        assert c == ok[0]


def test_safe_l1_bound_dominates():
    # tests/test_reference.py:84-95
    rng = np.random.default_rng(77)
    a = rng.integers(-40, 41, size=(9, 31), dtype=np.int64)
    b = rng.integers(-50, 51, size=(31, 7), dtype=np.int64)
    bound = ro.safe_l1_dot_bound(int(np.abs(a).sum(1).max()), int(np.abs(b).max()))
    assert int(np.abs(a @ b).max()) <= bound


def test_adaptive_oracle_exact_low_and_high():
    rng = np.random.default_rng(41)
    w = rng.integers(-40, 41, (64, 32)).astype(np.int8)
    low = rng.integers(-8, 9, (16, 64)).astype(np.int8)
    high = rng.integers(-127, 128, (16, 64)).astype(np.int8)
    mods = ro.choose_moduli_for_dot(64, 127, 127, strategy="dense_coprime")
    for a in (low, high):
        out, meta = ro.adaptive_matmul(a, w, mods, min_channels=3)
        np.testing.assert_array_equal(out, ro.exact_matmul(a, w))
        assert meta["bound"] <= meta["capacity"]


# --------------------------------------------------------------------------
# RNSLinear float chain
# --------------------------------------------------------------------------
def test_linear_oracle_exact_power_of_two_case():
    # every quantity is a power-of-two multiple, so each float op is exact
    w = torch.tensor([[127.0, -64.0], [2.0, 127.0]]) / 128.0
    x = torch.tensor([[127.0, 0.0], [-127.0, 63.0]]) / 8.0
    bias = torch.tensor([0.5, -0.25])
    y, integer = linear_oracle.linear_forward(x, w, bias)
    # W is already on the int8 grid (per-row scale 1/128); x scale = 1/8
    np.testing.assert_array_equal(integer.numpy(), np.array([[127 * 127, 2 * 127],
                                                            [-127 * 127 - 64 * 63, -2 * 127 + 127 * 63]]))
    expected = integer.double() / 128.0 / 8.0 + bias.double()
    np.testing.assert_array_equal(y.double().numpy(), expected.numpy())


def test_linear_oracle_close_to_float_linear():
    gen = torch.Generator().manual_seed(5)
    w = torch.randn(48, 64, generator=gen) * 0.02
    b = torch.randn(48, generator=gen) * 0.01
    x = torch.randn(3, 7, 64, generator=gen)
    y, _ = linear_oracle.linear_forward(x, w, b)
    ref = torch.nn.functional.linear(x, w, b)
    # int8 quantisation of both operands: error well below 2% of the output scale
    assert y.shape == ref.shape
    assert float((y - ref).abs().max()) < 0.02 * float(ref.abs().max())


def test_quantize_is_half_to_even_and_clamped():
    s = torch.tensor([[0.5]])
    q = linear_oracle.quantize(torch.tensor([[0.25, 0.75, -0.25, 1000.0, -1000.0]]), s)
    assert q.tolist() == [[0, 2, 0, 127, -127]]


def test_scale_uses_gpu_reciprocal_rounding():
    """The oracle's scale is amax * fl32(1/127) (the rounding of torch's GPU
    ``tensor / 127.0``, which multiplies by the reciprocal of a CPU scalar),
    not the correctly rounded quotient.  Known answer for one amax, worked
    out with exact rational arithmetic: fl32(1/127) = 0x3C010204, the
    product rounds to 0x3B1BA940, and the float nearest amax / 127 is the
    next one up, 0x3B1BA941 (what the CPU division returns).  The GPU side
    of the claim is tested against torch's own GPU ops in
    tests/test_gpu_parity.py."""
    from fractions import Fraction

    def bits(t):
        return int(t.view(torch.int32).item()) & 0xFFFFFFFF

    def f32(b):
        return torch.tensor([b], dtype=torch.int64).to(torch.int32).view(torch.float32)

    amax = f32(1050309102)
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(127.0, dtype=torch.float32)
    assert bits(inv.reshape(1)) == 0x3C010204
    s = linear_oracle.symmetric_scale(amax.reshape(1, 1))
    assert bits(s) == 0x3B1BA940
    # the correctly rounded quotient is the neighbour above, by exact arithmetic
    exact = Fraction(float(amax.item())) / 127
    lo, hi = Fraction(float(f32(0x3B1BA940).item())), Fraction(float(f32(0x3B1BA941).item()))
    assert lo < exact < hi and hi - exact < exact - lo
    assert bits((amax / 127.0).reshape(1)) == 0x3B1BA941
    # and the product itself is the float nearest amax * fl32(1/127)
    prod = Fraction(float(amax.item())) * Fraction(float(inv.item()))
    assert abs(Fraction(float(s.item())) - prod) <= abs(Fraction(float(f32(0x3B1BA941).item())) - prod)


def test_adaptive_select_sums_each_row():
    """Known answers for ``adaptive_select`` (``cuda_backend.py:577-600``:
    bound = max over rows of sum_k |a_ik|, times max|B|; the first prefix of
    at least min_channels whose product exceeds twice the bound).  With
    moduli (3, 5, 7, 11, 13) the prefix products are 3, 15, 105, 1155,
    15015.  Case 1: row L1 36, column L1 at most 10, |B| <= 3: bound 108,
    2 * 108 >= 105 so 4 channels (capacity (1155 - 1) / 2 = 577); summing
    columns would give bound 30 and 3 channels.  Case 2: row L1 36 and 32,
    total 68, |B| <= 10: bound 360, 4 channels; summing every element would
    give 680 and 5 channels.  Case 3: no prefix holds the bound."""
    mods = (3, 5, 7, 11, 13)
    a1 = np.array([[9, -9, 9, -9], [1, 0, 0, 0]], dtype=np.int8)
    assert ro.adaptive_select(a1, 3, mods, min_channels=2) == (4, 108, 577)
    a2 = np.array([[9, 9, -9, 9], [8, -8, 8, 8]], dtype=np.int8)
    assert ro.adaptive_select(a2, 10, mods, min_channels=2) == (4, 360, 577)
    # the transposed operand and the whole-matrix sum give other answers
    assert ro.adaptive_select(a1.T.copy(), 3, mods, min_channels=2)[0] == 3
    assert ro.adaptive_select(a2.reshape(1, -1), 10, mods, min_channels=2)[0] == 5
    with pytest.raises(OverflowError):
        ro.adaptive_select(np.full((2, 64), 127, dtype=np.int8), 127, mods, min_channels=2)


def test_linear_oracle_row_sample_equals_full_rows():
    gen = torch.Generator().manual_seed(8)
    w = torch.randn(24, 40, generator=gen) * 0.02
    b = torch.randn(24, generator=gen)
    x = torch.randn(5, 3, 40, generator=gen)
    full, full_int = linear_oracle.linear_forward(x, w, b)
    rows = [0, 7, 14]
    part, part_int = linear_oracle.linear_forward(x, w, b, rows=rows)
    assert torch.equal(part, full.reshape(-1, 24)[rows])
    assert torch.equal(part_int, full_int[rows])


def test_torch_cpu_restatement_is_exact():
    """oracle/torch_cpu_oracle.py (the reference's TorchReferenceBackend
    path, timed as bench.py's all-cores CPU baseline) against the closed
    form, the NumPy oracle's encoder and CRT decoder, and the reference's
    known CRT answer (tests/test_torch_reference.py:6-13 shape)."""
    from oracle import torch_cpu_oracle as tco

    gen = torch.Generator().manual_seed(13)
    a = torch.randint(-127, 128, (9, 40), generator=gen, dtype=torch.int8)
    b = torch.randint(-127, 128, (40, 11), generator=gen, dtype=torch.int8)
    mods = (255, 253, 251, 247)
    np.testing.assert_array_equal(tco.matmul_int8(a, b, mods).numpy(), ro.exact_matmul(a.numpy(), b.numpy()))
    np.testing.assert_array_equal(tco.encode(a, mods).numpy(), ro.encode_canonical(a.numpy(), mods))
    res = ro.encode_canonical(ro.exact_matmul(a.numpy(), b.numpy()), mods)
    np.testing.assert_array_equal(tco.decode(torch.from_numpy(res.astype(np.uint8)), mods).numpy(),
                                  ro.decode_crt(res, mods))
    big_p, coeffs = tco.crt_coefficients(mods)
    assert big_p == 3_999_736_455
    assert all(c % m == 1 and all(c % o == 0 for o in mods if o != m) for c, m in zip(coeffs, mods))


def test_pack16_split_round_trip_every_int16():
    v = np.arange(-(1 << 15), 1 << 15, dtype=np.int64)
    hi, lo = ro.pack16_split(v)
    assert hi.min() == -128 and hi.max() == 127 and lo.min() == -128 and lo.max() == 127
    np.testing.assert_array_equal(256 * hi + lo + 128, v)
    # the bytes the device stores: two's-complement high byte, low byte with its top bit flipped
    np.testing.assert_array_equal(hi & 0xFF, (v >> 8) & 0xFF)
    np.testing.assert_array_equal(lo & 0xFF, (v & 0xFF) ^ 0x80)
    with pytest.raises(ValueError):
        ro.pack16_split([1 << 15])


@pytest.mark.parametrize("strategy", ["dense_coprime", "large_primes", "small_primes"])
def test_packed_congruence_every_modulus(strategy):
    """v = (256 mod m) hi + lo + 128 (mod m) for every int16 v and every
    candidate modulus: the identity the packed kernels rely on."""
    v = np.arange(-(1 << 15), 1 << 15, dtype=np.int64)
    hi, lo = ro.pack16_split(v)
    for m in ro.candidates_for_strategy(strategy):
        np.testing.assert_array_equal(np.mod((256 % m) * hi + lo + 128, m), np.mod(v, m))


@pytest.mark.parametrize("moduli,a_lim,b_lim", [((255, 253, 251, 247, 241, 239), 32767, 32767),
                                                ((255, 253, 251, 247, 241), 2047, 32767),
                                                ((255, 253, 251, 247), 127, 127)])
def test_packed_channel_residues_equal_exact_product(moduli, a_lim, b_lim):
    """The packed kernels' per-channel sum (a' hi + a lo + 128 rowsum a)
    reduces to the residues of the exact product, including the int16
    extremes; dropping the row term or using d = m - 256 fails."""
    rng = np.random.default_rng(7)
    a = rng.integers(-a_lim, a_lim + 1, size=(9, 70))
    b = rng.integers(-b_lim - 1, b_lim + 1, size=(70, 11))
    b[0, 0], b[1, 1], a[0, 0] = -b_lim - 1, b_lim, -a_lim
    want = ro.encode_canonical(ro.exact_matmul(a, b), moduli).astype(np.int64)
    np.testing.assert_array_equal(ro.packed_channel_residues(a, b, moduli), want)
    # a planted mistake in the restatement (no row term) is caught
    hi, lo = ro.pack16_split(b)
    ac = ro.encode_centered(a, moduli).astype(np.int64)
    m = moduli[0]
    r = np.mod((256 % m) * ac[0], m)
    wrong = np.mod((r - m * (r > m // 2)) @ hi + ac[0] @ lo, m)
    assert not np.array_equal(wrong, want[0])
