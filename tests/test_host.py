"""CPU tests of the host side: the C-ABI library loads and exports every
symbol include/rnsmx.h declares; its host-only constant builders agree with
the oracle; the package's host logic keeps the reference's results and
exception types; torch-mode QKV fusion mirrors tests/test_qkv_fusion.py."""
import ctypes
import os
import re
from math import prod

import numpy as np
import pytest
import torch
from torch import nn

from oracle import rns_oracle as ro
from rns_llm_amd import _native, moduli as host_moduli
from rns_llm_amd.backends.hip_backend import HipRNSBackend, RNSWorkspace
from rns_llm_amd.layers import CachedRNSQKV, RNSLinear, RNSQKVProjection

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rnsmx.h")
DENSE4 = (255, 253, 251, 247)


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(rnsmx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    names = declared_symbols()
    assert names, "header declares no entry points"
    for name in names:
        assert hasattr(lib, name), f"librnsmx.so does not export {name}"
    assert sorted(_native.EXPORTED_SYMBOLS) == names


def test_abi_struct_layout_matches_header():
    # sizeof(rnsmx_moduli_t) with natural alignment: 4 + 4*10*4 + 4*100 + pad + 8*11 + 2*4*10
    assert ctypes.sizeof(_native.Moduli) == 4 + 40 * 4 + 400 + 4 + 88 + 80
    assert _native.lib().rnsmx_abi_version() == _native.ABI_VERSION


def gemm_plan(m, n, k, channels=4, raw_a=1):
    out = _native.Plan()
    _native.check(_native.lib().rnsmx_gemm_plan(m, n, k, channels, raw_a, ctypes.byref(out)))
    return out.as_tuple()


# (M, N, K, channels) -> (kind, mb, nb, ks, splits): kind 1 stream, 2 MFMA,
# 3 LDS-staged (256 x 64), 4 stream with 8-step chunks, 5 MFMA with 48-column
# tiles, 7 LDS-staged (256 x 96);
# splits: workgroups sharing each output tile's K range
PLANS = [
    ((1, 2304, 768, 4), (1, 1, 1, 3, 1, 0)),       # decode: stream, 3 waves split 12 K steps
    ((64, 2304, 768, 4), (1, 1, 1, 4, 1, 0)),      # stream up to 64 rows at short K, 4 waves from 16 rows
    ((8, 2304, 768, 4), (1, 1, 1, 3, 1, 0)),       # under 16 rows: 3 waves (12 K steps in chunks of 4)
    ((96, 2304, 768, 4), (1, 2, 1, 3, 1, 0)),      # stream: 432 tiles of 32 x 16
    ((128, 768, 768, 4), (1, 1, 1, 4, 1, 0)),      # stream: 384 tiles of 16 x 16 (at most 768)
    ((80, 2304, 768, 4), (1, 1, 1, 4, 1, 0)),      # 720 tiles of 16 x 16
    ((128, 2304, 768, 4), (5, 2, 1, 4, 1, 0)),     # 576 stream tiles: MFMA, 32 x 48 (192 tiles)
    ((256, 1536, 768, 4), (5, 2, 1, 4, 1, 0)),     # 32 x 48 fills 256 CUs (32 x 64: 192)
    ((256, 3072, 768, 4), (5, 4, 1, 4, 1, 0)),     # 64 x 48, 256 tiles, ties 64 x 64 on rows
    ((256, 3072, 1024, 4), (5, 4, 1, 4, 1, 0)),
    ((128, 2304, 768, 6), (2, 2, 1, 4, 1, 0)),     # 48-column tiles only up to 4 channels
    ((224, 2304, 768, 4), (2, 2, 1, 4, 1, 0)),     # 252 tiles of 32 rows: one round
    ((256, 2304, 768, 4), (2, 3, 1, 4, 1, 0)),     # headline: 216 tiles of 48 rows
    ((320, 2304, 768, 4), (2, 3, 1, 4, 1, 0)),     # 252 tiles of 48 rows
    ((384, 2304, 768, 4), (2, 4, 1, 0, 1, 0)),     # 64 rows (216 tiles) tie 32 rows (2 rounds)
    ((256, 4608, 768, 4), (2, 3, 1, 4, 1, 0)),     # no height fits one round: 48 rows (2 rounds)
    ((256, 2304, 768, 6), (2, 4, 1, 0, 1, 0)),     # no 48-row tile past 4 channels
    ((4096, 2304, 768, 4), (2, 4, 1, 0, 1, 0)),    # C4 QKV: over 512 tiles at every height
    ((1, 12288, 4096, 4), (4, 1, 1, 4, 1, 0)),     # C5 decode: stream with 8-step chunks
    ((16, 12288, 4096, 4), (4, 1, 1, 4, 1, 0)),    # long K, 16 rows: stream, 8-step chunks
    ((16, 2048, 2048, 4), (4, 1, 1, 4, 1, 0)),     # K = 2048, up to 32 rows: 8-step chunks
    ((48, 2048, 2048, 4), (1, 1, 1, 4, 1, 0)),     # past 32 rows: 4-step chunks
    ((1, 12288, 4096, 6), (2, 2, 1, 4, 1, 0)),     # no 8-step chunks past 4 channels: 192 MFMA tiles
    ((1, 4096, 4096, 6), (1, 1, 1, 4, 1, 0)),      # 64 MFMA tiles: stream, 4-step chunks
    ((48, 2304, 768, 6), (1, 1, 1, 4, 1, 0)),
    ((64, 4096, 4096, 6), (2, 2, 1, 4, 1, 0)),     # past 48 rows
    ((224, 2304, 768, 10), (2, 2, 1, 0, 1, 0)),    # 10 channels: the tile's default ring (3 steps)
    ((96, 48, 64, 10), (1, 1, 1, 4, 1, 0)),        # raw int8 past 4 channels: the raw stream rule
    ((96, 768, 768, 6), (1, 1, 1, 4, 1, 0)),
    ((32, 12288, 4096, 6), (2, 2, 1, 4, 1, 0)),    # no 8-step chunks past 4 channels: MFMA from 128 tiles
    ((256, 2304, 768, 10), (2, 4, 1, 0, 1, 0)),
    ((32, 12288, 4096, 4), (5, 2, 1, 4, 1, 0)),    # long K, wide N: MFMA, 32 rows, three waves (256 tiles)
    ((48, 12288, 4096, 4), (5, 3, 1, 4, 1, 0)),
    ((64, 12288, 4096, 4), (5, 4, 1, 4, 1, 0)),
    ((128, 12288, 4096, 4), (3, 0, 0, 0, 1, 0)),   # K = 4096, 192 LDS tiles: three quarters of a round
    ((256, 12288, 4096, 4), (3, 0, 0, 0, 1, 0)),
    ((128, 12288, 8192, 4), (2, 4, 1, 0, 2, 0)),   # K = 8192: MFMA tiles (K in two halves)
    ((256, 4096, 4096, 4), (2, 4, 1, 0, 1, 0)),    # 64 LDS tiles: MFMA
    ((64, 4096, 4096, 4), (5, 2, 1, 4, 1, 0)),     # 1024 stream tiles at long K: MFMA
    ((64, 4096, 8192, 4), (2, 2, 1, 4, 2, 0)),     # K = 8192: four waves, K in two halves
    ((512, 12288, 4096, 4), (7, 0, 0, 0, 1, 0)),   # LDS-staged, 256 x 96 tiles: 256, one round
    ((2048, 12288, 4096, 4), (7, 0, 0, 0, 1, 0)),  # 4 rounds of 96 columns against 6 of 64
    ((1024, 12288, 4096, 4), (7, 0, 0, 0, 1, 0)),
    ((2048, 4096, 4096, 4), (3, 0, 0, 0, 1, 0)),   # 2 rounds of 64 columns against 1.34 of 96
    ((2048, 12288, 4096, 6), (2, 4, 1, 0, 1, 0)),  # the LDS kernel holds at most 4 channels
    # K split over workgroups: few tiles and long K
    ((1, 768, 16384, 4), (4, 1, 1, 1, 8, 0)),    # decode: 8 one-wave workgroups per 16 x 16 tile
    ((1, 768, 4096, 4), (4, 1, 1, 1, 4, 0)),     # 16 K steps per split: 4 splits
    ((1, 768, 2048, 4), (4, 1, 1, 4, 1, 0)),     # 4 waves of 8-step chunks (2 one-wave splits lose)
    ((1, 2304, 16384, 4), (4, 1, 1, 4, 1, 0)),   # 144 stream tiles: no split
    ((256, 256, 8192, 4), (2, 2, 1, 4, 8, 0)),   # 32 tiles: 8 splits (256 workgroups)
    ((256, 768, 4096, 4), (2, 2, 1, 4, 4, 0)),   # 96 tiles: at most 512 workgroups -> 4
    ((512, 512, 8192, 4), (2, 2, 1, 4, 2, 0)),   # 128 tiles, K >= 8192: 2
    ((2048, 768, 16384, 4), (2, 4, 1, 0, 2, 0)),
    ((256, 256, 8192, 6), (2, 2, 1, 4, 1, 0)),   # the exchange holds at most 4 channels
    ((640, 12288, 4096, 4), (3, 0, 0, 0, 4, 1)),    # 576 LDS tiles: the last 64 split in 4
    ((1280, 12288, 4096, 4), (3, 0, 0, 0, 1, 0)),   # 960 tiles: 192 in the last round, not split
    ((512, 12288, 1024, 4), (7, 0, 0, 0, 1, 0)),    # short K: LDS only for full rounds (256 x 96: one)
    ((384, 12288, 1024, 4), (7, 0, 0, 0, 1, 0)),    # 2 x 128 tiles of 256 x 96 (the second row half padding)
    ((384, 12288, 768, 4), (7, 0, 0, 0, 1, 0)),
    ((256, 12288, 1024, 4), (3, 0, 0, 0, 1, 0)),    # 192 tiles of 256 x 64: one round from 144
    ((256, 8192, 1024, 4), (2, 4, 1, 0, 1, 0)),     # 128 of them: MFMA
    ((1536, 3072, 768, 4), (7, 0, 0, 0, 1, 0)),     # 192 wide tiles, one round (288 narrow: two)
    ((512, 4608, 768, 4), (3, 0, 0, 0, 1, 0)),      # 144 tiles at K = 768
    ((384, 3072, 4096, 4), (2, 4, 1, 0, 1, 0)),     # 288 MFMA tiles beat 384 of 48 rows at long K
    ((512, 3072, 2048, 4), (5, 4, 1, 4, 1, 0)),     # none under 320: the most up to 512
    ((192, 768, 768, 4), (1, 1, 1, 4, 1, 0)),       # stream up to 192 rows at short K, 576 tiles
    ((192, 768, 4096, 4), (2, 2, 1, 4, 4, 0)),      # at K = 4096 the MFMA kernel's K split
    ((384, 3072, 768, 4), (5, 3, 1, 4, 1, 0)),      # rows tie (96 per CU): the fuller last round, 512 tiles
    ((32, 8192, 768, 4), (5, 2, 1, 4, 1, 0)),       # 1024 stream tiles at short K too: MFMA
    ((1, 8192, 2048, 4), (1, 1, 1, 4, 1, 0)),       # K = 2048, 512 tiles: 4-step chunks
    ((192, 8192, 4096, 4), (3, 0, 0, 0, 1, 0)),     # K = 4096: one LDS round from 128 tiles
]


@pytest.mark.parametrize("shape,plan", PLANS)
def test_gemm_plan_rules(shape, plan):
    """The kernel choice at the boundaries of its rules (host logic of the
    library; the GPU tests check that every choice computes the exact
    product)."""
    m, n, k, channels = shape
    assert gemm_plan(m, n, k, channels) == plan


def test_gemm_plan_residue_plane_activations():
    # int16 / int32 activations (encoded per channel) with 4 or 6 channels:
    # the 128 x 128 LDS kernel from 129 rows (K a multiple of 256)
    assert gemm_plan(512, 12288, 4096, 6, raw_a=0) == (8, 0, 0, 0, 2, 1)   # 384 tiles: the last 128 split
    assert gemm_plan(2048, 12288, 4096, 6, raw_a=0) == (8, 0, 0, 0, 1, 0)  # six full rounds
    assert gemm_plan(256, 16384, 1024, 5, raw_a=0) == (8, 0, 0, 0, 1, 0)   # 5 channels: capacity 6
    assert gemm_plan(512, 12288, 4096, 4, raw_a=0) == (8, 0, 0, 0, 2, 1)   # 4 channels
    assert gemm_plan(512, 4096, 4096, 6, raw_a=0) == (8, 0, 0, 0, 2, 0)    # 128 tiles: every tile in two
    assert gemm_plan(256, 12288, 4096, 6, raw_a=0) == (8, 0, 0, 0, 1, 0)   # 192 tiles: no split
    assert gemm_plan(256, 4096, 1024, 6, raw_a=0)[0] == 2                  # 64 tiles x 16 steps: MFMA kernel
    assert gemm_plan(1024, 4096, 1024, 6, raw_a=0) == (8, 0, 0, 0, 1, 0)   # 256 tiles x 16 steps
    assert gemm_plan(512, 12288, 4096, 6)[0] == 2                          # raw int8: MFMA kernel
    assert gemm_plan(64, 12288, 4096, 6, raw_a=0) == (8, 0, 0, 0, 2, 0)    # 96 tiles: K in two halves
    assert gemm_plan(128, 12288, 4096, 6, raw_a=0) == (8, 0, 0, 0, 2, 0)
    assert gemm_plan(48, 12288, 4096, 6, raw_a=0) == (8, 0, 0, 0, 2, 0)    # from 48 rows: 96 tiles, K in two halves
    assert gemm_plan(32, 12288, 4096, 6, raw_a=0)[0] == 2                  # under 48 rows
    assert gemm_plan(256, 2304, 768, 6, raw_a=0) == (2, 2, 1, 4, 1, 0)     # residue planes: 32-row MFMA tiles
    assert gemm_plan(512, 2304, 768, 6, raw_a=0) == (2, 2, 1, 4, 1, 0)     # 576 of them
    assert gemm_plan(256, 2304, 768, 6) == (2, 4, 1, 0, 1, 0)              # raw int8: the rows-per-CU rule
    assert gemm_plan(256, 2304, 768, 4, raw_a=0)[0] != 8                   # 36 tiles x 12 steps: too little work
    assert gemm_plan(4096, 2304, 768, 4, raw_a=0) == (8, 0, 0, 0, 1, 0)    # 576 tiles
    assert gemm_plan(512, 12288, 4096, 3, raw_a=0)[0] == 2                 # 3-channel capacity


def test_gemm_plan_residue_plane_few_rows():
    # residue-plane activations at decode sizes: the stream kernel (chunks of
    # at most 4 K steps) only while the MFMA kernel's 32 x 64 tiles number
    # under 128 and the rows are at most 32, else 32-row MFMA tiles
    assert gemm_plan(1, 12288, 4096, 6, raw_a=0) == (2, 2, 1, 4, 1, 0)    # 192 MFMA tiles
    assert gemm_plan(16, 12288, 4096, 6, raw_a=0) == (2, 2, 1, 4, 1, 0)
    assert gemm_plan(16, 4096, 4096, 6, raw_a=0) == (1, 1, 1, 4, 1, 0)    # 64 MFMA tiles: stream
    assert gemm_plan(32, 4096, 4096, 4, raw_a=0) == (1, 1, 1, 4, 1, 0)
    assert gemm_plan(1, 4096, 4096, 4, raw_a=0) == (1, 1, 1, 4, 1, 0)     # never 8-step chunks
    assert gemm_plan(64, 4096, 4096, 6, raw_a=0) == (2, 2, 1, 4, 1, 0)    # past 32 rows
    assert gemm_plan(64, 2304, 768, 6, raw_a=0) == (2, 2, 1, 4, 1, 0)
    assert gemm_plan(16, 2304, 768, 6, raw_a=0)[0] == 1                   # 36 MFMA tiles
    # raw int8 keeps its rule: 8-step chunks at K = 4096, the stream kernel to 64 rows
    assert gemm_plan(1, 4096, 4096, 4) == (4, 1, 1, 4, 1, 0)
    assert gemm_plan(64, 2304, 768, 4)[0] == 1


def test_gemm_plan_rejects_bad_shapes():
    # residue-plane activations (K not a multiple of 16): never the LDS kernel
    assert gemm_plan(2048, 12288, 4104, raw_a=0)[0] == 2
    assert gemm_plan(2048, 12288, 4104, 6, raw_a=0)[0] == 2
    for bad in ((0, 8, 8, 4), (8, 8, 8, 1), (8, 8, 8, 11)):
        with pytest.raises(ValueError):
            gemm_plan(*bad)


@pytest.mark.parametrize("mods", [DENSE4, (251, 241, 239, 233), (3, 5, 7, 11, 13, 17, 19, 23, 29, 31),
                                  (127, 125, 121, 113), (2, 3), (254, 253, 251)])
def test_native_moduli_constants(mods):
    """rnsmx_moduli_init's Garner constants reproduce the oracle's mixed-radix
    digits for random residues, and its Barrett magic / 2^31 offsets are the
    closed forms."""
    c = _native.make_moduli(mods)
    r_count = len(mods)
    assert c.channels == r_count
    assert [c.prefix[i] for i in range(r_count + 1)] == [prod(mods[:i]) for i in range(r_count + 1)]
    for i, m in enumerate(mods):
        assert c.magic[i] == (1 << 32) // m
        assert c.c31[i] == (1 << 31) % m
        # digit constants: 2^16 q and 2^8 q mod m (the first centered)
        assert (c.qk16[i] - (1 << 16) * c.qinv[i]) % m == 0 and 2 * abs(c.qk16[i]) <= m
        assert c.qk8[i] == ((1 << 8) * c.qinv[i]) % m
    rng = np.random.default_rng(0)
    res = np.stack([rng.integers(0, m, 300) for m in mods])
    # digits from the native constants: d_i = (r_i q_i + sum_j d_j u_ji) mod m_i
    digits = []
    for i, m in enumerate(mods):
        s = res[i] * c.qinv[i]
        for j in range(i):
            s = s + digits[j] * c.ucoef[j][i]
        digits.append(np.mod(s, m))
    x = sum(d.astype(object) * prod(mods[:i]) for i, d in enumerate(digits))
    np.testing.assert_array_equal(np.array(x, dtype=object) % prod(mods),
                                  ro.decode_garner(res, mods, signed=False).astype(object))


def test_native_lut_matches_oracle():
    c = _native.make_moduli(DENSE4)
    lut = np.empty((4, 4, 256), dtype=np.int16)
    _native.check(_native.lib().rnsmx_compact_lut(ctypes.byref(c), lut.ctypes.data))
    np.testing.assert_array_equal(lut, ro.compact_byte_mod_lut(DENSE4))


@pytest.mark.parametrize("bad,exc", [((), ValueError), ((256, 3), ValueError), ((1, 3), ValueError),
                                     ((255, 15), ValueError), ((251,) * 11, ValueError),
                                     ((251, 241, 239, 233, 229, 227, 223, 211, 199), OverflowError)])
def test_native_moduli_errors(bad, exc):
    with pytest.raises(exc):
        _native.make_moduli(bad)


def test_workspace_bytes_queries():
    lib = _native.lib()
    tickets = 4 * _native.SPLIT_TICKETS
    # counters + residue planes of A (int16 sources) + row norms
    assert lib.rnsmx_prepared_workspace_bytes(256, 768, 2304, 4, None) >= tickets + 4 * 256 * 768 + 8 * 256
    assert lib.rnsmx_prepared_workspace_bytes(1, 100, 37, 3, None) >= tickets + 3 * 128 + 8
    assert lib.rnsmx_fused_workspace_bytes(16, 768, 2304, 4) >= tickets + 4 * 2304 * 768
    assert lib.rnsmx_fused_workspace_bytes(16, 100, 37, 3) >= tickets + 3 * 48 * 128 + 3 * 16 * 128
    assert lib.rnsmx_prepared_workspace_bytes(-1, 5, 5, 4, None) == -1
    # a K split adds its exchange area: R residue bytes per output element
    # and split (a whole 16 x 16 block per wave)
    one = _native.Plan(1, 1, 1, 1, 1)
    four = _native.Plan(1, 1, 1, 1, 4)
    base = lib.rnsmx_prepared_workspace_bytes(1, 768, 768, 4, ctypes.byref(one))
    split = lib.rnsmx_prepared_workspace_bytes(1, 768, 768, 4, ctypes.byref(four))
    assert split - base >= 4 * 16 * 768 * 4


def test_c_abi_rejects_bad_arguments_without_gpu():
    """Argument validation happens before any HIP call, so it is testable on CPU."""
    lib = _native.lib()
    c = _native.make_moduli(DENSE4)
    rc = lib.rnsmx_matmul_centered_fused_out(None, None, 4, 64, 4, ctypes.byref(c), None, 3,
                                             None, 0, None, None)
    assert rc == _native.EINVAL and b"lut_channels" in lib.rnsmx_last_error()
    rc = lib.rnsmx_matmul_prepared_fused(None, _native.INT8, 4, 200_000, 4, None, ctypes.byref(c),
                                         None, 0, None, None, None, None, 0, None, None)
    assert rc == _native.ERANGE
    rc = lib.rnsmx_encode_centered(None, _native.INT64, 1, 4, 4, ctypes.byref(c), None, None,
                                   None, None)
    assert rc == _native.EINVAL
    # zero-size problems are accepted and launch nothing
    assert lib.rnsmx_matmul_prepared_fused(None, _native.INT8, 0, 64, 8, None, ctypes.byref(c),
                                           None, 0, None, None, None, None, 0, None, None) == _native.OK
    # a plan that cannot split is rejected before any launch
    bad = _native.Plan(1, 1, 1, 2, 2)
    x = ctypes.c_int64(0)
    rc = lib.rnsmx_matmul_prepared_fused(ctypes.addressof(x), _native.INT8, 4, 64, 8, ctypes.addressof(x),
                                         ctypes.byref(c), None, 0, None, None, ctypes.byref(bad),
                                         ctypes.addressof(x), 1 << 20, ctypes.addressof(x), None)
    assert rc == _native.EINVAL and b"cannot split" in lib.rnsmx_last_error()


def packed_plan(m, n, k, channels=6):
    out = _native.Plan()
    _native.check(_native.lib().rnsmx_packed_plan(m, n, k, channels, ctypes.byref(out)))
    return out.as_tuple()


# packed weights: the channel-row kernel for up to eight blocks of 16 / R
# tokens (kind 6, mb = blocks, a power of two), then the stream kernel where the
# residue-plane choice takes it (16- or 32-row tiles, K over as many waves
# as chunks allow, at most 4), else the MFMA kernel with 32- or 64-row
# tiles (fewest rows per CU, 64 on a tie), or from 129 rows the
# residue-plane LDS kernel (K a multiple of 256), split over K as for
# residue-plane weights; the others never split
PACKED_PLANS = [
    ((1, 12288, 4096, 6), (6, 1, 1, 4, 1, 0)),   # decode: channel rows, chunks of 8 steps, 4 waves
    ((1, 768, 768, 6), (6, 1, 1, 2, 1, 0)),
    ((2, 768, 768, 6), (6, 1, 1, 2, 1, 0)),      # 2 tokens x 6 channel rows in one block
    ((3, 768, 768, 6), (6, 2, 1, 3, 1, 0)),      # two blocks, chunks of 4 steps
    ((8, 768, 768, 4), (6, 2, 1, 3, 1, 0)),      # 4 tokens x 4 channel rows per block
    ((5, 768, 768, 6), (6, 4, 1, 4, 1, 0)),      # four blocks, chunks of 2 steps
    ((9, 768, 768, 4), (6, 4, 1, 4, 1, 0)),
    ((16, 12288, 4096, 6), (6, 8, 1, 4, 1, 0)),  # eight blocks, chunks of 2 steps
    ((17, 768, 768, 6), (1, 2, 1, 4, 1, 0)),     # past eight blocks: stream, 32-row tiles
    ((33, 768, 768, 4), (1, 2, 1, 4, 1, 0)),     # 4 channels, 12 MFMA tiles: stream
    ((1, 768, 50_000, 6), (1, 1, 1, 4, 1, 0)),   # K past the channel-row sums' int32 range
    ((96, 2304, 768, 6), (2, 2, 1, 0, 1, 0)),    # past 48 rows: MFMA tiles
    ((100, 2304, 768, 6), (2, 2, 1, 0, 1, 0)),   # MFMA: 144 tiles of 32 rows beat 72 of 64
    ((256, 2304, 768, 6), (2, 2, 1, 0, 1, 0)),   # a tie in rows per CU (288 tiles of 32 rows, 144 of 64): 32
    ((1024, 4096, 1100, 6), (2, 4, 1, 0, 1, 0)),  # 256 rows per CU either way: 64 (K not 256-aligned)
    ((1024, 4096, 1024, 6), (8, 0, 0, 0, 1, 0)),  # residue-plane LDS kernel: 256 tiles of 128 x 128
    ((512, 12288, 4096, 6), (8, 0, 0, 0, 2, 1)),  # 384 tiles: the last 128 split K in two
    ((1024, 4096, 1000, 4), (8, 0, 0, 0, 1, 0)),  # K = 1000 padded to 1024
    ((1024, 2048, 1024, 6), (8, 0, 0, 0, 1, 0)),  # 128 tiles of 128 x 128: the residue-plane LDS kernel
    ((512, 2048, 1024, 6), (2, 2, 1, 0, 1, 0)),   # 64 of them, 16 K steps: MFMA kernel
    ((512, 4096, 4096, 6), (8, 0, 0, 0, 2, 0)),   # 128 tiles, 64 K steps: every tile in two
]


@pytest.mark.parametrize("shape,plan", PACKED_PLANS)
def test_packed_plan_rules(shape, plan):
    assert packed_plan(*shape) == plan


def test_packed_queries_and_rejects_without_gpu():
    lib = _native.lib()
    tickets = 4 * _native.SPLIT_TICKETS
    # counters + the larger of (2R activation planes + int32 row terms [R][round_up(M, 64) + 64])
    # and (up to 32 tokens) eight blocks of channel-row fragments [2][kp/64][1 KB] + row norms
    assert lib.rnsmx_packed_workspace_bytes(1, 768, 768, 6, None) == tickets + max(
        2 * 6 * 768 + 4 * 6 * 128, 8 * 2 * 768 * 16) + 256
    assert lib.rnsmx_packed_workspace_bytes(100, 100, 37, 5, None) == (
        tickets + (2 * 5 * 100 * 128 + 4 * 5 * 192 + 255) // 256 * 256 + (8 * 100 + 255) // 256 * 256)
    assert lib.rnsmx_packed_workspace_bytes(1, 768, 768, 7, None) == -1
    out = _native.Plan()
    assert lib.rnsmx_packed_plan(1, 768, 768, 7, ctypes.byref(out)) == _native.EINVAL
    x = ctypes.c_int64(0)
    assert lib.rnsmx_prepare_weight_packed(ctypes.addressof(x), _native.INT32, 4, 64, ctypes.addressof(x),
                                           None, None) == _native.EINVAL
    assert b"int8 or int16" in lib.rnsmx_last_error()
    c7 = _native.make_moduli((255, 253, 251, 247, 241, 239, 233))
    rc = lib.rnsmx_matmul_packed_fused(None, _native.INT16, 4, 64, 4, None, ctypes.byref(c7),
                                       None, 0, None, None, None, None, 0, None, None)
    assert rc == _native.EINVAL and b"at most 6" in lib.rnsmx_last_error()
    c6 = _native.make_moduli((255, 253, 251, 247, 241, 239))
    # 2 * K * 128 * 127 + 255 past 2^31 - 1 from K = 66,053
    rc = lib.rnsmx_matmul_packed_fused(None, _native.INT16, 4, 66_053, 4, None, ctypes.byref(c6),
                                       None, 0, None, None, None, None, 0, None, None)
    assert rc == _native.ERANGE
    rows_plan = _native.Plan(6, 1, 1, 2, 1)  # one block holds 2 tokens of 6 channels, not 4
    rc = lib.rnsmx_matmul_packed_fused(ctypes.addressof(x), _native.INT16, 4, 64, 8, ctypes.addressof(x),
                                       ctypes.byref(c6), None, 0, None, None, ctypes.byref(rows_plan),
                                       ctypes.addressof(x), 1 << 20, ctypes.addressof(x), None)
    assert rc == _native.EINVAL and b"more tokens" in lib.rnsmx_last_error()
    for bad in (_native.Plan(2, 3, 1, 0, 1), _native.Plan(1, 1, 1, 1, 2), _native.Plan(3, 0, 0, 0, 1),
                _native.Plan(6, 3, 1, 1, 1), _native.Plan(6, 16, 1, 1, 1), _native.Plan(6, 1, 1, 5, 1)):
        rc = lib.rnsmx_matmul_packed_fused(ctypes.addressof(x), _native.INT16, 4, 64, 8, ctypes.addressof(x),
                                           ctypes.byref(c6), None, 0, None, None, ctypes.byref(bad),
                                           ctypes.addressof(x), 1 << 20, ctypes.addressof(x), None)
        assert rc == _native.EINVAL and b"packed weights run" in lib.rnsmx_last_error()


# --------------------------------------------------------------------------
# host logic: moduli.py against the oracle
# --------------------------------------------------------------------------
@pytest.mark.parametrize("k,a,b,strategy", [(768, 127, 127, "dense_coprime"), (64, 2047, 2047, "dense_coprime"),
                                            (768, 2047, 2047, "large_primes"), (501, 127, 127, "dense_coprime"),
                                            (4096, 32767, 32767, "dense_coprime"), (64, 127, 127, "small_primes")])
def test_choose_moduli_matches_oracle(k, a, b, strategy):
    assert host_moduli.choose_moduli_for_dot(k, a, b, strategy=strategy) == \
        ro.choose_moduli_for_dot(k, a, b, strategy=strategy)


def test_prefix_and_capacity_match_oracle():
    for bound in (0, 5_000_000, 8_096_632, 8_096_633, 1_999_868_227):
        assert host_moduli.minimal_prefix_channels(DENSE4, bound, min_channels=2) == \
            ro.minimal_prefix_channels(DENSE4, bound, min_channels=2)
    with pytest.raises(OverflowError):
        host_moduli.minimal_prefix_channels(DENSE4, 1_999_868_228)
    assert host_moduli.signed_capacity(DENSE4) == ro.signed_capacity(DENSE4)
    with pytest.raises(ValueError):
        host_moduli.validate_moduli((255, 253, 51))


def test_check_workspace_rejects_mismatch():
    ws = RNSWorkspace(accumulators=torch.empty(0, dtype=torch.uint8),
                      output=torch.empty((4, 8), dtype=torch.int64), channels=4, m=4, n=8)
    HipRNSBackend._check_workspace(ws, channels=4, m=4, n=8, device=torch.device("cpu"))
    with pytest.raises(ValueError):
        HipRNSBackend._check_workspace(ws, channels=3, m=4, n=8, device=torch.device("cpu"))


def test_backend_requires_gpu():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(RuntimeError):
        HipRNSBackend()


def test_rns_linear_rns_mode_errors_on_cpu():
    layer = RNSLinear(16, 8, mode="rns").eval()
    with pytest.raises(RuntimeError):
        layer(torch.randn(2, 16))            # no backend
    layer.backend = object()
    with pytest.raises(RuntimeError):
        layer(torch.randn(2, 16))            # CPU weights
    layer.train()
    with pytest.raises(RuntimeError):
        layer(torch.randn(2, 16))            # training mode
    with pytest.raises(ValueError):
        RNSLinear(16, 8, quant_bits=10)
    with pytest.raises(ValueError):
        RNSLinear(16, 8, lut_channels=3)


def test_rns_linear_default_moduli():
    assert RNSLinear(768, 768).moduli == DENSE4
    assert RNSLinear(4096, 64).moduli == DENSE4
    assert RNSLinear(768, 8, quant_bits=12).moduli == ro.choose_moduli_for_dot(
        768, 2047, 2047, strategy="dense_coprime")


# --------------------------------------------------------------------------
# torch-mode QKV fusion (mirrors the reference tests/test_qkv_fusion.py)
# --------------------------------------------------------------------------
def make_linears():
    torch.manual_seed(123)
    return tuple(nn.Linear(16, 16, bias=True).eval() for _ in range(3))


def test_torch_qkv_fusion_matches_three_linears():
    q, k, v = make_linears()
    fused = RNSQKVProjection.from_linears(q, k, v, mode="torch").eval()
    x = torch.randn(2, 5, 16)
    for left, right in zip(fused(x), (q(x), k(x), v(x))):
        torch.testing.assert_close(left, right, rtol=1e-6, atol=2e-7)


def test_cached_qkv_computes_once_and_recomputes_next_call():
    q, k, v = make_linears()
    projection = RNSQKVProjection.from_linears(q, k, v, mode="torch").eval()
    coord = CachedRNSQKV(projection).eval()
    qp, kp, vp = coord.slices()
    x = torch.randn(2, 5, 16)
    out = (qp(x), kp(x), vp(x))
    assert projection.compute_count == 1 and coord.cache_misses == 1 and coord.cache_hits == 2
    for left, right in zip(out, (q(x), k(x), v(x))):
        torch.testing.assert_close(left, right, rtol=1e-6, atol=2e-7)
    qp(x)
    qp(x)  # repeated index: new logical call
    assert projection.compute_count == 3


def test_qkv_proxy_detects_destroyed_coordinator():
    q, k, v = make_linears()
    coord = CachedRNSQKV(RNSQKVProjection.from_linears(q, k, v, mode="torch"))
    proxy = coord.slices()[0]
    del coord
    import gc
    gc.collect()
    with pytest.raises(RuntimeError):
        proxy(torch.randn(1, 16))


def test_from_linears_validation():
    q, k, v = make_linears()
    with pytest.raises(ValueError):
        RNSQKVProjection.from_linears(q, k, nn.Linear(8, 16), mode="torch")
    with pytest.raises(TypeError):
        RNSQKVProjection.from_linears(q, k, nn.Identity(), mode="torch")


def test_installed_fusion_owns_parameters_once():
    from rns_llm_amd.layers import install_opt_qkv_fusion

    class Attention(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj, self.k_proj, self.v_proj = make_linears()
            self.out_proj = nn.Linear(16, 16)

    attention = Attention()
    q_w = attention.q_proj.weight.detach().clone()
    coord = install_opt_qkv_fusion(attention, backend=None)
    keys = set(attention.state_dict())
    assert {"rns_qkv.projection.combined.weight", "rns_qkv.projection.combined.bias"} <= keys
    assert not any(k.startswith(("q_proj", "k_proj", "v_proj")) for k in keys)
    assert attention.rns_qkv is coord and [p.index for p in (attention.q_proj, attention.k_proj,
                                                             attention.v_proj)] == [0, 1, 2]
    # q, k, v stacked in that order along the output features
    torch.testing.assert_close(coord.projection.combined.weight[:16], q_w, rtol=0, atol=0)
    with pytest.raises(TypeError):
        install_opt_qkv_fusion(attention, backend=None)  # q_proj is no longer nn.Linear


def test_qkv_cache_recomputes_for_a_new_hidden_state():
    q, k, v = make_linears()
    projection = RNSQKVProjection.from_linears(q, k, v, mode="torch").eval()
    coord = CachedRNSQKV(projection).eval()
    qp, kp, vp = coord.slices()
    x, y = torch.randn(2, 16), torch.randn(2, 16)
    qp(x)
    kp(y)  # another hidden state before the call finished: recompute
    assert projection.compute_count == 2 and coord.cache_misses == 2 and coord.cache_hits == 0
    vp(y)
    qp(y)  # k, v and q of y served from one product
    assert projection.compute_count == 2 and coord.cache_hits == 2
    with pytest.raises(ValueError):
        coord.forward_slice(x, 3)


def test_replace_opt_attention_blocks_structure():
    transformers = pytest.importorskip("transformers")
    from rns_llm_amd.layers import replace_opt_attention_blocks

    config = transformers.OPTConfig(hidden_size=16, num_attention_heads=2, ffn_dim=32,
                                    num_hidden_layers=3, vocab_size=64, max_position_embeddings=32,
                                    word_embed_proj_dim=16)
    model = transformers.OPTForCausalLM(config).eval()
    layers = model.model.decoder.layers
    before = layers[0].self_attn.out_proj.weight.detach().clone()
    replaced, coordinators = replace_opt_attention_blocks(model, backend=None, blocks=2)
    assert replaced == [f"model.decoder.layers.{i}.self_attn.{part}" for i in (0, 1)
                        for part in ("qkv_fused", "out_proj")]
    assert len(coordinators) == 2
    assert isinstance(layers[0].self_attn.out_proj, RNSLinear)
    torch.testing.assert_close(layers[0].self_attn.out_proj.weight, before, rtol=0, atol=0)
    assert isinstance(layers[2].self_attn.q_proj, nn.Linear)  # only the first two blocks
    with pytest.raises(ValueError):
        replace_opt_attention_blocks(model, backend=None, blocks=-1)
