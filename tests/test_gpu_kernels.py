"""Every GEMM kernel instance, forced through rnsmx_set_gemm_override, on
ragged shapes: raw int8 activations (one A matrix shared by all channels)
and residue-plane activations (int16 sources, K not a multiple of 16), full
and adaptive channel prefixes, integer and float epilogues.  Each output must
equal the exact int64 product (or the CPU oracle) bit for bit."""
import numpy as np
import pytest
import torch

from oracle import rns_oracle as ro
from rns_llm_amd import _native

pytestmark = pytest.mark.gpu

DEV = "cuda"
DENSE4 = (255, 253, 251, 247)
SETS = {3: (254, 253, 251), 4: DENSE4, 6: (255, 253, 251, 247, 241, 239),
        10: (3, 5, 7, 11, 13, 17, 19, 23, 29, 31)}
RCAP = {3: 3, 4: 4, 6: 6, 10: 10}
STREAM_TILES = [(1, 1), (2, 1), (4, 1), (1, 2)]
# MFMA tiles (mb, nb) -> ring depths built for them
_MFMA4 = {(2, 1): (3, 4), (3, 1): (3, 4), (4, 1): (3, 4), (2, 2): (3, 4), (4, 2): (3, 4), (8, 2): (3, 4)}
MFMA_TILES = {3: _MFMA4, 4: _MFMA4, 6: {(2, 1): (3, 4), (4, 1): (3, 4), (4, 2): (3,)},
              10: {(2, 1): (3,), (4, 1): (3,), (2, 2): (2,)}}


def stream_cases():
    out = []
    for r in (3, 4, 6, 10):
        for mb, nb in STREAM_TILES:
            if r >= 6 and (nb > 1 or mb > 2):
                continue
            for ks in (1, 2, 4):
                if ks > 1 and r * 256 * mb * nb * 4 > 65536:
                    continue
                out.append((r, mb, nb, ks))
    return out


def mfma_cases():
    return [(r, mb, nb, p) for r, tiles in MFMA_TILES.items() for (mb, nb), depths in tiles.items()
            for p in depths]


@pytest.fixture
def override(backend):
    lib = backend._lib

    def set_(kind, mb=0, nb=0, ks=0):
        _native.check(lib.rnsmx_set_gemm_override(kind, mb, nb, ks))

    yield set_
    _native.check(lib.rnsmx_set_gemm_override(0, 0, 0, 0))


def amax_for(mods, k):
    # largest int8 magnitude whose worst-case product the set still holds
    half = (np.prod(np.array(mods, dtype=object)) - 1) // 2
    return int(min(127, max(1, int((half // k) ** 0.5))))


def run_case(backend, mods, m, k, n, dtype=torch.int8, seed=0, adaptive=False, out_dtype=None):
    gen = torch.Generator().manual_seed(seed)
    amax = amax_for(mods, k)
    if adaptive:
        amax = 8
    a = torch.randint(-amax, amax + 1, (m, k), generator=gen).to(dtype)
    b = torch.randint(-amax, amax + 1, (k, n), generator=gen).to(torch.int8)
    want = ro.exact_matmul(a.numpy(), b.numpy())
    if adaptive:
        prepared = backend.prepare_weight_adaptive(b.to(DEV), mods, min_channels=2)
        out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), prepared, lut_channels=1,
                                                          return_metadata=True)
        assert meta["channels"] < len(mods)
        np.testing.assert_array_equal(out.cpu().numpy(), want)
        return
    prepared = backend.prepare_weight(b.to(DEV), mods)
    if out_dtype is None:
        out = backend.matmul_prepared_fused(a.to(DEV), prepared, lut_channels=min(2, len(mods)))
        np.testing.assert_array_equal(out.cpu().numpy(), want)
        return
    a_scale = torch.tensor([0.0123], dtype=torch.float32)
    w_scale = torch.rand((n,), generator=gen, dtype=torch.float32) * 0.01
    bias = torch.randn((n,), generator=gen, dtype=torch.float32)
    out = torch.empty((m, n), dtype=out_dtype, device=DEV)
    backend.matmul_prepared_fused(a.to(DEV), prepared, out=out, a_scale=a_scale.to(DEV),
                                  w_scale=w_scale.to(DEV), bias=bias.to(DEV))
    # the op order of RNSLinear's output chain, on the CPU (IEEE f32, no FMA)
    ref = ((torch.from_numpy(want).float() * a_scale.view(1, 1)) * w_scale.unsqueeze(0) + bias)
    bits = torch.int32 if out_dtype == torch.float32 else torch.int16
    assert torch.equal(out.cpu().view(bits), ref.to(out_dtype).view(bits))


@pytest.mark.parametrize("r,mb,nb,ks", stream_cases())
def test_stream_kernel_instances(backend, override, r, mb, nb, ks):
    override(1, mb, nb, ks)
    mods = SETS[r]
    # raw int8 A (K % 16 == 0), K tail inside the last 64-byte step
    run_case(backend, mods, 16 * mb * 2 + 3, 208, 16 * nb * 3 + 5, seed=r * 1000 + mb * 10 + nb)
    # residue-plane A: K % 16 != 0 and int16 sources
    run_case(backend, mods, 16 * mb + 1, 100, 16 * nb + 7, seed=ks)
    run_case(backend, mods, 7, 150, 37, dtype=torch.int16, seed=ks + 1)


@pytest.mark.parametrize("r,ks", [(r, ks) for r in (3, 4) for ks in (1, 2, 4)])
def test_wide_stream_kernel_instances(backend, override, r, ks):
    # 8-step chunks: several chunks per wave, the last past K
    override(4, 1, 1, ks)
    mods = SETS[r]
    run_case(backend, mods, 19, 64 * (8 * ks * 2 + 3) + 16, 16 * 3 + 5, seed=r * 10 + ks)
    run_case(backend, mods, 5, 208, 21, seed=ks)
    run_case(backend, mods, 7, 150, 37, dtype=torch.int16, seed=ks + 1)


@pytest.mark.parametrize("r,mb,p", [(r, mb, p) for r in (3, 4) for mb, p in ((2, 4), (3, 4), (4, 3), (4, 4))])
def test_three_wave_mfma_kernel_instances(backend, override, r, mb, p):
    # 48-column tiles: ragged N around multiples of 48 and 16, several trips
    # round the ring, the last partly past K
    override(5, mb, 1, p)
    mods = SETS[r]
    run_case(backend, mods, 16 * mb * 2 + 9, 336, 48 * 2 + 11, seed=r * 100 + mb)
    run_case(backend, mods, 16 * mb + 5, 64 * (2 * p + 1) + 16, 48 + 3, seed=p)
    run_case(backend, mods, 16 * mb + 3, 768, 2304, seed=r)
    run_case(backend, mods, 3, 320, 90, seed=7, adaptive=True)


@pytest.mark.parametrize("r,mb,nb,p", mfma_cases())
def test_mfma_kernel_instances(backend, override, r, mb, nb, p):
    override(2, mb, nb, p)
    mods = SETS[r]
    run_case(backend, mods, 16 * mb * 2 + 9, 336, 64 * nb * 2 + 11, seed=r * 100 + mb)
    # several trips round the load ring, the last one partly past K
    run_case(backend, mods, 16 * mb + 5, 64 * (2 * p + 1) + 16, 64 * nb + 3, seed=p)
    run_case(backend, mods, 16 * mb + 3, 100, 64 * nb + 1, seed=r)
    run_case(backend, mods, 40, 150, 70, dtype=torch.int16, seed=r + 1)


@pytest.mark.parametrize("m,k,n", [(256 * 2 + 37, 256, 64 * 3 + 5), (300, 512, 100), (17, 1024, 64),
                                   (256, 768, 2304)])
def test_lds_kernel(backend, override, m, k, n):
    # 256 x 64 tiles, four stages of direct-to-LDS loads: ragged M and N,
    # one and several trips round the stages
    override(3)
    run_case(backend, DENSE4, m, k, n, seed=m + k)


def test_lds_kernel_rejects_unfit_shapes(backend, override):
    override(3)
    prepared = backend.prepare_weight(torch.ones((320, 16), dtype=torch.int8, device=DEV), DENSE4)
    with pytest.raises(ValueError, match="no GEMM kernel"):  # K not a multiple of 256
        backend.matmul_prepared_fused(torch.ones((4, 320), dtype=torch.int8, device=DEV), prepared)
    prepared = backend.prepare_weight(torch.ones((256, 16), dtype=torch.int8, device=DEV), SETS[3])
    with pytest.raises(ValueError, match="no GEMM kernel"):  # 3-channel capacity
        backend.matmul_prepared_fused(torch.ones((4, 256), dtype=torch.int8, device=DEV), prepared)


@pytest.mark.parametrize("kind,mb,nb,ks,k", [(1, 1, 1, 4, 320), (1, 1, 2, 2, 320), (1, 2, 1, 1, 320),
                                             (2, 8, 2, 0, 320), (2, 2, 1, 0, 320), (3, 0, 0, 0, 512)])
def test_kernel_adaptive_prefix(backend, override, kind, mb, nb, ks, k):
    override(kind, mb, nb, ks)
    run_case(backend, DENSE4, 50, k, 90, seed=5, adaptive=True)
    # up to 4 raw rows: the row norms are summed inside the GEMM
    run_case(backend, DENSE4, 3, k, 90, seed=6, adaptive=True)


@pytest.mark.parametrize("kind,mb,nb,ks", [(1, 1, 2, 2), (1, 4, 1, 4), (1, 2, 1, 1), (2, 8, 2, 0), (2, 2, 1, 0),
                                           (3, 0, 0, 0)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_kernel_float_epilogue(backend, override, kind, mb, nb, ks, out_dtype):
    override(kind, mb, nb, ks)
    run_case(backend, DENSE4, 45, 256, 77, seed=9, out_dtype=out_dtype)


def test_prepared_residues_view_matches_encode(backend):
    # the fragment-major store unpacks to the reference [R, K, N] residues
    gen = torch.Generator().manual_seed(31)
    for k, n in ((100, 37), (768, 48), (64, 16)):
        b = torch.randint(-127, 128, (k, n), generator=gen).to(torch.int8)
        prepared = backend.prepare_weight(b.to(DEV), DENSE4)
        assert prepared.packed.shape == (4, (n + 15) // 16, (k + 63) // 64, 1024)
        np.testing.assert_array_equal(prepared.residues.cpu().numpy(),
                                      ro.encode_centered(b.numpy(), DENSE4))


@pytest.mark.parametrize("kind,mb,nb,ks", [(2, 3, 3, 0), (2, 8, 2, 8)])
def test_override_rejects_unbuilt_tile(backend, override, kind, mb, nb, ks):
    override(kind, mb, nb, ks)
    prepared = backend.prepare_weight(torch.ones((64, 16), dtype=torch.int8, device=DEV), DENSE4)
    with pytest.raises(ValueError, match="no GEMM kernel"):
        backend.matmul_prepared_fused(torch.ones((4, 64), dtype=torch.int8, device=DEV), prepared)
