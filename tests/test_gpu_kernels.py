"""Every GEMM kernel instance, forced through a per-call plan, on ragged
shapes: raw int8 activations (one A matrix shared by all channels) and
residue-plane activations (int16 sources, K not a multiple of 16), full and
adaptive channel prefixes, integer and float epilogues, with and without K
split over workgroups.  Each output must equal the exact int64 product (or
the CPU oracle) bit for bit."""
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


def amax_for(mods, k):
    # largest int8 magnitude whose worst-case product the set still holds
    half = (np.prod(np.array(mods, dtype=object)) - 1) // 2
    return int(min(127, max(1, int((half // k) ** 0.5))))


def run_case(backend, mods, m, k, n, dtype=torch.int8, seed=0, adaptive=False, out_dtype=None,
             plan=None, repeat=1):
    """One product through the plan; with repeat > 1 the same call runs
    again on one workspace (the K-split counters must return to zero)."""
    gen = torch.Generator().manual_seed(seed)
    amax = amax_for(mods, k)
    if adaptive:
        amax = 8
    a = torch.randint(-amax, amax + 1, (m, k), generator=gen).to(dtype)
    b = torch.randint(-amax, amax + 1, (k, n), generator=gen).to(torch.int8)
    want = ro.exact_matmul(a.numpy(), b.numpy())
    if adaptive:
        prepared = backend.prepare_weight_adaptive(b.to(DEV), mods, min_channels=2)
        ws = {len(mods): backend.create_workspace(device=torch.device(DEV), channels=len(mods),
                                                  m=m, n=n, k=k)}
        for _ in range(repeat):
            out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), prepared, lut_channels=1,
                                                              workspace_by_channels=ws,
                                                              return_metadata=True, plan=plan)
            assert meta["channels"] < len(mods)
            np.testing.assert_array_equal(out.cpu().numpy(), want)
        return
    prepared = backend.prepare_weight(b.to(DEV), mods)
    if out_dtype is None:
        ws = backend.create_workspace(device=torch.device(DEV), channels=len(mods), m=m, n=n, k=k)
        for _ in range(repeat):
            out = backend.matmul_prepared_fused(a.to(DEV), prepared, lut_channels=min(2, len(mods)),
                                                workspace=ws, plan=plan)
            np.testing.assert_array_equal(out.cpu().numpy(), want)
        return
    a_scale = torch.tensor([0.0123], dtype=torch.float32)
    w_scale = torch.rand((n,), generator=gen, dtype=torch.float32) * 0.01
    bias = torch.randn((n,), generator=gen, dtype=torch.float32)
    out = torch.empty((m, n), dtype=out_dtype, device=DEV)
    backend.matmul_prepared_fused(a.to(DEV), prepared, out=out, a_scale=a_scale.to(DEV),
                                  w_scale=w_scale.to(DEV), bias=bias.to(DEV), plan=plan)
    # the op order of RNSLinear's output chain, on the CPU (IEEE f32, no FMA)
    ref = ((torch.from_numpy(want).float() * a_scale.view(1, 1)) * w_scale.unsqueeze(0) + bias)
    bits = torch.int32 if out_dtype == torch.float32 else torch.int16
    assert torch.equal(out.cpu().view(bits), ref.to(out_dtype).view(bits))


@pytest.mark.parametrize("r,mb,nb,ks", stream_cases())
def test_stream_kernel_instances(backend, r, mb, nb, ks):
    plan = (1, mb, nb, ks)
    mods = SETS[r]
    # raw int8 A (K % 16 == 0), K tail inside the last 64-byte step
    run_case(backend, mods, 16 * mb * 2 + 3, 208, 16 * nb * 3 + 5, seed=r * 1000 + mb * 10 + nb, plan=plan)
    # residue-plane A: K % 16 != 0 and int16 sources
    run_case(backend, mods, 16 * mb + 1, 100, 16 * nb + 7, seed=ks, plan=plan)
    run_case(backend, mods, 7, 150, 37, dtype=torch.int16, seed=ks + 1, plan=plan)


@pytest.mark.parametrize("r,ks", [(r, ks) for r in (3, 4) for ks in (1, 2, 4)])
def test_wide_stream_kernel_instances(backend, r, ks):
    # 8-step chunks: several chunks per wave, the last past K
    plan = (4, 1, 1, ks)
    mods = SETS[r]
    run_case(backend, mods, 19, 64 * (8 * ks * 2 + 3) + 16, 16 * 3 + 5, seed=r * 10 + ks, plan=plan)
    run_case(backend, mods, 5, 208, 21, seed=ks, plan=plan)
    run_case(backend, mods, 7, 150, 37, dtype=torch.int16, seed=ks + 1, plan=plan)


@pytest.mark.parametrize("r,mb,p", [(r, mb, p) for r in (3, 4) for mb, p in ((2, 4), (3, 4), (4, 3), (4, 4))])
def test_three_wave_mfma_kernel_instances(backend, r, mb, p):
    # 48-column tiles: ragged N around multiples of 48 and 16, several trips
    # round the ring, the last partly past K
    plan = (5, mb, 1, p)
    mods = SETS[r]
    run_case(backend, mods, 16 * mb * 2 + 9, 336, 48 * 2 + 11, seed=r * 100 + mb, plan=plan)
    run_case(backend, mods, 16 * mb + 5, 64 * (2 * p + 1) + 16, 48 + 3, seed=p, plan=plan)
    run_case(backend, mods, 16 * mb + 3, 768, 2304, seed=r, plan=plan)
    run_case(backend, mods, 3, 320, 90, seed=7, adaptive=True, plan=plan)


@pytest.mark.parametrize("r,mb,nb,p", mfma_cases())
def test_mfma_kernel_instances(backend, r, mb, nb, p):
    plan = (2, mb, nb, p)
    mods = SETS[r]
    run_case(backend, mods, 16 * mb * 2 + 9, 336, 64 * nb * 2 + 11, seed=r * 100 + mb, plan=plan)
    # several trips round the load ring, the last one partly past K
    run_case(backend, mods, 16 * mb + 5, 64 * (2 * p + 1) + 16, 64 * nb + 3, seed=p, plan=plan)
    run_case(backend, mods, 16 * mb + 3, 100, 64 * nb + 1, seed=r, plan=plan)
    run_case(backend, mods, 40, 150, 70, dtype=torch.int16, seed=r + 1, plan=plan)


LDS_KINDS = [3, 7]  # 256 x 64 and 256 x 96 tiles


@pytest.mark.parametrize("kind", LDS_KINDS)
@pytest.mark.parametrize("m,k,n", [(256 * 2 + 37, 256, 64 * 3 + 5), (300, 512, 100), (17, 1024, 64),
                                   (256, 768, 2304), (256 * 3, 1024, 96 * 5 - 40), (200, 256, 96 + 1)])
def test_lds_kernel(backend, kind, m, k, n):
    # 256-row tiles, four stages of direct-to-LDS loads: ragged M and N,
    # one and several trips round the stages
    run_case(backend, DENSE4, m, k, n, seed=m + k, plan=(kind, 0, 0, 0))


@pytest.mark.parametrize("kind", LDS_KINDS)
def test_lds_kernel_rejects_unfit_shapes(backend, kind):
    lds = (kind, 0, 0, 0)
    prepared = backend.prepare_weight(torch.ones((320, 16), dtype=torch.int8, device=DEV), DENSE4)
    with pytest.raises(ValueError, match="no GEMM kernel"):  # K not a multiple of 256
        backend.matmul_prepared_fused(torch.ones((4, 320), dtype=torch.int8, device=DEV), prepared, plan=lds)
    prepared = backend.prepare_weight(torch.ones((256, 16), dtype=torch.int8, device=DEV), SETS[3])
    with pytest.raises(ValueError, match="no GEMM kernel"):  # 3-channel capacity
        backend.matmul_prepared_fused(torch.ones((4, 256), dtype=torch.int8, device=DEV), prepared, plan=lds)


# residue-plane LDS kernel (kind 8): 128 x 128 tiles, one staging unit per
# channel and pair of K steps, 4 or 6 channels
PLANE_SHAPES = [(128 * 2 + 37, 256, 128 * 3 + 5), (300, 512, 100), (17, 1024, 64), (128 * 3, 768, 128 * 2),
                (129, 256, 129), (640, 1024, 300)]


@pytest.mark.parametrize("r", [4, 6])
@pytest.mark.parametrize("m,k,n", PLANE_SHAPES)
def test_lds_planes_kernel(backend, r, m, k, n):
    # ragged M and N, one and several trips round the four slots (a trip is
    # lcm(R, 4) units: one pair of K steps at R = 4, two at R = 6)
    run_case(backend, SETS[r], m, k, n, dtype=torch.int16, seed=m + k + r, plan=(8, 0, 0, 0), repeat=2)


def test_lds_planes_kernel_full_int16(backend):
    # int16 x int16 over the whole range on the 6-channel set (the wide
    # path's operands): exact int64 product
    gen = torch.Generator().manual_seed(816)
    m, k, n = 300, 1024, 260
    a = torch.randint(-32767, 32768, (m, k), generator=gen, dtype=torch.int32).to(torch.int16)
    b = torch.randint(-32767, 32768, (k, n), generator=gen, dtype=torch.int32).to(torch.int16)
    prepared = backend.prepare_weight(b.to(DEV), SETS[6])
    out = backend.matmul_prepared_fused(a.to(DEV), prepared, plan=(8, 0, 0, 0))
    np.testing.assert_array_equal(out.cpu().numpy(), ro.exact_matmul(a.numpy(), b.numpy()))


@pytest.mark.parametrize("r", [4, 6])
def test_lds_planes_kernel_adaptive_prefix(backend, r):
    # the device picks fewer channels: the loads of the rest re-read channel
    # 0's planes and the epilogue reconstructs from the prefix
    run_case(backend, SETS[r], 300, 512, 200, dtype=torch.int16, seed=r, adaptive=True, plan=(8, 0, 0, 0),
             repeat=2)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_lds_planes_kernel_float_epilogue(backend, out_dtype):
    run_case(backend, SETS[6], 300, 512, 130, dtype=torch.int16, seed=9, out_dtype=out_dtype, plan=(8, 0, 0, 0))


@pytest.mark.parametrize("r", [4, 6])
@pytest.mark.parametrize("m,k,n,splits", [(300, 1024, 100, 2), (129, 2048, 260, 4)])
def test_split_k_lds_planes_kernel(backend, r, m, k, n, splits):
    # every tile's K range over `splits` workgroups: residue bytes of up to 6
    # channels exchanged in two words per element, twice on one workspace
    run_case(backend, SETS[r], m, k, n, dtype=torch.int16, seed=m + splits + r, plan=(8, 0, 0, 0, splits),
             repeat=2)


@pytest.mark.parametrize("r", [4, 6])
def test_tail_split_lds_planes_kernel(backend, r):
    # 3 x 86 = 258 tiles: 256 run whole, the last 2 split K in two halves
    gen = torch.Generator().manual_seed(258 + r)
    m, k, n = 300, 512, 128 * 86 - 5
    a = torch.randint(-2000, 2001, (m, k), generator=gen, dtype=torch.int32).to(torch.int16)
    b = torch.randint(-127, 128, (k, n), generator=gen, dtype=torch.int32).to(torch.int8)
    prepared = backend.prepare_weight(b.to(DEV), SETS[r])
    ws = backend.create_workspace(device=torch.device(DEV), channels=r, m=m, n=n, k=k)
    whole = backend.matmul_prepared_fused(a.to(DEV), prepared, workspace=ws, plan=(8, 0, 0, 0)).cpu()
    for _ in range(2):
        split = backend.matmul_prepared_fused(a.to(DEV), prepared, workspace=ws, plan=(8, 0, 0, 0, 2, 1)).cpu()
        assert torch.equal(split, whole)
    rows = [0, 127, 128, 299]
    np.testing.assert_array_equal(whole[rows].numpy(), ro.exact_matmul(a[rows].numpy(), b.numpy()))
    cols = slice(128 * 85 - 7, n)  # the split tiles' columns
    np.testing.assert_array_equal(whole[:, cols].numpy(), ro.exact_matmul(a.numpy(), b[:, cols].numpy()))


def test_lds_planes_kernel_rejects_unfit_shapes(backend):
    planes = (8, 0, 0, 0)
    prepared = backend.prepare_weight(torch.ones((256, 16), dtype=torch.int8, device=DEV), SETS[6])
    with pytest.raises(ValueError, match="no GEMM kernel"):  # raw int8 activations
        backend.matmul_prepared_fused(torch.ones((4, 256), dtype=torch.int8, device=DEV), prepared, plan=planes)
    prepared = backend.prepare_weight(torch.ones((320, 16), dtype=torch.int8, device=DEV), SETS[6])
    with pytest.raises(ValueError, match="no GEMM kernel"):  # K not a multiple of 256
        backend.matmul_prepared_fused(torch.ones((4, 320), dtype=torch.int16, device=DEV), prepared, plan=planes)
    prepared = backend.prepare_weight(torch.ones((256, 16), dtype=torch.int8, device=DEV), SETS[3])
    with pytest.raises(ValueError, match="no GEMM kernel"):  # 3-channel capacity
        backend.matmul_prepared_fused(torch.ones((4, 256), dtype=torch.int16, device=DEV), prepared, plan=planes)


@pytest.mark.parametrize("kind,mb,nb,ks,k", [(1, 1, 1, 4, 320), (1, 1, 2, 2, 320), (1, 2, 1, 1, 320),
                                             (2, 8, 2, 0, 320), (2, 2, 1, 0, 320), (3, 0, 0, 0, 512),
                                             (7, 0, 0, 0, 512)])
def test_kernel_adaptive_prefix(backend, kind, mb, nb, ks, k):
    plan = (kind, mb, nb, ks)
    run_case(backend, DENSE4, 50, k, 90, seed=5, adaptive=True, plan=plan)
    # up to 4 raw rows: the row norms are summed inside the GEMM
    run_case(backend, DENSE4, 3, k, 90, seed=6, adaptive=True, plan=plan)


@pytest.mark.parametrize("plan", [(1, 1, 1, 4), (1, 2, 1, 1), (1, 1, 1, 1, 4), (4, 1, 1, 4), (2, 4, 1, 0),
                                  (2, 2, 1, 0, 2), (3, 0, 0, 0), (3, 0, 0, 0, 2), (7, 0, 0, 0), (7, 0, 0, 0, 2)])
@pytest.mark.parametrize("dtype", [torch.int8, torch.int16])
@pytest.mark.parametrize("m", [3, 70, 600])  # row norms summed in the GEMM / folded there / reduced by the norm kernel first
def test_kernel_adaptive_three_of_four_channels(backend, plan, dtype, m):
    # the device picks 3 of the 4 channels: the stream and LDS kernels then
    # run a body without the fourth channel's loads and MFMAs; exact against
    # the full set and the product, twice on one workspace
    if dtype == torch.int16 and plan[0] in (3, 4, 7):
        pytest.skip("the LDS and wide-chunk kernels take raw int8 activations")
    gen = torch.Generator().manual_seed(sum(plan) + dtype.itemsize + m)
    k, n = 512, 200
    a = torch.randint(-8, 9, (m, k), generator=gen).to(dtype)
    b = torch.randint(-127, 128, (k, n), generator=gen).to(torch.int8)
    want = ro.exact_matmul(a.numpy(), b.numpy())
    prepared = backend.prepare_weight_adaptive(b.to(DEV), DENSE4, min_channels=3)
    ws = {4: backend.create_workspace(device=torch.device(DEV), channels=4, m=m, n=n, k=k)}
    for _ in range(2):
        out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), prepared, workspace_by_channels=ws,
                                                          return_metadata=True, plan=plan)
        assert meta["channels"] == 3
        np.testing.assert_array_equal(out.cpu().numpy(), want)
    full = backend.matmul_prepared_fused(a.to(DEV), prepared.variants[4], plan=plan)
    np.testing.assert_array_equal(full.cpu().numpy(), want)


@pytest.mark.parametrize("m,k,big", [(1030, 1088, 1029), (2100, 4160, 2099), (2100, 4160, 5), (300, 4096, 299)])
def test_adaptive_norm_kernel_partial_maxima(backend, m, k, big):
    # past 256 raw rows the norm kernel leaves one maximum per workgroup
    # (each wave two rows a pass, K in passes of 4 KB, the last one partial)
    # and every GEMM wave folds them: one large row anywhere, also the second
    # row of a pass, raises the bound past the 3-channel range
    gen = torch.Generator().manual_seed(m + k + big)
    n = 16
    a = torch.randint(-8, 9, (m, k), generator=gen).to(torch.int8)
    b = torch.randint(-127, 128, (k, n), generator=gen).to(torch.int8)
    b[0, 0] = 127  # max|B| = 127: small rows need 3 channels, a row of 127s 4
    prepared = backend.prepare_weight_adaptive(b.to(DEV), DENSE4, min_channels=3)
    ws = {4: backend.create_workspace(device=torch.device(DEV), channels=4, m=m, n=n, k=k)}
    for planted, channels in ((False, 3), (True, 4)):
        if planted:
            a[big] = 127
        want = ro.exact_matmul(a.numpy(), b.numpy())
        out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), prepared, workspace_by_channels=ws,
                                                          return_metadata=True)
        assert meta["channels"] == channels
        np.testing.assert_array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("kind,mb,nb,ks", [(1, 1, 2, 2), (1, 4, 1, 4), (1, 2, 1, 1), (2, 8, 2, 0), (2, 2, 1, 0),
                                           (3, 0, 0, 0), (7, 0, 0, 0)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_kernel_float_epilogue(backend, kind, mb, nb, ks, out_dtype):
    run_case(backend, DENSE4, 45, 256, 77, seed=9, out_dtype=out_dtype, plan=(kind, mb, nb, ks))


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
def test_plan_rejects_unbuilt_tile(backend, kind, mb, nb, ks):
    prepared = backend.prepare_weight(torch.ones((64, 16), dtype=torch.int8, device=DEV), DENSE4)
    with pytest.raises(ValueError, match="no GEMM kernel"):
        backend.matmul_prepared_fused(torch.ones((4, 64), dtype=torch.int8, device=DEV), prepared,
                                      plan=(kind, mb, nb, ks))


# --------------------------------------------------------------------------
# K split over workgroups: partial sums reduced to residues, exchanged, and
# reconstructed by the last workgroup of each tile
# --------------------------------------------------------------------------
SPLIT_PLANS = [
    # (kind, mb, nb, ks, splits)
    (1, 1, 1, 1, 2), (1, 1, 1, 1, 3), (1, 1, 1, 1, 12), (1, 2, 1, 1, 4), (1, 2, 1, 1, 5),
    (4, 1, 1, 1, 3),
    (2, 2, 1, 4, 2), (2, 3, 1, 4, 2), (2, 4, 1, 3, 3), (2, 4, 1, 4, 5), (2, 2, 1, 3, 2),
    (5, 2, 1, 4, 2), (5, 3, 1, 4, 3), (5, 4, 1, 4, 2),
]


@pytest.mark.parametrize("plan", SPLIT_PLANS, ids=lambda p: "k%d_%dx%d_ks%d_s%d" % p)
@pytest.mark.parametrize("r", [3, 4])
def test_split_k_instances(backend, plan, r):
    mods = SETS[r]
    kind, mb, nb = plan[0], plan[1], plan[2]
    cols = 48 * nb if kind == 5 else (16 * nb if kind in (1, 4) else 64 * nb)
    # ragged M and N; K with a tail inside the last step and several steps
    # per split; each call twice on one workspace (the counters reset)
    run_case(backend, mods, 16 * mb * 2 + 3, 64 * 13 + 16, cols * 3 + 5, seed=r + mb, plan=plan, repeat=2)
    # more splits than K steps: the split count shrinks to the steps
    run_case(backend, mods, 16 * mb + 1, 160, cols + 7, seed=r * 7, plan=plan)
    # residue-plane activations (int16 sources)
    if kind != 5:
        run_case(backend, mods, 9, 200, cols + 3, dtype=torch.int16, seed=r + 2, plan=plan)


@pytest.mark.parametrize("m,k,n,splits", [(512 + 37, 1024, 64 * 5 + 3, 2), (300, 2048, 100, 3),
                                          (256, 4096, 64, 4), (17, 512, 64, 2)])
@pytest.mark.parametrize("kind", LDS_KINDS)
def test_split_k_lds_kernel(backend, m, k, n, splits, kind):
    # whole trips of four stages per split
    run_case(backend, DENSE4, m, k, n, seed=m + splits, plan=(kind, 0, 0, 0, splits), repeat=2)


@pytest.mark.parametrize("m,n,splits", [(517, 64 * 90 - 3, 2), (256 * 2 + 9, 64 * 100 + 5, 4), (300, 64 * 160, 2)])
@pytest.mark.parametrize("kind", LDS_KINDS)
def test_tail_split_lds_kernel(backend, m, n, splits, kind):
    # tiles past the last full round of 256 split (64-column tiles: 270, 300
    # and 320 tiles, 14, 44 and 64 of them split; 96-column tiles: 180, 201
    # and 214 tiles, all in one round, all split), the others whole; ragged
    # M and N
    run_case(backend, DENSE4, m, 1024, n, seed=m + n, plan=(kind, 0, 0, 0, splits, 1), repeat=2)


@pytest.mark.parametrize("plan", [(1, 1, 1, 1, 4), (2, 3, 1, 4, 2), (5, 2, 1, 4, 2), (3, 0, 0, 0, 2),
                                  (7, 0, 0, 0, 2)])
def test_split_k_adaptive_prefix(backend, plan):
    k = 512
    run_case(backend, DENSE4, 50, k, 90, seed=15, adaptive=True, plan=plan, repeat=2)
    run_case(backend, DENSE4, 3, k, 90, seed=16, adaptive=True, plan=plan)


@pytest.mark.parametrize("plan", [(1, 1, 1, 1, 3), (2, 4, 1, 3, 2), (3, 0, 0, 0, 2), (7, 0, 0, 0, 2)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_split_k_float_epilogue(backend, plan, out_dtype):
    run_case(backend, DENSE4, 45, 512, 77, seed=19, out_dtype=out_dtype, plan=plan)


def test_split_k_rejects_unfit_plans(backend):
    prepared = backend.prepare_weight(torch.ones((256, 40), dtype=torch.int8, device=DEV), SETS[6])
    with pytest.raises(ValueError, match="cannot split"):  # more than 4 channels
        backend.matmul_prepared_fused(torch.ones((4, 256), dtype=torch.int8, device=DEV), prepared,
                                      plan=(2, 2, 1, 3, 2))
    prepared = backend.prepare_weight(torch.ones((256, 40), dtype=torch.int8, device=DEV), DENSE4)
    a = torch.ones((4, 256), dtype=torch.int8, device=DEV)
    # stream workgroups of several waves; tiles built without the exchange
    for plan in ((1, 1, 1, 2, 2), (1, 1, 2, 1, 2), (1, 4, 1, 1, 2), (2, 4, 2, 3, 2), (2, 8, 2, 3, 2)):
        with pytest.raises(ValueError, match="cannot split"):
            backend.matmul_prepared_fused(a, prepared, plan=plan)
