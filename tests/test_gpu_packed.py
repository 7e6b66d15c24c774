"""Packed weights: 2 bytes per weight value for any channel count
(rnsmx_prepare_weight_packed / rnsmx_matmul_packed_fused).

  * the device pack equals the oracle's byte split (hi = v >> 8, lo =
    (v & 255) - 128) in the fragment-major layout, padding included;
  * every packed product equals the exact int64 product: stream and MFMA
    kernels (automatic and every forced plan), ragged M, N and K, int8,
    int16 and int32 activations, 4 to 6 channels, int16 extremes;
  * decode shapes on the channel-row kernel (MFMA rows carry channels: 1
    to 8 blocks of 16 / R tokens), every wave count, float epilogues;
  * the device-side adaptive prefix on packed weights picks what the
    oracle's selection picks (5 and 6 channels);
  * RNSLinear with packed_weights equals the residue-plane layer and the
    CPU float chain bit for bit (quant_bits 12 and 16, float32/16/bf16)."""
import numpy as np
import pytest
import torch

from oracle import linear_oracle
from oracle import rns_oracle as ro
from rns_llm_amd import RNSLinear

pytestmark = pytest.mark.gpu

DEV = "cuda"
DENSE6 = (255, 253, 251, 247, 241, 239)
DENSE5 = DENSE6[:5]
DENSE4 = DENSE6[:4]


def ints(shape, lo, hi, seed, dtype=torch.int16):
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, shape, generator=gen, dtype=torch.int32).to(dtype)


def exact(a, w_nk):
    return torch.from_numpy(ro.exact_matmul(a.numpy(), w_nk.t().numpy()))


@pytest.mark.parametrize("n,k", [(1, 1), (37, 100), (64, 1024), (300, 777)])
@pytest.mark.parametrize("dtype", [torch.int8, torch.int16])
def test_pack_layout_matches_oracle_split(backend, n, k, dtype):
    lim = 127 if dtype == torch.int8 else 32767
    w = ints((n, k), -lim - 1, lim, n * 31 + k, dtype)
    w[0, 0] = -lim - 1
    w[-1, -1] = lim
    prepared = backend.prepare_weight_packed_nk(w.to(DEV), DENSE6)
    kp = (k + 63) // 64 * 64
    n16 = (n + 15) // 16
    assert prepared.form == "packed" and prepared.nbytes == 2 * n16 * 16 * kp
    # the fragment grid back to [2][kp][16 n16]: byte 16 l + b of fragment
    # (jb, ks) is column 16 jb + l % 16, K index 64 ks + 16 (l // 16) + b
    grid = prepared.packed.cpu().view(2, n16, kp // 64, 4, 16, 16).permute(0, 2, 3, 5, 1, 4)
    grid = grid.reshape(2, kp, n16 * 16).to(torch.int64)
    hi, lo = ro.pack16_split(w.t().numpy())
    np.testing.assert_array_equal(grid[0, :k, :n].numpy(), hi)
    np.testing.assert_array_equal(grid[1, :k, :n].numpy(), lo)
    # padding holds v = 0: hi 0, lo -128
    assert (grid[0, k:] == 0).all() and (grid[0, :, n:] == 0).all()
    assert (grid[1, k:] == -128).all() and (grid[1, :, n:] == -128).all()
    assert int(prepared.absmax.item()) == int(w.to(torch.int32).abs().max())
    assert torch.equal(prepared.values.cpu(), w.t().to(torch.int32))


# (M, K, N): stream tiles (M <= 64, or 32-row tiles), MFMA tiles of 32 and
# 64 rows, ragged everything, K below one step and spanning many
SHAPES = [(1, 768, 768), (3, 100, 37), (16, 4096, 512), (40, 1000, 300), (96, 768, 2304),
          (129, 768, 2304), (256, 2048, 1000), (500, 64, 70), (1024, 1024, 4096)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("moduli,a_lim", [(DENSE6, 32767), (DENSE5, 2047)], ids=["r6_int16", "r5_int12"])
def test_packed_product_is_exact(backend, m, k, n, moduli, a_lim):
    a = ints((m, k), -a_lim, a_lim, m + k + n)
    w = ints((n, k), -32768, 32767, m * 3 + k)
    a[0, : min(k, 8)] = -a_lim
    w[0, : min(k, 8)] = -32768
    want = exact(a, w)
    prepared = backend.prepare_weight_packed_nk(w.to(DEV), moduli)
    ws = backend.create_workspace(device=torch.device(DEV), channels=len(moduli), m=m, n=n)
    for _ in range(2):
        out = backend.matmul_prepared_fused(a.to(DEV), prepared, workspace=ws)
        assert torch.equal(out.cpu(), want)


# (kind, mb, nb, ks): stream 16 or 32 rows over 1-4 waves, MFMA 32 or 64 rows
PLANS = [(1, 1, 1, 1), (1, 1, 1, 2), (1, 1, 1, 4), (1, 2, 1, 1), (1, 2, 1, 3), (2, 2, 1, 0), (2, 4, 1, 0)]


@pytest.mark.parametrize("plan", PLANS, ids=lambda p: "k%d_%dx%d_ks%d" % p)
@pytest.mark.parametrize("moduli", [DENSE4, DENSE6], ids=["r4", "r6"])
@pytest.mark.parametrize("a_dtype", [torch.int8, torch.int16, torch.int32])
def test_packed_every_plan_and_activation_type(backend, plan, moduli, a_dtype):
    m, k, n = 70, 300, 130
    # 4 channels hold K * 127 * 32767 (int8-range activations); 6 hold int16 ones
    a_lim = 127 if len(moduli) == 4 else 32767
    a = ints((m, k), -a_lim, a_lim, plan[1] * 10 + plan[3], a_dtype)
    w = ints((n, k), -32768, 32767, 5 + len(moduli))
    prepared = backend.prepare_weight_packed_nk(w.to(DEV), moduli)
    out = backend.matmul_prepared_fused(a.to(DEV), prepared, plan=plan)
    assert torch.equal(out.cpu(), exact(a.to(torch.int32), w))


# the residue-plane LDS kernel (kind 8) on packed weights: two staging units
# per channel (a' x hi, a x lo), row terms added before the epilogue
@pytest.mark.parametrize("m,k,n", [(300, 512, 200), (129, 256, 129), (128 * 2 + 37, 1024, 128 * 3 + 5)])
@pytest.mark.parametrize("moduli", [DENSE4, DENSE5, DENSE6], ids=["r4", "r5", "r6"])
@pytest.mark.parametrize("a_dtype", [torch.int8, torch.int16, torch.int32])
def test_packed_lds_kernel(backend, m, k, n, moduli, a_dtype):
    # the worst-case sums must fit the set: K * a_lim * 32768 < P / 2
    a_lim = 16 if len(moduli) == 4 else 127 if a_dtype == torch.int8 else 2047 if len(moduli) == 5 else 32767
    a = ints((m, k), -a_lim, a_lim, m + k + len(moduli), a_dtype)
    w = ints((n, k), -32768, 32767, n + len(moduli))
    a[0, :8] = -a_lim
    w[0, :8] = -32768
    prepared = backend.prepare_weight_packed_nk(w.to(DEV), moduli)
    ws = backend.create_workspace(device=torch.device(DEV), channels=len(moduli), m=m, n=n)
    for _ in range(2):
        out = backend.matmul_prepared_fused(a.to(DEV), prepared, workspace=ws, plan=(8, 0, 0, 0))
        assert torch.equal(out.cpu(), exact(a.to(torch.int32), w))


@pytest.mark.parametrize("moduli", [DENSE4, DENSE6], ids=["r4", "r6"])
def test_packed_lds_kernel_split(backend, moduli):
    # 3 x 86 = 258 tiles: the tail split (the last 2 tiles in two halves of
    # K) and a split of every tile, both equal to the whole-K product; the
    # row terms are added by one half only
    m, k, n = 300, 512, 128 * 86 - 5
    a_lim = 16 if len(moduli) == 4 else 32767
    a = ints((m, k), -a_lim, a_lim, 17 + len(moduli))
    w = ints((n, k), -32768, 32767, 19 + len(moduli))
    prepared = backend.prepare_weight_packed_nk(w.to(DEV), moduli)
    ws = backend.create_workspace(device=torch.device(DEV), channels=len(moduli), m=m, n=n)
    whole = backend.matmul_prepared_fused(a.to(DEV), prepared, workspace=ws, plan=(8, 0, 0, 0)).cpu()
    for plan in ((8, 0, 0, 0, 2, 1), (8, 0, 0, 0, 2, 1), (8, 0, 0, 0, 2)):
        assert torch.equal(backend.matmul_prepared_fused(a.to(DEV), prepared, workspace=ws, plan=plan).cpu(), whole)
    rows = [0, 127, 128, 299]
    assert torch.equal(whole[rows], exact(a[rows].to(torch.int32), w))
    cols = slice(128 * 85 - 7, n)
    assert torch.equal(whole[:, cols], exact(a.to(torch.int32), w[cols]))


# decode: the channel-row kernel (kind 6) with 1, 2, 4 or 8 blocks of 16 / R
# tokens, every wave count, ragged N and K, three activation types
ROW_CASES = [(DENSE6, 1), (DENSE6, 2), (DENSE6, 3), (DENSE6, 4), (DENSE6, 7), (DENSE6, 16), (DENSE4, 1),
             (DENSE4, 5), (DENSE4, 8), (DENSE4, 12), (DENSE4, 32), (DENSE5, 3)]


@pytest.mark.parametrize("moduli,m", ROW_CASES, ids=lambda v: str(len(v)) if isinstance(v, tuple) else str(v))
@pytest.mark.parametrize("ks", [0, 1, 3, 4])
@pytest.mark.parametrize("a_dtype", [torch.int8, torch.int16, torch.int32])
def test_packed_channel_rows_exact(backend, moduli, m, ks, a_dtype):
    k, n = 1000, 77
    a_lim = 127 if len(moduli) == 4 or a_dtype == torch.int8 else 2047 if len(moduli) == 5 else 32767
    a = ints((m, k), -a_lim, a_lim, m * 7 + ks, a_dtype)
    a[0, :4] = -a_lim
    w = ints((n, k), -32768, 32767, 11 * len(moduli) + m)
    w[0, :4] = -32768
    prepared = backend.prepare_weight_packed_nk(w.to(DEV), moduli)
    tpb = 16 // (4 if len(moduli) <= 4 else 6)
    blocks = 1
    while blocks * tpb < m:
        blocks *= 2
    plan = None if ks == 0 else (6, blocks, 1, ks)
    ws = backend.create_workspace(device=torch.device(DEV), channels=len(moduli), m=m, n=n)
    for _ in range(2):
        out = backend.matmul_prepared_fused(a.to(DEV), prepared, workspace=ws, plan=plan)
        assert torch.equal(out.cpu(), exact(a.to(torch.int32), w))


@pytest.mark.parametrize("moduli,m", [(DENSE6, 1), (DENSE6, 3), (DENSE6, 16), (DENSE4, 5)],
                         ids=lambda v: str(len(v)) if isinstance(v, tuple) else str(v))
@pytest.mark.parametrize("a_dtype", [torch.int8, torch.int16, torch.int32])
def test_packed_channel_rows_whole_vectors(backend, moduli, m, a_dtype):
    """K a multiple of 16: the activation encode takes its vector loads (4
    values per thread, int8 / int16 / int32), and every row equals the exact
    product."""
    k, n = 1024, 130
    a_lim = 127 if len(moduli) == 4 or a_dtype == torch.int8 else 32767
    a = ints((m, k), -a_lim, a_lim, m * 5 + k, a_dtype)
    w = ints((n, k), -32768, 32767, 13 * len(moduli) + m)
    prepared = backend.prepare_weight_packed_nk(w.to(DEV), moduli)
    out = backend.matmul_prepared_fused(a.to(DEV), prepared)
    assert torch.equal(out.cpu(), exact(a.to(torch.int32), w))


@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_packed_channel_rows_float_epilogue(backend, m, out_dtype):
    k, n = 4096, 130
    a = ints((m, k), -32767, 32767, m)
    w = ints((n, k), -32767, 32767, m + 1)
    want = exact(a, w)
    gen = torch.Generator().manual_seed(9)
    a_scale = torch.tensor([3e-5], dtype=torch.float32)
    w_scale = torch.rand((n,), generator=gen) * 1e-4
    bias = torch.randn((n,), generator=gen)
    prepared = backend.prepare_weight_packed_nk(w.to(DEV), DENSE6)
    out = torch.empty((m, n), dtype=out_dtype, device=DEV)
    backend.matmul_prepared_fused(a.to(DEV), prepared, out=out, a_scale=a_scale.to(DEV),
                                  w_scale=w_scale.to(DEV), bias=bias.to(DEV))
    ref = ((want.float() * a_scale.view(1, 1)) * w_scale.unsqueeze(0) + bias).to(out_dtype)
    bits = torch.int32 if out_dtype == torch.float32 else torch.int16
    assert torch.equal(out.cpu().view(bits), ref.view(bits))


@pytest.mark.parametrize("m", [1, 3, 7])
@pytest.mark.parametrize("expect,b_max", [(5, 127), (6, 32767)])
def test_packed_adaptive_prefix(backend, m, expect, b_max):
    """As the residue-plane test of the device prefix: int16 activations
    against the 6-channel set, min_channels 3; a row L1 near K * 2^15 times
    max|B| = 127 needs 5 channels, times 32767 needs 6 (on the channel-row
    kernel: 1, 2 or 4 blocks)."""
    k, n = 1024, 40
    a = ints((m, k), -32767, 32767, expect + m)
    a[m // 2] = 32767
    w = ints((n, k), -b_max, b_max, expect + 1)
    w[0, 0] = b_max
    adaptive = backend.prepare_weight_adaptive_nk(w.to(DEV), DENSE6, min_channels=3, packed=True)
    assert adaptive.variants[6].form == "packed" and adaptive.device_selection_is_safe(torch.int16)
    out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), adaptive, return_metadata=True)
    c, bound, cap = ro.adaptive_select(a.numpy(), b_max, DENSE6, min_channels=3)
    assert c == expect
    assert dict(meta) == {"channels": c, "bound": bound, "capacity": cap}
    assert torch.equal(out.cpu(), exact(a, w))


@pytest.mark.parametrize("rows", [1, 3, 33])
@pytest.mark.parametrize("quant_bits", [12, 16])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_rnslinear_packed_equals_planes_and_oracle(backend, quant_bits, dtype, rows):
    k, n = 768, 200
    gen = torch.Generator().manual_seed(quant_bits)
    x = torch.randn((rows, k), generator=gen).to(dtype)
    layers = []
    for packed in (False, True):
        layer = RNSLinear(k, n, mode="rns", backend=backend, quant_bits=quant_bits,
                          packed_weights=packed).to(device=DEV, dtype=dtype).eval()
        layers.append(layer)
    with torch.no_grad():
        layers[1].weight.copy_(layers[0].weight)
        layers[1].bias.copy_(layers[0].bias)
        y_planes = layers[0](x.to(DEV))
        backend.reset_stats()
        y_packed = layers[1](x.to(DEV))
    assert backend.stats_snapshot().get("pack_weight_calls") == 1
    assert layers[1]._prepared_weight.form == "packed"
    assert layers[1]._prepared_weight.nbytes * len(layers[1].moduli) == 2 * layers[0]._prepared_weight.nbytes
    assert torch.equal(y_packed.cpu(), y_planes.cpu())
    want, _ = linear_oracle.linear_forward(x, layers[1].weight.detach().cpu(), layers[1].bias.detach().cpu(),
                                           bits=quant_bits)
    assert torch.equal(y_packed.cpu(), want)


def test_rnslinear_packed_adaptive(backend):
    k, n = 1024, 96
    gen = torch.Generator().manual_seed(3)
    layer = RNSLinear(k, n, mode="rns", backend=backend, quant_bits=16, adaptive_channels=True,
                      packed_weights=True).to(DEV).eval()
    x = torch.randn((5, k), generator=gen)
    with torch.no_grad():
        y = layer(x.to(DEV))
    want, _ = linear_oracle.linear_forward(x, layer.weight.detach().cpu(), layer.bias.detach().cpu(), bits=16)
    assert torch.equal(y.cpu(), want)
