"""Regimes at the edge of the path, each against the oracle or the exact
product:

  * the float epilogue where the integer result is past 2^24 (its int ->
    float32 conversion rounds), on every kernel family and on K splits, and
    RNSLinear at K = 4096 there (the OPT-6.7B width);
  * config C5 at its full shape (M = 1 and 2048, K = 4096, N = 12288), every
    row, fixed and adaptive;
  * the device-side prefix choosing 5 and 6 channels (int16 sources, the
    6-channel dense set, min_channels = 3);
  * the automatic plan at shapes where the kernel-choice rules switch
    family, against another kernel and sampled exact rows;
  * the residue-plane MFMA kernel on both sides of its single-row-tile
    instantiation (streaming weight loads), every row exact;
  * the few-row residue-plane encode and the decode kernels' chunk halves
    with partial last chunks."""
import numpy as np
import pytest
import torch

from oracle import linear_oracle
from oracle import rns_oracle as ro
from rns_llm_amd import RNSLinear

pytestmark = pytest.mark.gpu

DEV = "cuda"
DENSE4 = (255, 253, 251, 247)
DENSE6 = (255, 253, 251, 247, 241, 239)


def large_operands(m, k, n, seed):
    """int8 A, B whose products reach 66 M (> 2^24): rows of A are +-127
    with a few flipped entries, columns of B likewise, so most |y| lie
    between 2^25 and 4096 * 127^2 with low bits set."""
    gen = torch.Generator().manual_seed(seed)
    a = torch.full((m, k), 127, dtype=torch.int16)
    b = torch.full((k, n), 127, dtype=torch.int16)
    a[torch.rand((m, k), generator=gen) < 0.02] = -127
    b[torch.rand((k, n), generator=gen) < 0.03] = -127
    a[::3] = -a[::3]
    b[:, ::5] = torch.randint(-127, 128, (k, b[:, ::5].shape[1]), generator=gen, dtype=torch.int16)
    return a.to(torch.int8), b.to(torch.int8)


PLANS = [(1, 1, 1, 4, 1), (4, 1, 1, 4, 1), (2, 4, 1, 0, 1), (2, 3, 1, 4, 1), (5, 2, 1, 4, 1), (3, 0, 0, 0, 1),
         (1, 1, 1, 1, 4), (2, 2, 1, 4, 4), (3, 0, 0, 0, 2)]


@pytest.mark.parametrize("plan", PLANS, ids=lambda p: "k%d_%dx%d_ks%d_s%d" % p)
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_float_epilogue_past_2_24(backend, plan, out_dtype):
    m, k, n = 37, 4096, 70
    a, b = large_operands(m, k, n, seed=plan[0] * 10 + plan[4])
    want = torch.from_numpy(ro.exact_matmul(a.numpy(), b.numpy()))
    assert int((want.abs() > (1 << 24)).sum()) > m * n // 2
    gen = torch.Generator().manual_seed(3)
    a_scale = torch.tensor([0.0123], dtype=torch.float32)
    w_scale = torch.rand((n,), generator=gen, dtype=torch.float32) * 1e-3
    bias = torch.randn((n,), generator=gen, dtype=torch.float32)
    prepared = backend.prepare_weight(b.to(DEV), DENSE4)
    out = torch.empty((m, n), dtype=out_dtype, device=DEV)
    backend.matmul_prepared_fused(a.to(DEV), prepared, out=out, a_scale=a_scale.to(DEV),
                                  w_scale=w_scale.to(DEV), bias=bias.to(DEV), plan=plan)
    # RNSLinear's output chain on the CPU: int64 -> float32 (round to nearest
    # even), * a_scale, * w_scale, + bias, each rounded, then the cast
    ref = ((want.float() * a_scale.view(1, 1)) * w_scale.unsqueeze(0) + bias).to(out_dtype)
    bits = torch.int32 if out_dtype == torch.float32 else torch.int16
    assert torch.equal(out.cpu().view(bits), ref.view(bits))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_rnslinear_k4096_past_2_24(backend, dtype):
    k, n = 4096, 96
    gen = torch.Generator().manual_seed(21)
    a8, b8 = large_operands(20, k, n, seed=22)
    # RNSLinear quantizes these back to exactly a8 and b8^T (per-tensor and
    # per-row amax 127 * s), so the integer core reaches 66 M
    x = (a8.float() * 0.01).to(dtype)
    layer = RNSLinear(k, n, mode="rns", backend=backend).to(device=DEV, dtype=dtype).eval()
    with torch.no_grad():
        layer.weight.copy_((b8.t().float() * torch.rand((n, 1), generator=gen) * 1e-3).to(dtype))
        layer.bias.copy_(torch.randn((n,), generator=gen).to(dtype))
        y = layer(x.to(DEV))
    want, integer = linear_oracle.linear_forward(x, layer.weight.detach().cpu(), layer.bias.detach().cpu())
    assert int((integer.abs() > (1 << 24)).sum()) > integer.numel() // 2
    assert torch.equal(y.cpu(), want)


@pytest.mark.parametrize("m", [1, 2048])
def test_c5_full_shape_every_row(backend, m):
    k, n = 4096, 12288
    gen = torch.Generator(device=DEV).manual_seed(m)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
    a = torch.randint(-127, 128, (m, k), generator=gen, device=DEV, dtype=torch.int8)
    prepared = backend.prepare_weight_nk(w, DENSE4)
    out = backend.matmul_prepared_fused(a, prepared)
    want = a.double() @ w.double().t()  # exact: |sums| < 2^27
    assert torch.equal(out.double(), want)


@pytest.mark.parametrize("m", [1, 2048])
@pytest.mark.parametrize("tokens", ["normal", "adversarial"])
def test_c5_full_shape_adaptive(backend, m, tokens):
    """C5's adaptive form: per-token int8 of N(0, 1) tokens (the device picks
    its prefix from their row norms) and all +-127 tokens (bound 66,064,384,
    past the 3-channel capacity: the full set)."""
    k, n = 4096, 12288
    gen = torch.Generator(device=DEV).manual_seed(m + 5)
    wf = torch.randn((n, k), generator=gen, device=DEV) * 0.02
    w = torch.clamp(torch.round(wf / (wf.abs().amax(1, keepdim=True) / 127)), -127, 127).to(torch.int8)
    if tokens == "normal":
        xf = torch.randn((m, k), generator=gen, device=DEV)
        a = torch.clamp(torch.round(xf / (xf.abs().amax(1, keepdim=True) / 127)), -127, 127).to(torch.int8)
    else:
        a = torch.full((m, k), 127, dtype=torch.int8, device=DEV)
        a[1::2] = -127
    adaptive = backend.prepare_weight_adaptive_nk(w, DENSE4, min_channels=3)
    assert adaptive.device_selection_is_safe(torch.int8)
    out, meta = backend.matmul_prepared_adaptive_fused(a, adaptive, return_metadata=True)
    assert torch.equal(out.double(), a.double() @ w.double().t())
    c, bound, cap = ro.adaptive_select(a.cpu().numpy(), int(w.abs().max()), DENSE4, min_channels=3)
    assert dict(meta) == {"channels": c, "bound": bound, "capacity": cap}
    if tokens == "adversarial":
        assert c == 4 and bound == 4096 * 127 * int(w.abs().max())


@pytest.mark.parametrize("expect,b_max", [(5, 127), (6, 32767)])
@pytest.mark.parametrize("m", [3, 40])
def test_device_prefix_picks_five_and_six_channels(backend, expect, b_max, m):
    """int16 activations (quant_bits 12/16 sources) against the 6-channel
    dense set with min_channels = 3: a row L1 near K * 2^15 times max|B| =
    127 lands between P_4 / 2 and P_5 / 2 (5 channels), times 32767 between
    P_5 / 2 and P_6 / 2 (6 channels).  Decision, bound and capacity equal the
    oracle's selection; the product is exact."""
    k, n = 1024, 40
    gen = torch.Generator().manual_seed(expect * 100 + m)
    a = torch.randint(-32767, 32768, (m, k), generator=gen, dtype=torch.int32)
    a[m // 2] = 32767  # the largest row in the middle
    b = torch.randint(-b_max, b_max + 1, (k, n), generator=gen, dtype=torch.int32)
    b[0, 0] = b_max
    a16, b16 = a.to(torch.int16), b.to(torch.int16)
    adaptive = backend.prepare_weight_adaptive(b16.to(DEV), DENSE6, min_channels=3)
    assert adaptive.device_selection_is_safe(torch.int16)
    out, meta = backend.matmul_prepared_adaptive_fused(a16.to(DEV), adaptive, return_metadata=True)
    c, bound, cap = ro.adaptive_select(a.numpy(), b_max, DENSE6, min_channels=3)
    assert c == expect
    assert dict(meta) == {"channels": c, "bound": bound, "capacity": cap}
    np.testing.assert_array_equal(out.cpu().numpy(), ro.exact_matmul(a.numpy(), b.numpy()))


# (M, K, N, channels, int16 activations?, kernel kind the automatic plan picks)
AUTO_SHAPES = [
    (1536, 768, 3072, 4, False, 7),   # one round of 256 x 96 tiles where 256 x 64 needs two
    (512, 768, 4608, 4, False, 3),    # one round of 144 LDS tiles at K = 768
    (192, 768, 768, 4, False, 1),     # the stream kernel up to 192 rows
    (8, 2048, 768, 4, False, 4),      # 8-step chunks from K = 2048
    (384, 4096, 3072, 4, False, 2),   # 288 MFMA tiles past one round at long K
    (384, 768, 3072, 4, False, 5),    # the fuller last round on a rows tie
    (96, 768, 768, 6, False, 1),      # raw int8 past 4 channels: the raw stream rule
    (1024, 768, 2304, 6, True, 8),    # residue planes: the LDS kernel from 128 tiles
]


@pytest.mark.parametrize("m,k,n,channels,wide,kind", AUTO_SHAPES,
                         ids=lambda v: str(v) if not isinstance(v, bool) else ("int16" if v else "int8"))
def test_automatic_plan_at_rule_boundaries(backend, m, k, n, channels, wide, kind):
    """The automatic plan at shapes where the kernel-choice rules switch
    family: the kind the host query reports runs, its output equals the
    32 x 64 MFMA kernel's bit for bit, and sampled rows equal the exact
    product."""
    import ctypes

    from rns_llm_amd import _native

    mods = DENSE4 if channels == 4 else DENSE6
    plan = _native.Plan()
    _native.check(_native.lib().rnsmx_gemm_plan(m, n, k, channels, 0 if wide else 1, ctypes.byref(plan)))
    assert plan.kind == kind
    gen = torch.Generator().manual_seed(m + k + n + channels)
    lo, hi, dt = (-32767, 32768, torch.int16) if wide else (-127, 128, torch.int8)
    a = torch.randint(lo, hi, (m, k), generator=gen, dtype=torch.int32).to(dt)
    b = torch.randint(lo, hi, (k, n), generator=gen, dtype=torch.int32).to(dt)
    prepared = backend.prepare_weight(b.to(DEV), mods)
    out = backend.matmul_prepared_fused(a.to(DEV), prepared)
    other = backend.matmul_prepared_fused(a.to(DEV), prepared, plan=(2, 2, 1, 0))
    assert torch.equal(out, other)
    rows = torch.randperm(m, generator=gen)[:24]
    want = ro.exact_matmul(a[rows].numpy(), b.numpy())
    np.testing.assert_array_equal(out.cpu()[rows].numpy(), want)



@pytest.mark.parametrize("m,mb", [(1, 2), (32, 2), (33, 2), (1, 4), (17, 4), (64, 4), (65, 4)])
@pytest.mark.parametrize("channels", [4, 6])
def test_residue_plane_mfma_single_and_several_row_tiles(backend, m, mb, channels):
    """The residue-plane MFMA kernel loads its weights with the streaming
    hint when one row tile covers M (a separate instantiation) and with
    plain loads otherwise: both sides of that switch, at a ragged K and N
    (padding steps and a partial last column tile), equal the exact product
    on every row (int16 operands; within +-255 for 4 channels, whose range
    holds K * 255^2)."""
    mods = DENSE4 if channels == 4 else DENSE6
    lim = 256 if channels == 4 else 32768
    k, n = 1000, 1000
    gen = torch.Generator().manual_seed(m * 7 + mb + channels)
    a = torch.randint(1 - lim, lim, (m, k), generator=gen, dtype=torch.int32).to(torch.int16)
    b = torch.randint(1 - lim, lim, (k, n), generator=gen, dtype=torch.int32).to(torch.int16)
    prepared = backend.prepare_weight(b.to(DEV), mods)
    out = backend.matmul_prepared_fused(a.to(DEV), prepared, plan=(2, mb, 1, 0))
    np.testing.assert_array_equal(out.cpu().numpy(), ro.exact_matmul(a.numpy(), b.numpy()))


@pytest.mark.parametrize("k", [1000, 1024])
@pytest.mark.parametrize("a_dtype", [torch.int16, torch.int32])
@pytest.mark.parametrize("m", [1, 16, 17])
def test_few_row_residue_plane_encode(backend, k, a_dtype, m):
    """Up to 16 rows the residue-plane encode runs split over K (one thread
    per 4 values; 17 rows take the per-row encoder): vector and ragged K,
    int16 and int32 activations, every row exact."""
    gen = torch.Generator().manual_seed(k + m)
    a = torch.randint(-32767, 32768, (m, k), generator=gen, dtype=torch.int32).to(a_dtype)
    b = torch.randint(-32767, 32768, (k, 200), generator=gen, dtype=torch.int32).to(torch.int16)
    prepared = backend.prepare_weight(b.to(DEV), DENSE6)
    out = backend.matmul_prepared_fused(a.to(DEV), prepared)
    np.testing.assert_array_equal(out.cpu().numpy(), ro.exact_matmul(a.to(torch.int32).numpy(), b.numpy()))


@pytest.mark.parametrize("k", [4288, 2131])
@pytest.mark.parametrize("ks", [1, 2, 3, 4])
@pytest.mark.parametrize("m", [1, 5])
def test_long_k_chunk_halves_partial_chunks(backend, k, ks, m):
    """The 8-step stream chunks and the channel-row kernel walk the halves of
    each chunk in turn; with K = 67 (or a ragged 34) steps of 64 the last
    chunk of a wave is partly or wholly past K.  Raw int8 through the stream
    plan and int16 through packed weights, every row exact."""
    gen = torch.Generator().manual_seed(k * 10 + ks + m)
    a = torch.randint(-127, 128, (m, k), generator=gen, dtype=torch.int32).to(torch.int8)
    b = torch.randint(-127, 128, (k, 300), generator=gen, dtype=torch.int32).to(torch.int8)
    prepared = backend.prepare_weight(b.to(DEV), DENSE4)
    out = backend.matmul_prepared_fused(a.to(DEV), prepared, plan=(4, 1, 1, ks))
    np.testing.assert_array_equal(out.cpu().numpy(), ro.exact_matmul(a.to(torch.int32).numpy(), b.numpy()))
    a16 = torch.randint(-32767, 32768, (m, k), generator=gen, dtype=torch.int32).to(torch.int16)
    w16 = torch.randint(-32767, 32768, (300, k), generator=gen, dtype=torch.int32).to(torch.int16)
    packed = backend.prepare_weight_packed_nk(w16.to(DEV), DENSE6)
    blocks = 1 if m <= 2 else 4
    out16 = backend.matmul_prepared_fused(a16.to(DEV), packed, plan=(6, blocks, 1, ks))
    np.testing.assert_array_equal(out16.cpu().numpy(),
                                  ro.exact_matmul(a16.to(torch.int32).numpy(), w16.to(torch.int32).numpy().T))
