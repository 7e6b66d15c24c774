"""GPU parity: every result of the HIP path equals the CPU oracle / exact
int64 product bit for bit (integer outputs) or the op-by-op float chain bit
for bit (dequantized outputs).  Mirrors tests/test_cuda_backend.py of the
reference plus the BASELINE configs and their edge cases."""
import glob
import os

import numpy as np
import pytest
import torch
from torch import nn

from oracle import c_oracle, linear_oracle
from oracle import rns_oracle as ro
from rns_llm_amd import RNSLinear, RNSQKVProjection, choose_moduli_for_dot

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
DENSE4 = (255, 253, 251, 247)
DEV = "cuda"


def rand_i8(gen, shape, lo=-127, hi=127):
    return torch.randint(lo, hi + 1, shape, dtype=torch.int8, generator=gen)


def exact(a, b):
    return ro.exact_matmul(np.asarray(a), np.asarray(b))


# --------------------------------------------------------------------------
# encode
# --------------------------------------------------------------------------
@pytest.mark.parametrize("moduli", [DENSE4, (251, 241, 239, 233), (3, 5, 7, 11, 13, 17, 19, 23, 29, 31),
                                    (254, 253, 251), (2, 3)])
def test_encode_int8_exhaustive(backend, moduli):
    v = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8).repeat(3)[:700]  # ragged numel
    got = backend.encode_centered(v.to(DEV), moduli).cpu().numpy()
    np.testing.assert_array_equal(got, ro.encode_centered(v.numpy(), moduli))


@pytest.mark.parametrize("dtype", [torch.int16, torch.int32])
def test_encode_wide_dtypes(backend, dtype):
    gen = torch.Generator().manual_seed(3)
    info = torch.iinfo(dtype)
    v = torch.randint(info.min, info.max, (33, 47), dtype=torch.int64, generator=gen).to(dtype)
    v[0, :4] = torch.tensor([info.min, info.max, 0, -1], dtype=dtype)
    got = backend.encode_centered(v.to(DEV), DENSE4).cpu().numpy()
    assert got.shape == (4, 33, 47)
    np.testing.assert_array_equal(got, ro.encode_centered(v.numpy(), DENSE4))


def test_encode_empty(backend):
    out = backend.encode_centered(torch.empty((0, 5), dtype=torch.int8, device=DEV), DENSE4)
    assert out.shape == (4, 0, 5)


# --------------------------------------------------------------------------
# golden vectors through both fused entry points
# --------------------------------------------------------------------------
GOLDEN_CASES = [p for p in sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))
                if "expected" in np.load(p)]


@pytest.mark.parametrize("path", GOLDEN_CASES, ids=lambda p: os.path.basename(p)[:-4])
@pytest.mark.parametrize("lut", [0, 2])
def test_golden_prepared_fused(backend, path, lut):
    g = np.load(path)
    mods = tuple(int(m) for m in g["moduli"])
    a = torch.from_numpy(g["a"]).to(DEV)
    b = torch.from_numpy(g["b"]).to(DEV)
    prepared = backend.prepare_weight(b, mods)
    out = backend.matmul_prepared_fused(a, prepared, lut_channels=min(lut, len(mods)))
    np.testing.assert_array_equal(out.cpu().numpy(), g["expected"])


@pytest.mark.parametrize("path", GOLDEN_CASES, ids=lambda p: os.path.basename(p)[:-4])
def test_golden_centered_fused_dropin(backend, path):
    g = np.load(path)
    mods = tuple(int(m) for m in g["moduli"])
    a = torch.from_numpy(g["a"]).to(DEV)
    b = torch.from_numpy(g["b"]).to(DEV)
    out = backend.matmul_wide_fused(a, b, mods, lut_channels=1)
    np.testing.assert_array_equal(out.cpu().numpy(), g["expected"])


# --------------------------------------------------------------------------
# shapes: skinny and tiled kernels, ragged edges, every channel capacity
# --------------------------------------------------------------------------
SHAPES = [(1, 768, 2304), (4, 768, 768), (16, 768, 2304), (17, 64, 20), (33, 100, 37),
          (64, 768, 96), (65, 768, 130), (128, 768, 2304), (256, 768, 2304), (300, 200, 333),
          (1024, 768, 256)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_prepared_fused_shapes(backend, m, k, n):
    gen = torch.Generator().manual_seed(m * 7 + k + n)
    a = rand_i8(gen, (m, k))
    b = rand_i8(gen, (k, n))
    mods = choose_moduli_for_dot(k, 127, 127, strategy="dense_coprime")
    prepared = backend.prepare_weight(b.to(DEV), mods)
    out = backend.matmul_prepared_fused(a.to(DEV), prepared, lut_channels=2)
    np.testing.assert_array_equal(out.cpu().numpy(), exact(a, b))


@pytest.mark.parametrize("mods,amax", [((3, 5, 7, 11, 13, 17, 19, 23, 29, 31), 60),
                                       ((251, 241, 239, 233, 229), 127),
                                       ((255, 253, 251, 247, 241, 239), 127),
                                       ((127, 125, 121, 113), 127),
                                       ((251, 241), 3)])
@pytest.mark.parametrize("m", [5, 96])
def test_channel_counts(backend, mods, amax, m):
    gen = torch.Generator().manual_seed(len(mods) * 100 + m)
    k, n = 64, 48
    a = rand_i8(gen, (m, k), -amax, amax)
    b = rand_i8(gen, (k, n), -amax, amax)
    prepared = backend.prepare_weight(b.to(DEV), mods)
    out = backend.matmul_prepared_fused(a.to(DEV), prepared, lut_channels=min(2, len(mods)))
    np.testing.assert_array_equal(out.cpu().numpy(), ro.rns_matmul_centered(a.numpy(), b.numpy(), mods))


def test_wraparound_matches_oracle(backend):
    # product outside the centered range: the device reduces mod P exactly as
    # the reference's Garner path does (both C and NumPy oracles agree)
    mods = (3, 5, 7, 11)
    gen = torch.Generator().manual_seed(8)
    a = rand_i8(gen, (9, 16))
    b = rand_i8(gen, (16, 5))
    prepared = backend.prepare_weight(b.to(DEV), mods)
    out = backend.matmul_prepared_fused(a.to(DEV), prepared).cpu().numpy()
    np.testing.assert_array_equal(out, c_oracle.rns_matmul_centered(a.numpy(), b.numpy(), mods))


def test_int16_wide_inputs(backend):
    # tests/test_cuda_backend.py:49-58 and :73-94 (int12, lut 0/1/2)
    gen = torch.Generator().manual_seed(12)
    a = torch.randint(-2047, 2048, (24, 64), dtype=torch.int16, generator=gen)
    b = torch.randint(-2047, 2048, (64, 32), dtype=torch.int16, generator=gen)
    mods = choose_moduli_for_dot(64, 2047, 2047, strategy="dense_coprime")
    want = exact(a, b)
    np.testing.assert_array_equal(backend.matmul_wide(a.to(DEV), b.to(DEV), mods).cpu().numpy(), want)
    prepared = backend.prepare_weight(b.to(DEV), mods)
    for lut in (0, 1, 2):
        out = backend.matmul_prepared_fused(a.to(DEV), prepared, lut_channels=lut)
        np.testing.assert_array_equal(out.cpu().numpy(), want)


def test_int16_source_five_six_channels(backend):
    # quant_bits 12/16 style sources: K=768 needs 5 (int12) or 6+ channels
    gen = torch.Generator().manual_seed(16)
    for bits, amax in ((12, 2047), (16, 4000)):
        k = 768
        mods = choose_moduli_for_dot(k, amax, amax, strategy="dense_coprime")
        assert len(mods) >= 5
        a = torch.randint(-amax, amax + 1, (7, k), dtype=torch.int16, generator=gen)
        b = torch.randint(-amax, amax + 1, (k, 40), dtype=torch.int16, generator=gen)
        prepared = backend.prepare_weight(b.to(DEV), mods)
        out = backend.matmul_prepared_fused(a.to(DEV), prepared, lut_channels=2)
        np.testing.assert_array_equal(out.cpu().numpy(), exact(a, b))


# --------------------------------------------------------------------------
# reference backend contract
# --------------------------------------------------------------------------
def test_prepared_matches_uncached(backend):
    # tests/test_cuda_backend.py:61-71
    gen = torch.Generator().manual_seed(24)
    a = rand_i8(gen, (24, 64)).to(DEV)
    b = rand_i8(gen, (64, 32)).to(DEV)
    mods = choose_moduli_for_dot(64, 127, 127)
    prepared = backend.prepare_weight(b, mods)
    torch.testing.assert_close(backend.matmul_prepared(a, prepared),
                               backend.matmul_wide(a, b, mods), rtol=0, atol=0)


def test_garner_decoder_matches_crt_decoder(backend):
    # tests/test_cuda_backend.py:97-108
    gen = torch.Generator().manual_seed(32)
    a = rand_i8(gen, (32, 64)).to(DEV)
    b = rand_i8(gen, (64, 32)).to(DEV)
    mods = choose_moduli_for_dot(64, 127, 127, strategy="dense_coprime")
    residues = backend.matmul_centered_residues(backend.encode_centered(a, mods),
                                                backend.encode_centered(b, mods), mods)
    canon = ro.matmul_residues(ro.encode_canonical(a.cpu().numpy(), mods),
                               ro.encode_canonical(b.cpu().numpy(), mods), mods)
    want = np.stack([np.where(canon[c] > m // 2, canon[c] - m, canon[c]) for c, m in enumerate(mods)])
    np.testing.assert_array_equal(residues.cpu().numpy(), want)
    new = backend.decode_garner(residues, mods)
    old = backend.decode(residues, mods)
    torch.testing.assert_close(new, old, rtol=0, atol=0)
    np.testing.assert_array_equal(new.cpu().numpy(), exact(a.cpu(), b.cpu()))


def test_decode_garner_known_answer(backend):
    g = np.load(os.path.join(GOLDEN, "ref_garner_values.npz"))
    mods = tuple(int(m) for m in g["moduli"])
    res = torch.from_numpy(ro.encode_centered(g["values"], mods)).to(DEV)
    np.testing.assert_array_equal(backend.decode_garner(res, mods).cpu().numpy(), g["values"])


def test_continuous_batch_matches_independent_requests(backend):
    # tests/test_cuda_backend.py:111-138
    gen = torch.Generator().manual_seed(64)
    mods = choose_moduli_for_dot(64, 127, 127, strategy="dense_coprime")
    weight = rand_i8(gen, (64, 32))
    prepared = backend.prepare_weight(weight.to(DEV), mods)
    requests = [rand_i8(gen, (rows, 64)).to(DEV) for rows in (1, 3, 5, 2)]
    ws = backend.create_request_batch_workspace(
        device=torch.device(DEV), dtype=torch.int8, rows_per_request=[r.shape[0] for r in requests],
        k=64, channels=len(mods), n=32)
    merged = backend.matmul_prepared_fused_requests(requests, prepared, workspace=ws,
                                                    clone_outputs=True)
    for req, got in zip(requests, merged):
        torch.testing.assert_close(got, backend.matmul_prepared_fused(req, prepared), rtol=0, atol=0)
        np.testing.assert_array_equal(got.cpu().numpy(), exact(req.cpu(), weight))
    stats = backend.stats_snapshot()
    assert stats["continuous_batch_calls"] >= 1


@pytest.mark.parametrize("requests", [1, 2, 4])
def test_c3_decode_requests(backend, requests):
    gen = torch.Generator().manual_seed(300 + requests)
    w = rand_i8(gen, (768, 768))
    prepared = backend.prepare_weight(w.to(DEV), DENSE4)
    reqs = [rand_i8(gen, (1, 768)).to(DEV) for _ in range(requests)]
    merged = backend.matmul_prepared_fused_requests(reqs, prepared, clone_outputs=True)
    for req, got in zip(reqs, merged):
        np.testing.assert_array_equal(got.cpu().numpy(), exact(req.cpu(), w))


def test_adaptive_prefix_exact_and_falls_back(backend):
    # tests/test_cuda_backend.py:141-162 (device-side selection)
    gen = torch.Generator().manual_seed(141)
    mods = choose_moduli_for_dot(64, 127, 127, strategy="dense_coprime")
    weight = rand_i8(gen, (64, 32), -40, 40)
    adaptive = backend.prepare_weight_adaptive(weight.to(DEV), mods, min_channels=3)
    for lo, expect_c in ((8, 3), (127, None)):
        a = rand_i8(gen, (16, 64), -lo, lo)
        out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), adaptive, return_metadata=True)
        np.testing.assert_array_equal(out.cpu().numpy(), exact(a, weight))
        c, bound, cap = ro.adaptive_select(a.numpy(), int(weight.abs().max()), mods, min_channels=3)
        assert (meta["channels"], meta["bound"], meta["capacity"]) == (c, bound, cap)
        assert meta["bound"] <= meta["capacity"]
        if expect_c is not None:
            assert meta["channels"] == expect_c
    assert adaptive.max_abs_weight == int(weight.abs().max())


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("k", [4096, 1040])
def test_adaptive_small_batches(backend, m, k):
    # up to 4 raw int8 rows the GEMM workgroups sum the row norms themselves
    # (no encoder launch); 5 and more take the encoder's norms: both must
    # give the oracle's prefix, bound and capacity and the exact product
    gen = torch.Generator().manual_seed(m * 10 + k)
    b = rand_i8(gen, (k, 48))
    adaptive = backend.prepare_weight_adaptive(b.to(DEV), DENSE4, min_channels=3)
    for lo in (4, 127):
        a = rand_i8(gen, (m, k), -lo, lo)
        a[m - 1, : k // 2] = lo  # the largest row last
        out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), adaptive, return_metadata=True)
        np.testing.assert_array_equal(out.cpu().numpy(), exact(a, b))
        c, bound, cap = ro.adaptive_select(a.numpy(), int(b.abs().max()), DENSE4, min_channels=3)
        assert (meta["channels"], meta["bound"], meta["capacity"]) == (c, bound, cap)


def test_adaptive_adversarial_full_set_k4096(backend):
    # C5 edge: all +-127 at K=4096 -> bound 66,064,384, prefix 3 cannot hold
    # it, so the device must pick the full 4-channel set
    k, n = 4096, 64
    a = torch.full((3, k), 127, dtype=torch.int8)
    a[1] = -127
    a[2, ::2] = -127
    b = torch.full((k, n), 127, dtype=torch.int8)
    b[:, ::3] = -127
    adaptive = backend.prepare_weight_adaptive(b.to(DEV), DENSE4, min_channels=3)
    out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), adaptive, return_metadata=True)
    np.testing.assert_array_equal(out.cpu().numpy(), exact(a, b))
    assert meta["channels"] == 4 and meta["bound"] == 4096 * 127 * 127


@pytest.mark.parametrize("return_metadata", [False, True])
def test_adaptive_overflow_raises_before_computing(backend, return_metadata):
    # adaptive.py:36-41: callers must never silently wrap around.  A
    # two-channel set cannot hold full-range int8 products, so preparation
    # cannot prove the device selection safe: the call takes the
    # reference's synchronous selection and raises before any launch.
    mods = (251, 241)
    gen = torch.Generator().manual_seed(5)
    b = rand_i8(gen, (64, 8))
    a = rand_i8(gen, (4, 64))
    adaptive = backend.prepare_weight_adaptive(b.to(DEV), mods, min_channels=2)
    assert not adaptive.device_selection_is_safe(torch.int8)
    ws = backend.create_workspace(device=torch.device(DEV), channels=2, m=4, n=8, k=64)
    ws.output.fill_(-7)
    backend.reset_stats()
    with pytest.raises(OverflowError):
        backend.matmul_prepared_adaptive_fused(a.to(DEV), adaptive, workspace_by_channels={2: ws},
                                               return_metadata=return_metadata)
    torch.cuda.synchronize()
    assert bool((ws.output == -7).all())
    assert backend.stats_snapshot().get("fused_gemm_calls", 0) == 0


def test_rnslinear_adaptive_with_undersized_moduli_raises(backend):
    layer = RNSLinear(64, 8, mode="rns", backend=backend, moduli=(251, 241), adaptive_channels=True,
                      adaptive_min_channels=2).to(DEV).eval()
    with torch.no_grad():
        layer.weight.copy_(torch.linspace(-1, 1, 64 * 8).reshape(8, 64))
    with pytest.raises(OverflowError):
        layer(torch.ones((3, 64), device=DEV))


def test_adaptive_synchronous_path_is_exact_and_counted(backend):
    # a set too small for worst-case int8 products but large enough for
    # these: the synchronous selection picks 3 of 4 channels, exactly as
    # select_adaptive_variant + matmul_prepared_fused do in the reference
    mods = (13, 11, 7, 5)
    gen = torch.Generator().manual_seed(9)
    b = rand_i8(gen, (64, 24), -2, 2)
    a = rand_i8(gen, (5, 64), -2, 2)
    adaptive = backend.prepare_weight_adaptive(b.to(DEV), mods, min_channels=2)
    assert not adaptive.device_selection_is_safe(torch.int8)
    backend.reset_stats()
    out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), adaptive, return_metadata=True)
    np.testing.assert_array_equal(out.cpu().numpy(), exact(a, b))
    c, bound, cap = ro.adaptive_select(a.numpy(), int(b.abs().max()), mods, min_channels=2)
    assert dict(meta) == {"channels": c, "bound": bound, "capacity": cap}
    stats = backend.stats_snapshot()
    assert stats["adaptive_selections"] == 1 and stats[f"adaptive_channels_{c}"] == 1
    assert stats["fused_gemm_calls"] == 1 and stats[f"fused_gemm_channels_{c}"] == 1


def test_adaptive_device_path_counts_prefix_when_read(backend):
    # the default dense set holds every int8 product at this K: the prefix
    # is chosen on the device, and counted once, when the metadata is read
    gen = torch.Generator().manual_seed(10)
    b = rand_i8(gen, (256, 40), -40, 40)
    a = rand_i8(gen, (6, 256), -8, 8)
    adaptive = backend.prepare_weight_adaptive(b.to(DEV), DENSE4, min_channels=3)
    assert adaptive.device_selection_is_safe(torch.int8)
    backend.reset_stats()
    out, meta = backend.matmul_prepared_adaptive_fused(a.to(DEV), adaptive, return_metadata=True)
    stats = backend.stats_snapshot()
    assert stats["adaptive_selections"] == 1 and stats["fused_gemm_calls"] == 1
    assert not any(key.startswith(("fused_gemm_channels_", "adaptive_channels_")) for key in stats)
    assert meta["channels"] == 3 and meta["channels"] == 3  # read twice, counted once
    stats = backend.stats_snapshot()
    assert stats["adaptive_channels_3"] == 1 and stats["fused_gemm_channels_3"] == 1
    np.testing.assert_array_equal(out.cpu().numpy(), exact(a, b))


def test_streams_have_independent_workspaces(backend):
    gen = torch.Generator().manual_seed(77)
    w = rand_i8(gen, (768, 512))
    prepared = backend.prepare_weight(w.to(DEV), DENSE4)
    xs = [rand_i8(gen, (32, 768)) for _ in range(4)]
    streams = [torch.cuda.Stream() for _ in range(4)]
    outs = []
    torch.cuda.synchronize()
    for x, s in zip(xs, streams):
        with torch.cuda.stream(s):
            ws = backend.create_workspace(device=torch.device(DEV), channels=4, m=32, n=512, k=768)
            xd = x.to(DEV, non_blocking=False)
            outs.append((backend.matmul_prepared_fused(xd, prepared, workspace=ws), ws))
    torch.cuda.synchronize()
    for x, (o, _) in zip(xs, outs):
        np.testing.assert_array_equal(o.cpu().numpy(), exact(x, w))


def test_validation_errors(backend):
    a = torch.zeros((4, 64), dtype=torch.int8, device=DEV)
    prepared = backend.prepare_weight(torch.zeros((64, 8), dtype=torch.int8, device=DEV), DENSE4)
    with pytest.raises(ValueError):
        backend.matmul_prepared_fused(torch.zeros((4, 32), dtype=torch.int8, device=DEV), prepared)
    with pytest.raises(ValueError):
        backend.matmul_prepared_fused(a.float(), prepared)
    with pytest.raises(ValueError):
        backend.matmul_prepared_fused(a, prepared, lut_channels=3)
    ws = backend.create_workspace(device=torch.device(DEV), channels=4, m=5, n=8)
    with pytest.raises(ValueError):
        backend.matmul_prepared_fused(a, prepared, workspace=ws)
    with pytest.raises(ValueError):
        backend.matmul_centered_fused(torch.zeros((3, 4, 64), dtype=torch.int8, device=DEV),
                                      torch.zeros((4, 64, 8), dtype=torch.int8, device=DEV), DENSE4)


# --------------------------------------------------------------------------
# float epilogue and the RNSLinear / fused QKV layers
# --------------------------------------------------------------------------
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_dequant_epilogue_matches_torch_chain(backend, out_dtype):
    gen = torch.Generator().manual_seed(9)
    m, k, n = 37, 768, 200
    a = rand_i8(gen, (m, k)).to(DEV)
    b = rand_i8(gen, (k, n)).to(DEV)
    a_scale = torch.rand(1, generator=gen).to(DEV) * 0.01 + 1e-3
    w_scale = (torch.rand(n, generator=gen) * 0.01 + 1e-4).to(DEV)
    bias = torch.randn(n, generator=gen).to(DEV)
    prepared = backend.prepare_weight(b, DENSE4)
    integer = backend.matmul_prepared_fused(a, prepared).clone()
    want = ((integer.float() * a_scale.view(1, 1)) * w_scale.unsqueeze(0) + bias).to(out_dtype)
    out = torch.empty((m, n), dtype=out_dtype, device=DEV)
    backend.matmul_prepared_fused(a, prepared, out=out, a_scale=a_scale, w_scale=w_scale, bias=bias)
    assert torch.equal(out.view(torch.int16 if out_dtype != torch.float32 else torch.int32),
                       want.view(torch.int16 if out_dtype != torch.float32 else torch.int32))


def make_opt_linears(hidden=768, seed=17, dtype=torch.float16):
    torch.manual_seed(seed)
    return tuple(nn.Linear(hidden, hidden, bias=True, device=DEV, dtype=dtype).eval()
                 for _ in range(3))


@pytest.mark.parametrize("tokens", [1, 16, 128, 256])
@pytest.mark.parametrize("fused_epilogue", [True, False])
def test_fused_qkv_equals_three_rnslinear_and_oracle(backend, tokens, fused_epilogue):
    originals = make_opt_linears()
    kw = dict(backend=backend, mode="rns", fused=True, lut_channels=2, fused_epilogue=fused_epilogue)
    separate = [RNSLinear.from_linear(l, **kw).eval() for l in originals]
    fused = RNSQKVProjection.from_linears(*originals, **{k: v for k, v in kw.items()}).eval()
    gen = torch.Generator().manual_seed(tokens)
    x = torch.randn(1, tokens, 768, generator=gen).to(DEV, torch.float16)
    fused_out = fused(x)
    for part, layer, orig in zip(fused_out, separate, originals):
        sep = layer(x)
        assert torch.equal(part, sep)                     # fused == three separate, bit-exact
        want, _ = linear_oracle.linear_forward(x.cpu(), orig.weight.cpu(), orig.bias.cpu())
        assert torch.equal(sep.cpu(), want)               # == the reference float chain


def test_rnslinear_adaptive_matches_oracle(backend):
    torch.manual_seed(3)
    lin = nn.Linear(256, 96, device=DEV).eval()
    layer = RNSLinear.from_linear(lin, backend=backend, mode="rns", adaptive_channels=True).eval()
    x = torch.randn(5, 256, device=DEV) * 0.05
    y = layer(x)
    want, integer = linear_oracle.linear_forward(x.cpu(), lin.weight.cpu(), lin.bias.cpu())
    assert torch.equal(y.cpu(), want)
    meta = layer.last_adaptive_metadata
    assert meta["bound"] <= meta["capacity"]


def test_rnslinear_weight_version_invalidates_cache(backend):
    torch.manual_seed(4)
    lin = nn.Linear(64, 32, device=DEV).eval()
    layer = RNSLinear.from_linear(lin, backend=backend, mode="rns").eval()
    x = torch.randn(3, 64, device=DEV)
    layer(x)
    first = layer._prepared_weight
    layer(x)
    assert layer._prepared_weight is first
    with torch.no_grad():
        layer.weight.mul_(2.0)
    y = layer(x)
    assert layer._prepared_weight is not first
    want, _ = linear_oracle.linear_forward(x.cpu(), layer.weight.detach().cpu(), layer.bias.detach().cpu())
    assert torch.equal(y.cpu(), want)


def test_rnslinear_rejects_misshaped_inputs_before_and_after_binding(backend):
    # the reference's flatten-and-restore raises RuntimeError on every input
    # whose last dimension is not in_features; here that holds on the first
    # call and on calls after the one-call forward is bound, and the bad call
    # writes nothing
    torch.manual_seed(5)
    lin = nn.Linear(4, 8, device=DEV).eval()
    layer = RNSLinear.from_linear(lin, backend=backend, mode="rns").eval()
    bad = [torch.randn(2, 8, device=DEV), torch.randn(3, 2, device=DEV), torch.randn(5, 3, device=DEV),
           torch.randn((), device=DEV)]
    for x in bad:  # nothing bound yet
        with pytest.raises(RuntimeError):
            layer(x)
    good = torch.randn(3, 4, device=DEV)
    y = layer(good)  # binds the one-call path
    assert layer._linear_call is not None
    for x in bad:
        with pytest.raises(RuntimeError):
            layer(x)
    want, _ = linear_oracle.linear_forward(good.cpu(), layer.weight.detach().cpu(), layer.bias.detach().cpu())
    assert torch.equal(y.cpu(), want)
    assert torch.equal(layer(good).cpu(), want)
    # a switch of the path's options re-binds (or unbinds) the one-call path
    layer.fused_epilogue = False
    assert torch.equal(layer(good).cpu(), want)
    assert layer._linear_call is None


# ---------------------------------------------------------------------------
# activation quantization (RNSLinear._symmetric_scale / _quantize)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 768), (3, 100), (256, 768), (4096, 768), (2, 5, 33),
                                   (16, 1024), (1, 16385)])  # one-workgroup form up to 16384 values
@pytest.mark.parametrize("bits", [8, 12])
def test_quantize_symmetric_matches_reference_chain(backend, dtype, shape, bits):
    gen = torch.Generator().manual_seed(sum(shape) + bits)
    x = (torch.randn(shape, generator=gen) * 3).to(dtype)
    # a few fixed values: zeros of both signs, halves, the largest magnitude
    x.view(-1)[: min(8, x.numel())] = torch.tensor([0.5, -0.5, 1.5, -2.5, 0.0, -0.0, 3.5, 127.0],
                                                  dtype=dtype)[: min(8, x.numel())]
    q, scale = backend.quantize_symmetric(x.to(DEV), bits)
    want_q, want_scale = linear_oracle.quantize_activations(x, shape[-1], bits)
    assert scale.shape == (1, 1) and torch.equal(scale.cpu(), want_scale)
    assert torch.equal(q.cpu().reshape(-1, shape[-1]), want_q)
    # the scratch is left ready: a second call on the same stream agrees
    q2, scale2 = backend.quantize_symmetric(x.to(DEV), bits)
    assert torch.equal(q2, q) and torch.equal(scale2, scale)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [8, 12, 16])
def test_oracle_quantization_matches_torch_gpu_ops(dtype, bits):
    """The reference RNSLinear runs its activation quantization with torch on
    the GPU (rns_linear.py:154-166, after flat = inputs.reshape(-1, K).float());
    the oracle restates it on the CPU with the GPU's rounding of
    ``tensor / 127.0``.  Pin that restatement against torch's own GPU ops:
    10^5 tensors per dtype and bit width as the rows of one batch (amax per
    row; the division is the same elementwise kernel as in the per-tensor
    form), then 200 separate calls in the reference's exact per-tensor form.
    A correctly rounded GPU division would fail the scale comparison."""
    qmax = (1 << (bits - 1)) - 1
    eps = torch.finfo(torch.float32).eps
    gen = torch.Generator().manual_seed(1000 * bits + {torch.float32: 1, torch.float16: 2, torch.bfloat16: 3}[dtype])
    rows, cols = 100_000, 16
    span = 8 if dtype == torch.float16 else 40  # binades of the row magnitudes (fp16 must not overflow)
    mag = torch.exp2(torch.randint(-span, span // 4 + 1, (rows, 1), generator=gen).float())
    x = (torch.randn((rows, cols), generator=gen) * mag).to(dtype).float()
    x[:64] = 0.0  # all-zero tensors: the eps clamp
    xg = x.to(DEV)
    s_gpu = torch.clamp(xg.abs().amax(dim=1, keepdim=True) / float(qmax), min=eps)
    q_gpu = torch.clamp(torch.round(xg / s_gpu), -qmax, qmax)
    s_or = linear_oracle.symmetric_scale(x, bits, dim=1)
    q_or = linear_oracle.quantize(x, s_or, bits)
    assert torch.equal(s_gpu.cpu().view(torch.int32), s_or.view(torch.int32))
    assert torch.equal(q_gpu.cpu().to(q_or.dtype), q_or)
    # float32 amax values on which a correctly rounded division differs from
    # the reciprocal product for some entries (so the check can tell them apart)
    a = (torch.rand((20_000, 1), generator=gen) + 1) * torch.exp2(
        torch.randint(-30, 30, (20_000, 1), generator=gen).float())
    s_or = linear_oracle.symmetric_scale(a, bits, dim=1)
    assert not torch.equal(torch.clamp(a / float(qmax), min=eps).view(torch.int32), s_or.view(torch.int32))
    s_gpu = torch.clamp(a.to(DEV) / float(qmax), min=eps)
    assert torch.equal(s_gpu.cpu().view(torch.int32), s_or.view(torch.int32))
    for i in range(200):
        t = xg[97 * i: 97 * i + 1 + i % 6].reshape(-1, cols if i % 2 else 8)
        s1 = torch.clamp(t.abs().amax(dim=None, keepdim=True) / float(qmax), min=eps)
        q1 = torch.clamp(torch.round(t / s1), -qmax, qmax)
        s1_or, = (linear_oracle.symmetric_scale(t.cpu(), bits),)
        assert torch.equal(s1.cpu().view(torch.int32), s1_or.view(torch.int32))
        assert torch.equal(q1.cpu().to(torch.int8 if bits == 8 else torch.int16),
                           linear_oracle.quantize(t.cpu(), s1_or, bits))


def test_quantize_symmetric_validation(backend):
    with pytest.raises(ValueError):
        backend.quantize_symmetric(torch.ones(4, 4, dtype=torch.int8, device=DEV))
    with pytest.raises(ValueError):
        backend.quantize_symmetric(torch.ones(4, 4, device=DEV), quant_bits=7)


@pytest.mark.parametrize("count", [37, 4096, 70_000])  # one-workgroup and two-launch forms
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_quantize_symmetric_non_finite(backend, count, dtype):
    """Non-finite activations: the scale is what the reference chain's float
    ops give (torch's amax propagates NaN, clamp keeps it; an infinity makes
    it +inf), and every element whose quotient is NaN quantizes to 0, so a
    dequantized output is all NaN, as the reference's is."""
    eps = torch.finfo(torch.float32).eps
    gen = torch.Generator().manual_seed(count)
    base = torch.randn(count, generator=gen).to(dtype)
    cases = {"nan": (float("nan"), None), "inf": (float("inf"), None), "-inf": (float("-inf"), None),
             "nan+inf": (float("nan"), float("inf"))}
    for name, (v0, v1) in cases.items():
        x = base.clone()
        x[count // 3] = v0
        if v1 is not None:
            x[count // 2] = v1
        xg = x.to(DEV)
        q, s = backend.quantize_symmetric(xg, 8)
        s_ref = torch.clamp(xg.float().abs().amax() / 127.0, min=eps)  # the reference's scale, on the GPU
        if name.startswith("nan"):
            assert torch.isnan(s).all() and torch.isnan(s_ref).all(), name
            assert int(q.abs().sum()) == 0, name  # every quotient is NaN
        else:
            assert torch.equal(s.reshape(-1).cpu(), s_ref.reshape(-1).cpu()) and torch.isinf(s).all(), name
            # finite / inf = 0; inf / inf = NaN -> 0
            assert int(q.abs().sum()) == 0, name
    # finite inputs are unchanged by the NaN handling
    q, s = backend.quantize_symmetric(base.to(DEV), 8)
    s_or = linear_oracle.symmetric_scale(base.float(), 8)
    assert torch.equal(s.reshape(-1).cpu().view(torch.int32), s_or.reshape(-1).view(torch.int32))
    assert torch.equal(q.cpu(), linear_oracle.quantize(base.float(), s_or, 8))


def test_rnslinear_nan_input_gives_nan_output(backend):
    # the reference: scale NaN -> every output int * NaN * s_w + b = NaN
    torch.manual_seed(6)
    lin = nn.Linear(64, 32, device=DEV).eval()
    layer = RNSLinear.from_linear(lin, backend=backend, mode="rns").eval()
    x = torch.randn(4, 64, device=DEV)
    x[1, 7] = float("nan")
    for _ in range(2):  # first call (unbound) and the bound one-call path
        assert torch.isnan(layer(x)).all()
    x[1, 7] = float("inf")
    assert torch.isnan(layer(x)).all()  # 0 * inf
