"""rnsmx_matmul_prepared_fused_noalloc (static scratch, no allocation) against
rnsmx_matmul_prepared_fused (caller workspace) through the C ABI: two calls
in a row, the second with a smaller input, each bit-identical to the
workspace entry point and to the exact product; a call whose scratch need
exceeds the static maximum is rejected before any launch."""
import ctypes

import pytest
import torch

from rns_llm_amd import _native
from rns_llm_amd.backends.hip_backend import _stream_handle

pytestmark = pytest.mark.gpu

DEV = "cuda"
DENSE4 = (255, 253, 251, 247)


def noalloc_call(backend, a, prepared, out, plan=None):
    consts = backend._constants(a.device, prepared.moduli)
    m, k = int(a.shape[0]), int(a.shape[1])
    return backend._lib.rnsmx_matmul_prepared_fused_noalloc(
        a.data_ptr(), _native.dtype_code(a.dtype), m, k, prepared.n, prepared.packed.data_ptr(),
        consts.native_ref, consts.compact_lut.data_ptr(), 2, None, None,
        None if plan is None else ctypes.byref(_native.make_plan(plan)), out.data_ptr(),
        _stream_handle(a.device))


def test_noalloc_matches_workspace_entry_on_two_calls(backend):
    gen = torch.Generator(device=DEV).manual_seed(77)
    # first: long K, few tiles (the automatic plan splits K 8 ways: counters
    # and exchange area in the static scratch); second: smaller, int16
    # activations (residue planes in the scratch), ragged shape
    cases = [(256, 8192, 256, torch.int8, 127), (5, 200, 37, torch.int16, 127)]
    for m, k, n, dtype, amax in cases:
        w = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
        a = torch.randint(-amax, amax + 1, (m, k), generator=gen, device=DEV, dtype=torch.int32).to(dtype)
        prepared = backend.prepare_weight_nk(w, DENSE4)
        want = backend.matmul_prepared_fused(a, prepared).clone()
        out = torch.full((m, n), -1, dtype=torch.int64, device=DEV)
        _native.check(noalloc_call(backend, a, prepared, out))
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        assert torch.equal(out.double(), a.double() @ w.double().t())


def test_noalloc_drops_a_split_that_does_not_fit(backend):
    # M=640 on the C5 projection with int8 activations: the automatic plan is
    # the 256 x 64 LDS kernel's tail split (576 tiles, the last 64 split in
    # 4), whose exchange area alone is 16 MiB; unsplit the call needs a few
    # KB, so the no-allocation entry point runs it unsplit
    m, k, n = 640, 4096, 12288
    auto = _native.Plan()
    _native.check(backend._lib.rnsmx_gemm_plan(m, n, k, 4, 1, ctypes.byref(auto)))
    need_auto = backend._lib.rnsmx_prepared_workspace_bytes(m, k, n, 4, None)
    gen = torch.Generator(device=DEV).manual_seed(91)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
    a = torch.randint(-127, 128, (m, k), generator=gen, device=DEV, dtype=torch.int8)
    prepared = backend.prepare_weight_nk(w, DENSE4)
    want = backend.matmul_prepared_fused(a, prepared).clone()
    for mm in (m, 300):  # the second call smaller
        out = torch.full((mm, n), -1, dtype=torch.int64, device=DEV)
        _native.check(noalloc_call(backend, a[:mm].contiguous(), prepared, out))
        torch.cuda.synchronize()
        assert torch.equal(out, want[:mm])
    # the case is the one described: the automatic plan splits and needs more
    # than the static scratch
    assert auto.splits > 1 and need_auto > 16 << 20
    rows = torch.arange(0, m, 37, device=DEV)
    exact = a[rows].double() @ w.double().t()
    assert torch.equal(want[rows].double(), exact)


def test_noalloc_residue_planes_drop_the_split(backend):
    # int16 activations, 6 channels, C5 M=512: the automatic plan is the
    # residue-plane LDS kernel with its tail split, whose exchange (two words
    # per element) does not fit the static scratch next to the 12 MiB of
    # activation planes; the no-allocation entry point runs it unsplit
    m, k, n = 512, 4096, 12288
    mods = (255, 253, 251, 247, 241, 239)
    auto = _native.Plan()
    _native.check(backend._lib.rnsmx_gemm_plan(m, n, k, 6, 0, ctypes.byref(auto)))
    assert auto.as_tuple() == (8, 0, 0, 0, 2, 1)
    assert backend._lib.rnsmx_prepared_workspace_bytes(m, k, n, 6, None) > 16 << 20
    gen = torch.Generator(device=DEV).manual_seed(512)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
    a = torch.randint(-3000, 3001, (m, k), generator=gen, device=DEV, dtype=torch.int32).to(torch.int16)
    prepared = backend.prepare_weight_nk(w, mods)
    want = backend.matmul_prepared_fused(a, prepared).clone()
    for mm in (m, 200):  # the second call smaller
        out = torch.full((mm, n), -1, dtype=torch.int64, device=DEV)
        _native.check(noalloc_call(backend, a[:mm].contiguous(), prepared, out))
        torch.cuda.synchronize()
        assert torch.equal(out, want[:mm])
    rows = torch.arange(0, m, 29, device=DEV)
    assert torch.equal(want[rows].double(), a[rows].double() @ w.double().t())


def test_noalloc_rejects_oversize_without_launch(backend):
    # int16 activations need R * M * kp bytes of residue planes: 4 * 8192 *
    # 1024 = 32 MiB > 16 MiB
    m, k, n = 8192, 1024, 16
    w = torch.ones((n, k), dtype=torch.int8, device=DEV)
    prepared = backend.prepare_weight_nk(w, DENSE4)
    a = torch.ones((m, k), dtype=torch.int16, device=DEV)
    out = torch.zeros((m, n), dtype=torch.int64, device=DEV)
    rc = noalloc_call(backend, a, prepared, out)
    assert rc == _native.ESPACE
    assert b"static scratch" in backend._lib.rnsmx_last_error()
    torch.cuda.synchronize()
    assert int(out.abs().sum()) == 0
