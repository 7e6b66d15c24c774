"""Maximum-size edge case: int8 activations past 4 GB (2^20 rows x 4096).

The LDS-staged kernel addresses A rows through 32-bit per-lane offsets, so
the kernel choice must route such a call to a kernel with 64-bit row
addressing; rows at both ends of A must come out exact."""
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
DENSE4 = (255, 253, 251, 247)


def test_activations_beyond_4gb(backend):
    m, k, n = 1 << 20, 4096, 64
    gen = torch.Generator(device=DEV).manual_seed(5)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
    prepared = backend.prepare_weight_nk(w, DENSE4)
    a = torch.randint(-127, 128, (m, k), generator=gen, device=DEV, dtype=torch.int8)
    assert a.numel() >= 1 << 32
    out = backend.matmul_prepared_fused(a, prepared)
    torch.cuda.synchronize()
    for rows in (slice(0, 512), slice(m // 2 - 256, m // 2 + 256), slice(m - 512, m)):
        want = a[rows].double() @ w.double().t()  # exact: integer sums below 2^53
        assert torch.equal(out[rows].double(), want), rows
    del a, out
    torch.cuda.empty_cache()
