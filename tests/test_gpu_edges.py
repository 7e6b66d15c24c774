"""Empty inputs through every fused entry point: zero activation rows give
an empty [0, N] result of the right dtype without touching the weights, and
the quantizer's scale for an empty tensor is the reference's floor
(torch.finfo(float32).eps, rns_linear.py:154-158)."""
import pytest
import torch
from torch import nn

from rns_llm_amd import RNSLinear

pytestmark = pytest.mark.gpu

DEV = "cuda"
DENSE4 = (255, 253, 251, 247)


def test_fused_gemm_with_zero_rows(backend):
    w = torch.randint(-127, 128, (96, 256), device=DEV, dtype=torch.int8)
    prepared = backend.prepare_weight_nk(w, DENSE4)
    a = torch.empty((0, 256), device=DEV, dtype=torch.int8)
    out = backend.matmul_prepared_fused(a, prepared)
    assert out.shape == (0, 96) and out.dtype == torch.int64
    adaptive = backend.prepare_weight_adaptive_nk(w, DENSE4, min_channels=3)
    out = backend.matmul_prepared_adaptive_fused(a, adaptive)
    assert out.shape == (0, 96)
    f = torch.empty((0, 96), device=DEV, dtype=torch.float16)
    backend.matmul_prepared_fused(a, prepared, out=f, a_scale=torch.ones(1, device=DEV),
                                  w_scale=torch.ones(96, device=DEV))
    torch.cuda.synchronize()


def test_quantize_empty_gives_eps_scale(backend):
    q, scale = backend.quantize_symmetric(torch.empty((0, 64), device=DEV, dtype=torch.float16))
    torch.cuda.synchronize()
    assert q.shape == (0, 64) and q.dtype == torch.int8
    assert scale.item() == torch.finfo(torch.float32).eps


@pytest.mark.parametrize("shape", [(0, 128), (2, 0, 128)])
def test_rnslinear_zero_tokens(backend, shape):
    torch.manual_seed(9)
    lin = nn.Linear(128, 48, device=DEV, dtype=torch.float16).eval()
    layer = RNSLinear.from_linear(lin, backend=backend, mode="rns").eval()
    y = layer(torch.empty(shape, device=DEV, dtype=torch.float16))
    torch.cuda.synchronize()
    assert y.shape == shape[:-1] + (48,) and y.dtype == torch.float16
