"""HIP-graph capture of the fused paths.

Each path is captured once and the graph replayed several times on new
inputs copied into its static buffers, with eager calls and
synchronisations between the replays; every replay must equal the eager
call and the exact product (or the CPU float chain) bit for bit.  The
library records only kernel launches (no memset nodes), and the adaptive
prefix is chosen on the device, so one graph serves every prefix."""
import pytest
import torch
from torch import nn

from oracle import linear_oracle
from rns_llm_amd import RNSLinear

pytestmark = pytest.mark.gpu

DEV = "cuda"
DENSE4 = (255, 253, 251, 247)


def exact(a, w):
    """A @ W^T in float64: every partial sum of int8 products here is an
    integer below 2^53, so the result is exact whatever the summation order."""
    return a.double() @ w.double().t()


def capture(fn):
    """Warm up on a side stream, then capture fn() in a graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        result = fn()
    return graph, result


# (m, k, n): the stream kernel (decode), the MFMA kernel (C2 headline shape),
# the LDS-staged kernel (256 full-round tiles), and K split over workgroups
# (stream and MFMA: their arrival counters must return to zero every replay)
@pytest.mark.parametrize("m,k,n", [(1, 768, 2304), (256, 768, 2304), (1024, 1024, 4096),
                                   (1, 8192, 768), (256, 8192, 256)])
def test_graph_replays_fused_gemm(backend, m, k, n):
    gen = torch.Generator(device=DEV).manual_seed(m + k)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
    prepared = backend.prepare_weight_nk(w, DENSE4)
    a = torch.randint(-127, 128, (m, k), generator=gen, device=DEV, dtype=torch.int8)
    ws = backend.create_workspace(device=a.device, channels=4, m=m, n=n, k=k)
    graph, out = capture(lambda: backend.matmul_prepared_fused(a, prepared, workspace=ws))
    for _ in range(4):
        a.copy_(torch.randint(-127, 128, (m, k), generator=gen, device=DEV, dtype=torch.int8))
        eager = backend.matmul_prepared_fused(a, prepared).clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(out.double(), exact(a, w))


def test_graph_replays_adaptive_prefix(backend):
    """Small activations need 3 channels, all-127 ones the full 4 (bound
    4096 * 127 * 127 = 66,064,384 > the 3-channel half-capacity): the
    device picks the prefix inside the same graph on every replay."""
    m, k, n = 64, 4096, 512
    gen = torch.Generator(device=DEV).manual_seed(11)
    w = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
    w[0, 0] = 127  # max|B| = 127
    prepared = backend.prepare_weight_adaptive_nk(w, DENSE4, min_channels=3)
    a = torch.zeros((m, k), device=DEV, dtype=torch.int8)
    ws = {4: backend.create_workspace(device=a.device, channels=4, m=m, n=n, k=k)}
    graph, (out, meta) = capture(lambda: backend.matmul_prepared_adaptive_fused(
        a, prepared, workspace_by_channels=ws, return_metadata=True))
    for kind, channels in (("small", 3), ("adversarial", 4), ("small", 3), ("adversarial", 4)):
        if kind == "small":
            a.copy_(torch.randint(-3, 4, (m, k), generator=gen, device=DEV, dtype=torch.int8))
        else:
            sign = torch.randint(0, 2, (m, k), generator=gen, device=DEV, dtype=torch.int8) * 2 - 1
            a.copy_(sign * 127)
        eager = backend.matmul_prepared_fused(a, prepared.variants[4]).clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert int(meta.device_tensor[0].item()) == channels
        assert not meta.overflow
        assert torch.equal(out, eager)
        assert torch.equal(out.double(), exact(a, w))


@pytest.mark.parametrize("tokens", [1, 256])
def test_graph_replays_rnslinear_forward(backend, tokens):
    """Quantization (two launches) + GEMM with the fused dequant epilogue."""
    torch.manual_seed(23)
    lin = nn.Linear(768, 2304, bias=True, device=DEV, dtype=torch.float16).eval()
    layer = RNSLinear.from_linear(lin, backend=backend, mode="rns").eval()
    gen = torch.Generator().manual_seed(tokens)
    x = torch.randn(tokens, 768, generator=gen).to(DEV, torch.float16)
    with torch.no_grad():
        layer(x)  # prepares and caches the weight before capture
        graph, y = capture(lambda: layer(x))
        for rep in range(3):
            x.copy_((torch.randn(tokens, 768, generator=gen) * (1 + rep)).to(DEV, torch.float16))
            eager = layer(x).clone()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, eager)
            want, _ = linear_oracle.linear_forward(x.cpu(), lin.weight.cpu(), lin.bias.cpu())
            assert torch.equal(y.cpu(), want)
