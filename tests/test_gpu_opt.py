"""a random-init OPT-125m-architecture decoder (fp16),
batch 8 x 512 tokens, with fused RNS QKV and an RNS out_proj in its first 4
attention blocks (``scripts/evaluate_ppl.py:53-94, 204-217`` of the
reference).  Checks the backend call counts per forward (with the
reference's guard that the RNS path actually ran), every replaced layer's
output against the CPU float chain of RNSLinear bit for bit (on a sample
of rows of each layer's real input inside the model), and reports the
logit error against the fp16 model."""
import pytest
import torch

from oracle import linear_oracle
from rns_llm_amd import RNSLinear, replace_opt_attention_blocks

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")

DEV = "cuda"


def build_opt(seed: int) -> torch.nn.Module:
    config = transformers.OPTConfig()  # opt-125m: 12 layers, hidden 768, 12 heads, FFN 3072
    config._attn_implementation = "sdpa"
    torch.manual_seed(seed)
    return transformers.OPTForCausalLM(config).to(device=DEV, dtype=torch.float16).eval()


@torch.no_grad()
def test_opt_c4_blocks_counts_layers_and_logit_error(backend):
    model = build_opt(11)
    gen = torch.Generator().manual_seed(12)
    ids = torch.randint(0, model.config.vocab_size, (8, 512), generator=gen).to(DEV)
    ref = model(ids).logits.float()
    replaced, coordinators = replace_opt_attention_blocks(model, backend=backend, blocks=4)
    assert len(replaced) == 8 and len(coordinators) == 4
    assert all(name.endswith(("qkv_fused", "out_proj")) for name in replaced)
    seen = []

    def record(module, args, output):
        seen.append((module, args[0].detach().cpu(), output.detach().cpu()))

    hooks = [m.register_forward_hook(record) for m in model.modules() if isinstance(m, RNSLinear)]
    for forward in range(2):
        backend.reset_stats()
        seen.clear()
        out = model(ids).logits.float()
        stats = backend.stats_snapshot()
        # the reference refuses to report when the RNS path did not run
        # (evaluate_ppl.py:212-217); here: 4 fused QKV + 4 out_proj GEMMs, and
        # the weights are prepared (encoded) on the first forward
        assert stats.get("fused_gemm_calls", 0) == 8
        assert stats["fused_gemm_channels_4"] == 8
        assert stats["encode_centered_calls"] == (16 if forward == 0 else 8)
        assert all(c.projection.compute_count == forward + 1 for c in coordinators)
        assert len(seen) == 8 and torch.isfinite(out).all()
        err = (out - ref).abs()
        scale = ref.abs().mean().item()
        print(f"forward {forward}: logit max err {err.max().item():.4g}, mean err "
              f"{err.mean().item():.4g}, mean |logit| {scale:.4g}")
        assert err.mean().item() < 0.05 * scale
    for h in hooks:
        h.remove()
    # each replaced layer against RNSLinear's float chain on the CPU, on its
    # own input from the second forward (per-tensor scale from all 4096 rows)
    rows = torch.linspace(0, 8 * 512 - 1, 48).long()
    for module, x, y in seen:
        want, _ = linear_oracle.linear_forward(x, module.weight.detach().cpu(), module.bias.detach().cpu(),
                                               rows=rows)
        assert torch.equal(y.reshape(-1, module.out_features)[rows], want)
