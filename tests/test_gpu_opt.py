"""a random-init OPT-125m-architecture decoder (fp16) with
fused RNS QKV and an RNS out_proj in its first 4 attention blocks
(``scripts/evaluate_ppl.py:53-94, 204-217`` of the reference).  Checks the
backend call counts per forward and reports the logit error against the
fp16 model; the replaced blocks' integer cores are pinned bit-exact by the
layer tests, so here the error only has to stay at int8 quantization level."""
import pytest
import torch

from rns_llm_amd import replace_opt_attention_blocks

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")

DEV = "cuda"


def build_opt(seed: int) -> torch.nn.Module:
    config = transformers.OPTConfig()  # opt-125m: 12 layers, hidden 768, 12 heads, FFN 3072
    config._attn_implementation = "sdpa"
    torch.manual_seed(seed)
    return transformers.OPTForCausalLM(config).to(device=DEV, dtype=torch.float16).eval()


@torch.no_grad()
def test_opt_c4_blocks_counts_and_logit_error(backend):
    model = build_opt(11)
    gen = torch.Generator().manual_seed(12)
    ids = torch.randint(0, model.config.vocab_size, (2, 128), generator=gen).to(DEV)
    ref = model(ids).logits.float()
    replaced, coordinators = replace_opt_attention_blocks(model, backend=backend, blocks=4)
    assert len(replaced) == 8 and len(coordinators) == 4
    assert all(name.endswith(("qkv_fused", "out_proj")) for name in replaced)
    for forward in range(2):
        backend.reset_stats()
        out = model(ids).logits.float()
        stats = backend.stats_snapshot()
        # 4 fused QKV + 4 out_proj GEMMs; weights are prepared on the first forward
        assert stats["fused_gemm_calls"] == 8
        assert stats["encode_centered_calls"] == (16 if forward == 0 else 8)
        assert all(c.projection.compute_count == forward + 1 for c in coordinators)
        assert torch.isfinite(out).all()
        err = (out - ref).abs()
        scale = ref.abs().mean().item()
        print(f"forward {forward}: logit max err {err.max().item():.4g}, mean err "
              f"{err.mean().item():.4g}, mean |logit| {scale:.4g}")
        assert err.mean().item() < 0.05 * scale
