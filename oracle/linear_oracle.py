"""CPU oracle for the float chain around the integer core of ``RNSLinear``.

TEST INFRASTRUCTURE ONLY (see ``oracle/rns_oracle.py``).

Restates ``src/rns_llm/layers/rns_linear.py`` of the reference op by op on the
CPU with torch float32 tensors, so the same IEEE operations run as on the GPU:

  * ``_symmetric_scale`` (``rns_linear.py:154-159``): amax(|v|) / 127,
    clamped below at float32 eps; per tensor for activations, per output
    channel (dim=1) for weights; the division by the Python float 127.0 is
    restated with the GPU rounding (see ``symmetric_scale``);
  * ``_quantize`` (``:161-166``): round-half-to-even(v / s) clamped to
    +-quant_max, cast to int8 (int16 for 12/16-bit);
  * weight preparation (``:183-185``): B = quantized(W).T, contiguous;
  * forward (``:238-275``): int64 result -> float32, then ``* s_a``, then
    ``* s_w[None, :]``, then ``+ bias``, then cast to the input dtype.

The integer product is the exact int64 matmul, which every RNS backend must
reproduce bit for bit.  Pinned by tests/test_oracle.py against hand-computed
float32 values and against ``torch.nn.functional.linear`` within quantization
error bounds.
"""
from __future__ import annotations

import numpy as np
import torch


def quant_max(bits: int) -> int:
    return (1 << (bits - 1)) - 1


def symmetric_scale(values: torch.Tensor, bits: int = 8, dim=None) -> torch.Tensor:
    """amax(|v|) / quant_max, clamped at float32 eps, with the rounding of
    the device the reference runs this on.  ``RNSLinear`` requires GPU
    weights (``rns_linear.py:172-173``), and on the GPU torch evaluates
    ``tensor / python_float`` as ``tensor * fl32(1 / python_float)`` (ATen's
    true-divide kernel multiplies by the reciprocal of a CPU scalar), which
    differs in the last bit from a correctly rounded division for about 4%
    of inputs; the CPU ``/`` divides.  The GPU form is restated here."""
    amax = values.detach().abs().amax(dim=dim, keepdim=True)
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(float(quant_max(bits)),
                                                                dtype=torch.float32)
    return torch.clamp(amax * inv, min=torch.finfo(torch.float32).eps)


def quantize(values: torch.Tensor, scale: torch.Tensor, bits: int = 8) -> torch.Tensor:
    q = quant_max(bits)
    dtype = torch.int8 if bits == 8 else torch.int16
    return torch.clamp(torch.round(values / scale), -q, q).to(dtype)


def prepare_weight(weight: torch.Tensor, bits: int = 8):
    """(B [K, N] int, per-output-channel scale [N] f32)."""
    w = weight.detach().float().cpu()
    scale = symmetric_scale(w, bits, dim=1)
    b = quantize(w, scale, bits).transpose(0, 1).contiguous()
    return b, scale.squeeze(1)


def quantize_activations(inputs: torch.Tensor, in_features: int, bits: int = 8):
    """(A [M, K] int, per-tensor scale [1, 1] f32)."""
    flat = inputs.detach().cpu().reshape(-1, in_features).float().contiguous()
    scale = symmetric_scale(flat, bits)
    return quantize(flat, scale, bits).contiguous(), scale


def linear_forward(inputs: torch.Tensor, weight: torch.Tensor, bias, bits: int = 8, rows=None):
    """Full rns-mode ``RNSLinear.forward`` on the CPU; returns (output, int64
    integer product).  With ``rows`` (indices into the flattened [M, K]
    input) the activation scale still comes from the whole input (it is per
    tensor), but only those rows are multiplied and returned, as [len(rows),
    N], so large layers can be checked on a sample of their rows."""
    out_features, in_features = weight.shape
    b, w_scale = prepare_weight(weight, bits)
    a, a_scale = quantize_activations(inputs, in_features, bits)
    if rows is not None:
        a = a[torch.as_tensor(rows, dtype=torch.long)]
    integer = torch.from_numpy(a.numpy().astype(np.int64) @ b.numpy().astype(np.int64))
    out = integer.float() * a_scale * w_scale.unsqueeze(0)
    if bias is not None:
        out = out + bias.detach().cpu().float()
    shape = (integer.shape[0], out_features) if rows is not None else tuple(inputs.shape[:-1]) + (out_features,)
    return out.reshape(shape).to(inputs.dtype), integer
