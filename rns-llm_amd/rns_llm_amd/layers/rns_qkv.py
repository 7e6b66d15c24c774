"""Fused QKV projection for OPT-style attention on the RNS path.

Mirrors ``src/rns_llm/layers/rns_qkv.py:13-203`` of the reference: q, k and v
weights (and biases) concatenated along the output features in q, k, v order
into one ``RNSLinear`` (N = Nq + Nk + Nv), outputs split back as views; a
cache that serves HF OPT's three projection calls on the same hidden state
from one compute; an installer that swaps ``q_proj``/``k_proj``/``v_proj``
for weakly-referencing proxies so the combined parameters appear once in the
state dict.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Iterable

import torch
from torch import nn

from .rns_linear import RNSLinear


class RNSQKVProjection(nn.Module):
    """One combined projection; splitting gives exactly the three products
    because all three consume the same activation (and the same per-tensor
    activation scale), and weight scales are per output channel."""

    def __init__(self, combined: RNSLinear, split_sizes: tuple[int, int, int]) -> None:
        super().__init__()
        if sum(split_sizes) != combined.out_features:
            raise ValueError("split sizes do not match combined output size")
        self.combined = combined
        self.split_sizes = tuple(int(x) for x in split_sizes)
        self.compute_count = 0

    @classmethod
    def from_linears(cls, q_proj: nn.Linear, k_proj: nn.Linear, v_proj: nn.Linear, *,
                     backend=None, moduli: Iterable[int] | None = None,
                     moduli_strategy: str = "dense_coprime", mode: str = "rns",
                     quant_bits: int = 8, fused: bool = True, lut_channels: int = 2,
                     adaptive_channels: bool = False, adaptive_min_channels: int = 3,
                     fused_epilogue: bool = True) -> "RNSQKVProjection":
        layers = (q_proj, k_proj, v_proj)
        if any(not isinstance(layer, nn.Linear) for layer in layers):
            raise TypeError("q_proj, k_proj and v_proj must be nn.Linear")
        if len({layer.in_features for layer in layers}) != 1:
            raise ValueError("Q/K/V input sizes must match")
        if len({layer.weight.device for layer in layers}) != 1:
            raise ValueError("Q/K/V weights must share a device")
        if len({layer.weight.dtype for layer in layers}) != 1:
            raise ValueError("Q/K/V weights must share a dtype")
        if len({layer.bias is None for layer in layers}) != 1:
            raise ValueError("Q/K/V must consistently use or omit bias")
        split = tuple(layer.out_features for layer in layers)
        combined = RNSLinear(
            q_proj.in_features, sum(split), bias=q_proj.bias is not None, backend=backend,
            moduli=moduli, moduli_strategy=moduli_strategy, mode=mode, quant_bits=quant_bits,
            fused=fused, lut_channels=lut_channels, adaptive_channels=adaptive_channels,
            adaptive_min_channels=adaptive_min_channels, fused_epilogue=fused_epilogue,
        ).to(device=q_proj.weight.device, dtype=q_proj.weight.dtype)
        with torch.no_grad():
            combined.weight.copy_(torch.cat([layer.weight for layer in layers], dim=0))
            if combined.bias is not None:
                combined.bias.copy_(torch.cat([layer.bias for layer in layers], dim=0))
        return cls(combined, split)

    def forward(self, inputs: torch.Tensor):
        self.compute_count += 1
        q, k, v = torch.split(self.combined(inputs), self.split_sizes, dim=-1)
        return q, k, v


class _QKVSlice(nn.Module):
    """Stand-in for q_proj / k_proj / v_proj; holds only a weak reference to
    the coordinator so its parameters are registered once."""

    def __init__(self, coordinator: "CachedRNSQKV", index: int) -> None:
        super().__init__()
        object.__setattr__(self, "_coordinator_ref", weakref.ref(coordinator))
        self.index = int(index)

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        coordinator = self._coordinator_ref()
        if coordinator is None:
            raise RuntimeError("QKV coordinator has been destroyed")
        return coordinator.forward_slice(inputs, self.index)


class CachedRNSQKV(nn.Module):
    """Computes the fused projection once per logical attention call."""

    def __init__(self, projection: RNSQKVProjection) -> None:
        super().__init__()
        self.projection = projection
        self._cache_key = None
        self._cache_outputs = None
        self._served: set[int] = set()
        self.cache_hits = 0
        self.cache_misses = 0

    @staticmethod
    def _key(inputs: torch.Tensor):
        return (id(inputs), int(inputs.data_ptr()), int(inputs._version), tuple(inputs.shape),
                inputs.dtype, inputs.device)

    def clear_cache(self) -> None:
        self._cache_key = None
        self._cache_outputs = None
        self._served.clear()

    def forward_slice(self, inputs: torch.Tensor, index: int) -> torch.Tensor:
        if index not in (0, 1, 2):
            raise ValueError("QKV index must be 0, 1 or 2")
        key = self._key(inputs)
        # A slice index served twice means a new logical call: recompute.
        stale = self._cache_outputs is None or self._cache_key != key or index in self._served
        if stale:
            self._cache_outputs = self.projection(inputs)
            self._cache_key = key
            self._served = set()
            self.cache_misses += 1
        else:
            self.cache_hits += 1
        result = self._cache_outputs[index]
        self._served.add(index)
        if len(self._served) == 3:
            self.clear_cache()
        return result

    def slices(self):
        return _QKVSlice(self, 0), _QKVSlice(self, 1), _QKVSlice(self, 2)


@dataclass(frozen=True)
class InstalledQKVFusion:
    module_name: str
    coordinator: CachedRNSQKV


def install_opt_qkv_fusion(attention: nn.Module, *, backend, quant_bits: int = 8,
                           moduli_strategy: str = "dense_coprime", lut_channels: int = 2,
                           adaptive_channels: bool = False, adaptive_min_channels: int = 3,
                           fused_epilogue: bool = True) -> CachedRNSQKV:
    """Replace an OPT-style attention's q/k/v projections by one cached fused
    RNS projection (``rns_qkv.py:169-203``)."""
    for name in ("q_proj", "k_proj", "v_proj"):
        if not isinstance(getattr(attention, name, None), nn.Linear):
            raise TypeError(f"attention.{name} must be nn.Linear before fusion")
    projection = RNSQKVProjection.from_linears(
        attention.q_proj, attention.k_proj, attention.v_proj, backend=backend, mode="rns",
        quant_bits=quant_bits, moduli_strategy=moduli_strategy, lut_channels=lut_channels,
        adaptive_channels=adaptive_channels, adaptive_min_channels=adaptive_min_channels,
        fused_epilogue=fused_epilogue).eval()
    coordinator = CachedRNSQKV(projection).eval()
    attention.rns_qkv = coordinator
    attention.q_proj, attention.k_proj, attention.v_proj = coordinator.slices()
    return coordinator


def replace_opt_attention_blocks(model: nn.Module, *, backend, blocks: int, quant_bits: int = 8,
                                 include_out_proj: bool = True, adaptive_channels: bool = False,
                                 fused_epilogue: bool = True):
    """Fused RNS QKV (and, optionally, an RNS ``out_proj``) in the first
    ``blocks`` attention modules of an OPT-style model, in module order
    (``scripts/evaluate_ppl.py:53-94``): every module whose ``q_proj``,
    ``k_proj`` and ``v_proj`` are ``nn.Linear`` is a candidate.  Returns the
    replaced module names and the QKV coordinators."""
    if blocks < 0:
        raise ValueError("blocks must be non-negative")
    candidates = [(name, module) for name, module in model.named_modules()
                  if all(isinstance(getattr(module, attr, None), nn.Linear)
                         for attr in ("q_proj", "k_proj", "v_proj"))]
    replaced: list[str] = []
    coordinators: list[CachedRNSQKV] = []
    for name, attention in candidates[:blocks]:
        coordinators.append(install_opt_qkv_fusion(
            attention, backend=backend, quant_bits=quant_bits, moduli_strategy="dense_coprime",
            lut_channels=2, adaptive_channels=adaptive_channels, fused_epilogue=fused_epilogue))
        replaced.append(f"{name}.qkv_fused")
        if include_out_proj:
            if not isinstance(getattr(attention, "out_proj", None), nn.Linear):
                raise TypeError(f"{name}.out_proj is not nn.Linear")
            attention.out_proj = RNSLinear.from_linear(
                attention.out_proj, backend=backend, mode="rns", quant_bits=quant_bits, fused=True,
                lut_channels=2, moduli_strategy="dense_coprime",
                adaptive_channels=adaptive_channels, fused_epilogue=fused_epilogue).eval()
            replaced.append(f"{name}.out_proj")
    return replaced, coordinators
