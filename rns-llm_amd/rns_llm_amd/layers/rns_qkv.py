"""Fused q/k/v projection on the RNS path, and its use in OPT-style attention.

Contract kept from the reference (``src/rns_llm/layers/rns_qkv.py:13-203``):
the public classes and installer, their constructor arguments, the q, k, v
order of the concatenated output features, ``compute_count`` /
``cache_hits`` / ``cache_misses``, the per-call cache key
``(id, data_ptr, _version, shape, dtype, device)`` of the hidden state, and
the rule that a projection index asked for a second time starts a new
logical call.  Exception types are the reference's; texts are this
package's own.

Why one product suffices: q, k and v read the same hidden state, so
stacking their weights along the output features gives one GEMM whose
output columns are the three projections side by side.  ``RNSLinear``
quantizes activations per tensor (one scale shared by all columns) and
weights per output row, so every column of the stacked product is
bit-identical to the column of the separate projection.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Iterable

import torch
from torch import nn

from .rns_linear import RNSLinear

_PROJECTIONS = ("q_proj", "k_proj", "v_proj")


def _common(values, what: str):
    """The single value shared by every element of `values`, or ValueError."""
    distinct = set(values)
    if len(distinct) != 1:
        raise ValueError(f"q, k and v projections disagree on {what}: {sorted(map(str, distinct))}")
    return distinct.pop()


class RNSQKVProjection(nn.Module):
    """One ``RNSLinear`` over the stacked q, k and v weights; ``forward``
    returns the three column blocks as views of its output."""

    def __init__(self, combined: RNSLinear, split_sizes: tuple[int, int, int]) -> None:
        super().__init__()
        sizes = tuple(int(s) for s in split_sizes)
        if len(sizes) != 3 or sum(sizes) != combined.out_features:
            raise ValueError(f"split sizes {sizes} do not cover the {combined.out_features} output features")
        self.combined = combined
        self.split_sizes = sizes
        self.compute_count = 0

    @classmethod
    def from_linears(cls, q_proj: nn.Linear, k_proj: nn.Linear, v_proj: nn.Linear, *,
                     backend=None, moduli: Iterable[int] | None = None,
                     moduli_strategy: str = "dense_coprime", mode: str = "rns",
                     quant_bits: int = 8, fused: bool = True, lut_channels: int = 2,
                     adaptive_channels: bool = False, adaptive_min_channels: int = 3,
                     fused_epilogue: bool = True) -> "RNSQKVProjection":
        parts = (q_proj, k_proj, v_proj)
        for name, layer in zip(_PROJECTIONS, parts):
            if not isinstance(layer, nn.Linear):
                raise TypeError(f"{name} is a {type(layer).__name__}, not an nn.Linear")
        in_features = _common((p.in_features for p in parts), "input size")
        device = _common((p.weight.device for p in parts), "device")
        dtype = _common((p.weight.dtype for p in parts), "dtype")
        has_bias = _common((p.bias is not None for p in parts), "bias presence")
        sizes = tuple(p.out_features for p in parts)
        stacked = RNSLinear(in_features, sum(sizes), bias=has_bias, backend=backend, moduli=moduli,
                            moduli_strategy=moduli_strategy, mode=mode, quant_bits=quant_bits,
                            fused=fused, lut_channels=lut_channels,
                            adaptive_channels=adaptive_channels,
                            adaptive_min_channels=adaptive_min_channels,
                            fused_epilogue=fused_epilogue).to(device=device, dtype=dtype)
        with torch.no_grad():
            offset = 0
            for p, rows in zip(parts, sizes):
                stacked.weight[offset:offset + rows].copy_(p.weight)
                if has_bias:
                    stacked.bias[offset:offset + rows].copy_(p.bias)
                offset += rows
        return cls(stacked, sizes)

    def forward(self, inputs: torch.Tensor):
        self.compute_count += 1
        return tuple(self.combined(inputs).split(self.split_sizes, dim=-1))


@dataclass
class _Served:
    """Outputs of one logical attention call and the indices not yet handed out."""

    key: tuple
    outputs: tuple
    pending: set


class CachedRNSQKV(nn.Module):
    """Serves an attention module's three projection calls on one hidden
    state from a single fused product."""

    def __init__(self, projection: RNSQKVProjection) -> None:
        super().__init__()
        self.projection = projection
        self._current: _Served | None = None
        self.cache_hits = 0
        self.cache_misses = 0

    @staticmethod
    def _key(inputs: torch.Tensor):
        # the identity of a hidden state within one attention call
        return (id(inputs), int(inputs.data_ptr()), int(inputs._version), tuple(inputs.shape),
                inputs.dtype, inputs.device)

    def clear_cache(self) -> None:
        self._current = None

    def forward_slice(self, inputs: torch.Tensor, index: int) -> torch.Tensor:
        if index not in (0, 1, 2):
            raise ValueError(f"projection index {index!r} is not 0 (q), 1 (k) or 2 (v)")
        key = self._key(inputs)
        current = self._current
        # reuse only within one logical call: same hidden state and an index
        # not handed out yet; anything else starts the next call
        if current is not None and current.key == key and index in current.pending:
            self.cache_hits += 1
        else:
            current = _Served(key, self.projection(inputs), {0, 1, 2})
            self._current = current
            self.cache_misses += 1
        current.pending.discard(index)
        result = current.outputs[index]
        if not current.pending:
            self._current = None  # do not keep the hidden state alive past the call
        return result

    def slices(self):
        return tuple(_QKVSlice(self, i) for i in range(3))


class _QKVSlice(nn.Module):
    """Stands in for one of q_proj / k_proj / v_proj.  It refers to the
    coordinator weakly (a plain attribute, which nn.Module does not register),
    so the fused parameters belong to the coordinator alone in state_dict."""

    def __init__(self, coordinator: CachedRNSQKV, index: int) -> None:
        super().__init__()
        self._owner = weakref.ref(coordinator)
        self.index = int(index)

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        owner = self._owner()
        if owner is None:
            raise RuntimeError(f"{_PROJECTIONS[self.index]} outlived its fused QKV module")
        return owner.forward_slice(inputs, self.index)


@dataclass(frozen=True)
class InstalledQKVFusion:
    module_name: str
    coordinator: CachedRNSQKV


def install_opt_qkv_fusion(attention: nn.Module, *, backend, quant_bits: int = 8,
                           moduli_strategy: str = "dense_coprime", lut_channels: int = 2,
                           adaptive_channels: bool = False, adaptive_min_channels: int = 3,
                           fused_epilogue: bool = True) -> CachedRNSQKV:
    """Swap an OPT-style attention module's q/k/v projections for one cached
    fused RNS projection; the coordinator is registered as
    ``attention.rns_qkv`` (``rns_qkv.py:169-203``)."""
    linears = [getattr(attention, name, None) for name in _PROJECTIONS]
    missing = [name for name, layer in zip(_PROJECTIONS, linears) if not isinstance(layer, nn.Linear)]
    if missing:
        raise TypeError(f"cannot fuse: {', '.join(missing)} of {type(attention).__name__} "
                        "must be nn.Linear")
    fused = RNSQKVProjection.from_linears(
        *linears, backend=backend, mode="rns", quant_bits=quant_bits,
        moduli_strategy=moduli_strategy, lut_channels=lut_channels,
        adaptive_channels=adaptive_channels, adaptive_min_channels=adaptive_min_channels,
        fused_epilogue=fused_epilogue).eval()
    coordinator = CachedRNSQKV(fused).eval()
    attention.rns_qkv = coordinator
    for name, proxy in zip(_PROJECTIONS, coordinator.slices()):
        setattr(attention, name, proxy)
    return coordinator


def replace_opt_attention_blocks(model: nn.Module, *, backend, blocks: int, quant_bits: int = 8,
                                 include_out_proj: bool = True, adaptive_channels: bool = False,
                                 fused_epilogue: bool = True):
    """Config-4 integration: the first ``blocks`` attention modules (in
    ``named_modules`` order, any module with nn.Linear q/k/v projections)
    get a fused RNS QKV and, with ``include_out_proj``, an RNS out_proj, all
    with the dense coprime moduli and lut_channels=2, as the reference's
    PPL script does (``scripts/evaluate_ppl.py:53-94``).  Returns the names
    of the replaced parts and the QKV coordinators."""
    if blocks < 0:
        raise ValueError("blocks must be >= 0")
    attentions = [(name, module) for name, module in model.named_modules()
                  if all(isinstance(getattr(module, p, None), nn.Linear) for p in _PROJECTIONS)]
    replaced: list[str] = []
    coordinators: list[CachedRNSQKV] = []
    options = dict(backend=backend, quant_bits=quant_bits, adaptive_channels=adaptive_channels,
                   fused_epilogue=fused_epilogue)
    for name, attention in attentions[:blocks]:
        out_proj = getattr(attention, "out_proj", None) if include_out_proj else None
        if include_out_proj and not isinstance(out_proj, nn.Linear):
            raise TypeError(f"cannot replace {name}.out_proj: it is a {type(out_proj).__name__}")
        coordinators.append(install_opt_qkv_fusion(attention, moduli_strategy="dense_coprime",
                                                   lut_channels=2, **options))
        replaced.append(f"{name}.qkv_fused")
        if include_out_proj:
            attention.out_proj = RNSLinear.from_linear(out_proj, mode="rns", fused=True, lut_channels=2,
                                                       moduli_strategy="dense_coprime", **options).eval()
            replaced.append(f"{name}.out_proj")
    return replaced, coordinators
