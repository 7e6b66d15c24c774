"""Inference-only ``RNSLinear`` for the HIP backend.

Same constructor arguments, buffers, caches and forward semantics as the
reference's ``src/rns_llm/layers/rns_linear.py:17-275``:

  * per-output-channel symmetric weight quantization, cached on
    ``weight._version`` (``:168-204``);
  * per-tensor symmetric activation quantization (``:154-166, 238-241``);
  * workspaces keyed by ``(rows, channels, stream)`` so concurrent streams
    never share scratch (``:206-223``);
  * output ``int * s_a * s_w[n] + bias`` cast to the input dtype
    (``:272-275``).

With the HIP backend the dequantization runs inside the GEMM epilogue
(``fused_epilogue=True``, the default): the same float32 operations in the
same order, each rounded to nearest even, so the result is bit-identical to
the torch chain while saving its five elementwise launches.  The whole
device part of a forward (activation quantization, GEMM, epilogue) is then
one call into the library (``bind_linear``), bound once per prepared
weight.  Any other backend object with the reference contract is driven
exactly as the reference drives it.
"""
from __future__ import annotations

from typing import Iterable

import torch
from torch import nn
from torch.nn import functional as F

from ..moduli import choose_moduli_for_dot, validate_moduli

_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_FLOAT_OUT = (torch.float32, torch.float16, torch.bfloat16)


def _current_stream_handle(device: torch.device) -> int:
    """Identity of the current stream on `device` (the workspace cache key):
    ATen's raw accessor when present, it is ~20x cheaper than
    torch.cuda.current_stream()."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return int(_raw_stream(index))
    return int(torch.cuda.current_stream(device).cuda_stream)

class RNSLinear(nn.Module):
    def __init__(self, in_features: int, out_features: int, *, bias: bool = True, backend=None,
                 moduli: Iterable[int] | None = None, moduli_strategy: str = "dense_coprime",
                 mode: str = "torch", kernel: str = "auto", quant_bits: int = 8,
                 fused: bool = True, lut_channels: int = 2, adaptive_channels: bool = False,
                 adaptive_min_channels: int = 3, fused_epilogue: bool = True,
                 packed_weights: bool = False) -> None:
        super().__init__()
        if quant_bits not in (8, 12, 16):
            raise ValueError("quant_bits must be 8, 12 or 16")
        if lut_channels not in (0, 1, 2):
            raise ValueError("lut_channels must be 0, 1 or 2")
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.backend = backend
        self.mode = mode
        self.kernel = kernel
        self.quant_bits = int(quant_bits)
        self.fused = bool(fused)
        self.lut_channels = int(lut_channels)
        self.moduli_strategy = moduli_strategy
        self.adaptive_channels = bool(adaptive_channels)
        self.adaptive_min_channels = int(adaptive_min_channels)
        self.fused_epilogue = bool(fused_epilogue)

        qmax = self.quant_max
        chosen = tuple(moduli) if moduli is not None else choose_moduli_for_dot(
            self.in_features, qmax, qmax, strategy=moduli_strategy)
        self.moduli = validate_moduli(chosen)
        # packed_weights (no counterpart in the reference): keep the quantized
        # weight as 2 bytes per value instead of one byte per channel
        self.packed_weights = bool(packed_weights)
        if self.packed_weights and len(self.moduli) > 6:
            raise ValueError("packed weights take at most 6 channels")

        self.weight = nn.Parameter(torch.empty(out_features, in_features))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features))
        else:
            self.register_parameter("bias", None)
        self.register_buffer("_weight_scale", torch.empty(0), persistent=False)
        self.register_buffer("_weight_residues", torch.empty(0, dtype=torch.int8),
                             persistent=False)
        self._prepared_weight_version: int | None = None
        self._prepared_weight = None
        self._adaptive_prepared_weight = None
        self._workspace_by_rows: dict[tuple[int, int, int], object] = {}
        self.last_adaptive_metadata = None
        self._linear_call = None
        self._linear_key = None
        self._linear_scratch: dict[tuple[int, int], torch.Tensor] = {}
        self.reset_parameters()

    @property
    def quant_max(self) -> int:
        return (1 << (self.quant_bits - 1)) - 1

    @property
    def quant_dtype(self) -> torch.dtype:
        return torch.int8 if self.quant_bits == 8 else torch.int16

    def reset_parameters(self) -> None:
        # Same initialisers and generator consumption as nn.Linear and the
        # reference (rns_linear.py:100-105).
        nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)
        if self.bias is not None:
            bound = 1 / self.in_features ** 0.5
            nn.init.uniform_(self.bias, -bound, bound)
        self.clear_weight_cache()

    def clear_weight_cache(self) -> None:
        self._weight_scale = torch.empty(0, device=self.weight.device)
        self._weight_residues = torch.empty(0, dtype=torch.int8, device=self.weight.device)
        self._prepared_weight_version = None
        self._prepared_weight = None
        self._adaptive_prepared_weight = None
        self._workspace_by_rows = {}
        self.last_adaptive_metadata = None
        self._linear_call = None
        self._linear_key = None
        self._linear_scratch = {}

    @classmethod
    def from_linear(cls, layer: nn.Linear, *, backend=None, moduli=None,
                    moduli_strategy: str = "dense_coprime", mode: str = "torch",
                    kernel: str = "auto", quant_bits: int = 8, fused: bool = True,
                    lut_channels: int = 2, adaptive_channels: bool = False,
                    adaptive_min_channels: int = 3, fused_epilogue: bool = True,
                    packed_weights: bool = False) -> "RNSLinear":
        result = cls(layer.in_features, layer.out_features, bias=layer.bias is not None,
                     backend=backend, moduli=moduli, moduli_strategy=moduli_strategy, mode=mode,
                     kernel=kernel, quant_bits=quant_bits, fused=fused,
                     lut_channels=lut_channels, adaptive_channels=adaptive_channels,
                     adaptive_min_channels=adaptive_min_channels,
                     fused_epilogue=fused_epilogue,
                     packed_weights=packed_weights).to(device=layer.weight.device,
                                                       dtype=layer.weight.dtype)
        result.weight.data.copy_(layer.weight.data)
        if layer.bias is not None and result.bias is not None:
            result.bias.data.copy_(layer.bias.data)
        return result

    def _symmetric_scale(self, values: torch.Tensor, dim=None) -> torch.Tensor:
        max_abs = values.detach().abs().amax(dim=dim, keepdim=True)
        return torch.clamp(max_abs / float(self.quant_max), min=torch.finfo(torch.float32).eps)

    def _quantize(self, values: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        return torch.clamp(torch.round(values / scale), -self.quant_max,
                           self.quant_max).to(self.quant_dtype)

    def _bias_float(self):
        """float32 copy of the bias for the fused epilogue, cached per bias
        version (one conversion per weight update, not per call)."""
        if self.bias is None:
            return None
        key = (self.bias.data_ptr(), self.bias._version, self.bias.dtype)
        if getattr(self, "_bias_key", None) != key:
            self._bias_f32 = self.bias.detach().float().contiguous()
            self._bias_key = key
        return self._bias_f32

    def prepare_weight(self) -> None:
        """Quantizes and encodes the weight when its version changed
        (rns_linear.py:168-204); a no-op otherwise.  The version check runs
        on every forward, so it stays outside the no-grad context, which
        costs a few microseconds to enter."""
        if self.backend is None:
            raise RuntimeError("RNSLinear requires a backend in mode='rns'")
        if not self.weight.is_cuda:
            raise RuntimeError("RNSLinear expects GPU weights in mode='rns'")
        if self._prepared_weight_version == self.weight._version and self._prepared_weight is not None:
            return
        self._prepare_weight_now()

    @torch.no_grad()
    def _prepare_weight_now(self) -> None:
        version = self.weight._version
        w = self.weight.float()
        scale = self._symmetric_scale(w, dim=1)
        quantized = self._quantize(w, scale)  # [N, K]
        native_nk = hasattr(self.backend, "prepare_weight_nk")
        if self.packed_weights and not hasattr(self.backend, "prepare_weight_packed_nk"):
            raise ValueError("this backend has no packed weights")
        adaptive_prepared = None
        if self.adaptive_channels and self.packed_weights:
            adaptive_prepared = self.backend.prepare_weight_adaptive_nk(
                quantized.contiguous(), self.moduli, min_channels=self.adaptive_min_channels, packed=True)
            prepared = adaptive_prepared.variants[len(self.moduli)]
        elif self.packed_weights:
            prepared = self.backend.prepare_weight_packed_nk(quantized.contiguous(), self.moduli)
        elif self.adaptive_channels:
            if native_nk:
                adaptive_prepared = self.backend.prepare_weight_adaptive_nk(
                    quantized.contiguous(), self.moduli, min_channels=self.adaptive_min_channels)
            else:
                adaptive_prepared = self.backend.prepare_weight_adaptive(
                    quantized.transpose(0, 1).contiguous(), self.moduli,
                    min_channels=self.adaptive_min_channels)
            prepared = adaptive_prepared.variants[len(self.moduli)]
        elif native_nk:
            prepared = self.backend.prepare_weight_nk(quantized.contiguous(), self.moduli)
        else:
            prepared = self.backend.prepare_weight(quantized.transpose(0, 1).contiguous(),
                                                   self.moduli)
        self._weight_scale = scale.squeeze(1).to(self.weight.device).contiguous()
        self._weight_residues = prepared.packed
        self._prepared_weight = prepared
        self._adaptive_prepared_weight = adaptive_prepared
        self._prepared_weight_version = version
        self._workspace_by_rows = {}
        self._linear_call = None
        self._linear_key = None

    def _live_key(self):
        """What the bound one-call forward depends on: the weight version, the
        identity of the bias values (their float32 copy is bound) and the
        switches that choose the path (a change re-binds or unbinds it)."""
        bias = self.bias
        return (self.weight._version,
                None if bias is None else (bias.data_ptr(), bias._version, bias.dtype),
                self.fused, self.fused_epilogue, self.adaptive_channels)

    def _bind_linear(self):
        """The backend's one-call forward for the current weight and bias
        (None when the backend has none, or cannot serve this layer).  The
        weight must be prepared."""
        key = self._live_key()
        if key != self._linear_key:
            self._linear_call = None
            bind = getattr(self.backend, "bind_linear", None)
            if bind is not None and self.fused and self.fused_epilogue:
                self._linear_call = bind(self._prepared_weight, self._weight_scale, self._bias_float(),
                                         self.quant_bits,
                                         self._adaptive_prepared_weight if self.adaptive_channels else None)
            self._linear_key = key
            self._linear_scratch = {}
        return self._linear_call

    def _workspace(self, rows: int, channels: int | None = None):
        channels = len(self.moduli) if channels is None else int(channels)
        key = (int(rows), channels, _current_stream_handle(self.weight.device))
        cached = self._workspace_by_rows.get(key)
        if cached is None:
            kwargs = dict(device=self.weight.device, channels=channels, m=rows,
                          n=self.out_features)
            if hasattr(self.backend, "prepare_weight_nk"):
                kwargs["k"] = self.in_features
            cached = self.backend.create_workspace(**kwargs)
            self._workspace_by_rows[key] = cached
        return cached

    def _supports_fused(self) -> bool:
        probe = getattr(self.backend, "supports_fused", None)
        if probe is not None:
            return bool(probe(self._prepared_weight))
        return self._prepared_weight.kernel == "cublas"

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        call = self._linear_call
        if (call is not None and self.mode == "rns" and not self.training and inputs.is_cuda
                and inputs.dtype in _FLOAT_OUT and inputs.dim() > 0
                and inputs.shape[-1] == self.in_features and self._linear_key == self._live_key()):
            # prepared weight, unchanged since the call was bound: one library
            # call (quantize, GEMM, dequant epilogue) into a fresh output
            x = inputs if inputs.is_contiguous() else inputs.contiguous()
            rows = x.numel() // self.in_features
            key = (rows, _current_stream_handle(x.device))
            scratch = self._linear_scratch.get(key)
            if scratch is None:
                scratch = self.backend.create_linear_scratch(call, rows, x.device)
                self._linear_scratch[key] = scratch
            out = torch.empty(inputs.shape[:-1] + (self.out_features,), dtype=inputs.dtype, device=x.device)
            metadata = call(x, rows, out, scratch)
            if metadata is not None:
                self.last_adaptive_metadata = metadata
            return out
        if self.mode == "torch":
            return F.linear(inputs, self.weight, self.bias)
        if self.mode != "rns":
            raise ValueError(f"unknown mode: {self.mode}")
        if self.training:
            raise RuntimeError("RNSLinear is inference-only; call eval()")
        if self.backend is None:
            raise RuntimeError("RNSLinear mode='rns' requires a backend")

        if inputs.dim() == 0 or inputs.shape[-1] != self.in_features:
            # the reference's flatten-and-restore fails on such inputs (its
            # final reshape to (*inputs.shape[:-1], out_features) cannot hold
            # the product's rows); here it fails before anything is computed
            raise RuntimeError(
                f"RNSLinear expects inputs of shape (*, {self.in_features}), got {tuple(inputs.shape)}")
        self.prepare_weight()
        original_shape = inputs.shape[:-1]
        flat = inputs.reshape(-1, self.in_features)
        if inputs.dtype in _FLOAT_OUT and inputs.is_cuda:
            if self._bind_linear() is not None:
                return self.forward(inputs)  # the bound path above
        if (hasattr(self.backend, "quantize_symmetric") and flat.is_cuda
                and flat.dtype in (torch.float32, torch.float16, torch.bfloat16)):
            # the same scale and integers as the torch chain below, in two launches
            quantized_a, activation_scale = self.backend.quantize_symmetric(
                flat, self.quant_bits)
        else:
            flat = flat.float().contiguous()
            activation_scale = self._symmetric_scale(flat)
            quantized_a = self._quantize(flat, activation_scale).contiguous()
        rows = flat.shape[0]

        fused_epi = (self.fused_epilogue and hasattr(self.backend, "prepare_weight_nk")
                     and inputs.dtype in (torch.float32, torch.float16, torch.bfloat16))
        if fused_epi and (self.adaptive_channels or (self.fused and self._supports_fused())):
            out = torch.empty((rows, self.out_features), dtype=inputs.dtype, device=inputs.device)
            bias = self._bias_float()
            epi = dict(out=out, a_scale=activation_scale.reshape(1), w_scale=self._weight_scale,
                       bias=bias)
            if self.adaptive_channels:
                adaptive = self._adaptive_prepared_weight
                device_safe = getattr(adaptive, "device_selection_is_safe", None)
                if device_safe is not None and device_safe(quantized_a.dtype):
                    # the prefix is chosen on the device: the full set's workspace serves all
                    workspaces = {len(self.moduli): self._workspace(rows)}
                else:
                    workspaces = {c: self._workspace(rows, c) for c in adaptive.variants}
                _, metadata = self.backend.matmul_prepared_adaptive_fused(
                    quantized_a, adaptive, lut_channels=self.lut_channels,
                    workspace_by_channels=workspaces, return_metadata=True, **epi)
                self.last_adaptive_metadata = metadata
            else:
                self.backend.matmul_prepared_fused(
                    quantized_a, self._prepared_weight, lut_channels=self.lut_channels,
                    workspace=self._workspace(rows), **epi)
            return out.reshape(*original_shape, self.out_features)

        if self.adaptive_channels:
            workspaces = {c: self._workspace(rows, c)
                          for c in self._adaptive_prepared_weight.variants}
            integer_result, metadata = self.backend.matmul_prepared_adaptive_fused(
                quantized_a, self._adaptive_prepared_weight, lut_channels=self.lut_channels,
                workspace_by_channels=workspaces, return_metadata=True)
            self.last_adaptive_metadata = metadata
            integer_result = integer_result.float()
        elif self.fused and self._supports_fused():
            integer_result = self.backend.matmul_prepared_fused(
                quantized_a, self._prepared_weight, lut_channels=self.lut_channels,
                workspace=self._workspace(rows)).float()
        else:
            integer_result = self.backend.matmul_prepared(
                quantized_a, self._prepared_weight, kernel=self.kernel).float()
        output = integer_result * activation_scale * self._weight_scale.unsqueeze(0)
        if self.bias is not None:
            output = output + self.bias.float()
        return output.reshape(*original_shape, self.out_features).to(inputs.dtype)
