"""HIP / gfx950 implementation of the reference's RNS backend contract.

``HipRNSBackend`` implements the method contract of the reference's
``CudaRNSBackend`` (``src/rns_llm/backends/cuda_backend.py:110-799``) under its
own name: same method names, keyword arguments, return values, aliasing of
workspace outputs, stats counters and exception types.  Every device
computation goes through ``librnsmx.so`` (``include/rnsmx.h``); there is no
host or torch fallback for the integer path.

Deliberate deviations (each keeps results bit-identical):
  * prepared weights are stored fragment-major ``[R, N/16, kp/64, 1024]``
    (``packed``, the MFMA operand layout); the public ``residues`` field is
    the reference-shaped ``[R, K, N]`` tensor, unpacked on first access;
  * ``kernel`` names are ``"mfma"``; ``RNSLinear`` asks ``supports_fused`` instead
    of comparing the kernel string with ``"cublas"``;
  * the workspace's ``accumulators`` tensor is byte scratch sized by the
    library (the fused kernel has no int32 round trip);
  * ``matmul_prepared_adaptive_fused`` selects the channel prefix on the
    device whenever the weight's preparation proved that even the worst
    activation of the call's dtype fits the full moduli set (the usual case:
    the set was chosen for that range); its metadata is then a lazy mapping
    read from the device, and the per-prefix counters are taken when it is
    read.  Otherwise it takes the reference's synchronous selection and
    raises ``OverflowError`` before computing, as the reference does.
"""
from __future__ import annotations

import ctypes
import functools
import itertools
from collections import Counter
from collections.abc import Mapping
from dataclasses import dataclass, field
from math import prod
from typing import Iterable, Sequence

import torch

from .. import _native
from ..moduli import (
    centered_accumulator_bound,
    minimal_prefix_channels,
    safe_l1_dot_bound,
    validate_moduli,
)

KERNEL_NAME = "mfma"


@dataclass
class _DeviceConstants:
    moduli: torch.Tensor          # int32 [R] on the device
    compact_lut: torch.Tensor     # int16 [R, 4, 256] on the device
    modulus_product: int
    native: _native.Moduli        # rnsmx_moduli_t (kernel-argument constants)
    native_ref: object            # ctypes.byref(native), built once


@dataclass(frozen=True)
class PreparedRNSWeight:
    """Weight prepared once for the fused GEMM.

    ``packed`` is the storage the kernels read, fragment-major
    ``[P, ceil(N/16), kp/64, 1024]``: the 1 KB fragment of column block ``jb``
    and K step ``ks`` holds, at byte ``16*l``, column ``16*jb + l % 16`` and K
    bytes ``64*ks + 16*(l // 16)`` .. ``+16`` (zero past N and K).  With
    ``form == "planes"`` the P = R planes are the centered residues of every
    channel; with ``form == "packed"`` (int8/int16 weights, 2 bytes per value
    whatever R) the two planes are ``hi = v >> 8`` and ``lo = (v & 255) -
    128`` and the kernels form each channel's residue from them.
    ``residues`` is the reference-shaped ``[R, K, N]`` tensor, unpacked on
    first access.
    """

    moduli: tuple[int, ...]
    k: int
    n: int
    kernel: str
    packed: torch.Tensor
    absmax: torch.Tensor | None = None  # int32 [1], max |B| on the device
    form: str = "planes"

    def _unpack(self, planes: torch.Tensor) -> torch.Tensor:
        p, n16, nk, _ = planes.shape
        grid = planes.view(p, n16, nk, 4, 16, 16).permute(0, 2, 3, 5, 1, 4)
        return grid.reshape(p, nk * 64, n16 * 16)[:, :self.k, :self.n]

    @functools.cached_property
    def values(self) -> torch.Tensor:
        """The weight as int32 [K, N] (packed form only)."""
        if self.form != "packed":
            raise ValueError("values are kept only by packed weights")
        hi, lo = self._unpack(self.packed).to(torch.int32)
        return hi * 256 + lo + 128

    @functools.cached_property
    def residues(self) -> torch.Tensor:
        if self.form == "packed":
            mods = torch.tensor(self.moduli, dtype=torch.int32, device=self.packed.device).view(-1, 1, 1)
            r = torch.remainder(self.values.unsqueeze(0), mods)
            return torch.where(r > mods // 2, r - mods, r).to(torch.int8)
        return self._unpack(self.packed)

    @property
    def kp(self) -> int:
        return int(self.packed.shape[2]) * _native.K_ALIGN

    @property
    def nbytes(self) -> int:
        """Bytes of weight storage the kernels read."""
        return int(self.packed.numel())


@dataclass
class RNSWorkspace:
    """Reusable memory for one (rows, channels, stream) of one layer."""

    accumulators: torch.Tensor  # uint8 scratch for the library
    output: torch.Tensor        # [M, N] int64
    channels: int
    m: int
    n: int


class PreparedAdaptiveRNSWeight:
    """One encoded weight with every safe prefix variant (views, no copies).

    ``max_abs_weight`` is read from the device once, at preparation (the
    reference reads it there too, ``cuda_backend.py:569``)."""

    def __init__(self, variants: dict, full_moduli: tuple[int, ...],
                 absmax: torch.Tensor, min_channels: int):
        self.variants = variants
        self.full_moduli = full_moduli
        self.absmax = absmax
        self.min_channels = min_channels
        self.max_abs_weight = int(absmax.item())
        self.full_capacity = (prod(full_moduli) - 1) // 2

    def device_selection_is_safe(self, a_dtype: torch.dtype) -> bool:
        """Whether no activation of this dtype can overflow the full set:
        K * max|a| * max|B| <= (P - 1) / 2, i.e. 2 * bound < P for the
        largest bound any input could have.  Then the device-side selection
        always finds a prefix and no call can wrap."""
        amax = _DTYPE_MAX_ABS.get(a_dtype)
        k = self.variants[len(self.full_moduli)].k
        return amax is not None and k * amax * self.max_abs_weight <= self.full_capacity


@dataclass
class RNSRequestBatchWorkspace:
    """Preallocated activation buffer plus fused GEMM workspace."""

    activations: torch.Tensor
    fused: RNSWorkspace
    rows_per_request: tuple[int, ...]
    k: int


_DTYPE_MAX_ABS = {torch.int8: 128, torch.int16: 1 << 15, torch.int32: 1 << 31}


class AdaptiveMetadata(Mapping):
    """``{"channels", "bound", "capacity"}`` of one device-selected adaptive
    call, read lazily from the device.  Reading it synchronises with the
    stream and, once, adds the call to the backend's per-prefix counters
    ``adaptive_channels_{c}`` and ``fused_gemm_channels_{c}`` (the prefix is
    known only on the device until then).  The device path is taken only
    when overflow is impossible; should the device still flag one, reading
    raises ``OverflowError`` like ``minimal_prefix_channels``."""

    _KEYS = ("channels", "bound", "capacity")

    def __init__(self, meta: torch.Tensor, full_moduli: tuple[int, ...], stats: Counter | None = None):
        self.device_tensor = meta
        self._full = full_moduli
        self._stats = stats
        self._host: dict | None = None

    def _load(self) -> dict:
        if self._host is None:
            channels, bound, capacity, overflow = (int(v) for v in self.device_tensor.tolist())
            if overflow:
                raise OverflowError(
                    f"full moduli set cannot represent bound {bound}; capacity={capacity}")
            self._host = {"channels": channels, "bound": bound, "capacity": capacity}
            if self._stats is not None:
                self._stats[f"adaptive_channels_{channels}"] += 1
                self._stats[f"fused_gemm_channels_{channels}"] += 1
        return self._host

    @property
    def overflow(self) -> bool:
        return bool(int(self.device_tensor[3].item()))

    def __getitem__(self, key):
        return self._load()[key]

    def __iter__(self):
        return iter(self._KEYS)

    def __len__(self):
        return len(self._KEYS)

    def __repr__(self):
        return f"AdaptiveMetadata({self._host if self._host is not None else '<on device>'})"


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_FLOAT_CODES = {torch.float32: _native.FLOAT32, torch.float16: _native.FLOAT16,
                torch.bfloat16: _native.BFLOAT16}


def _stream_handle(device: torch.device) -> int:
    """The current stream of `device` as a raw handle: ATen's accessor
    (~0.1 us) when this torch build has it, else the public path (~2 us per
    call, a measurable share of an eager GEMM call)."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def _aligned(t: torch.Tensor) -> torch.Tensor:
    return t if t.data_ptr() % 16 == 0 else t.clone()


class LinearCall:
    """``RNSLinear.forward``'s device work bound to one prepared weight: one
    ``rnsmx_linear_forward`` call per forward (activation quantization, then
    the GEMM with the dequant epilogue), with every per-weight argument
    resolved once here instead of on each call.  Counts the backend stats
    the reference's forward counts (one activation encode, one fused GEMM)."""

    def __init__(self, backend: "HipRNSBackend", prepared: "PreparedRNSWeight", w_scale: torch.Tensor,
                 bias: torch.Tensor | None, quant_bits: int, adaptive: "PreparedAdaptiveRNSWeight | None"):
        device = prepared.packed.device
        consts = backend._constants(device, prepared.moduli)
        self._fn = backend._lib.rnsmx_linear_forward
        self._bytes_fn = backend._lib.rnsmx_linear_workspace_bytes
        self._keep = (prepared, w_scale, bias, consts, adaptive)  # the pointers below stay valid
        self._packed = prepared.packed.data_ptr()
        self._mods = consts.native_ref
        self._w_scale = w_scale.data_ptr()
        self._bias = None if bias is None else bias.data_ptr()
        self.k, self.n, self.bits = prepared.k, prepared.n, int(quant_bits)
        self.channels = len(prepared.moduli)
        self._index = device.index if device.index is not None else torch.cuda.current_device()
        self._adaptive = adaptive
        self._full_moduli = prepared.moduli
        self._stats = backend._stats
        self._gemm_key = f"fused_gemm_channels_{self.channels}"
        self._ws_bytes: dict[int, int] = {}

    def workspace_bytes(self, rows: int) -> int:
        nbytes = self._ws_bytes.get(rows)
        if nbytes is None:
            nbytes = int(self._bytes_fn(rows, self.k, self.n, self.channels, self.bits))
            if nbytes < 0:
                raise ValueError("bad linear shape")
            self._ws_bytes[rows] = nbytes
        return nbytes

    def __call__(self, x: torch.Tensor, rows: int, out: torch.Tensor, scratch: torch.Tensor):
        """x: contiguous float activations holding [rows, K]; out: contiguous,
        of x's dtype, holding [rows, N]; scratch: zero-initialised uint8 of
        workspace_bytes(rows).  Returns the adaptive metadata when the layer
        is adaptive, else None."""
        meta = adaptive = None
        if self._adaptive is not None:
            meta = torch.empty((4,), dtype=torch.int64, device=x.device)
            adaptive = ctypes.byref(_native.Adaptive(self._adaptive.min_channels,
                                                     self._adaptive.absmax.data_ptr(), meta.data_ptr()))
        rc = self._fn(x.data_ptr(), _FLOAT_CODES[x.dtype], rows, self.k, self.n, self.bits, self._packed,
                      self._mods, self._w_scale, self._bias, adaptive, scratch.data_ptr(), scratch.numel(),
                      out.data_ptr(), _raw_stream(self._index) if _raw_stream is not None
                      else torch.cuda.current_stream().cuda_stream)
        if rc:
            _native.check(rc)
        stats = self._stats
        stats["encode_centered_calls"] += 1
        stats["encode_centered_values"] += rows * self.k
        stats["fused_gemm_calls"] += 1
        if meta is None:
            stats[self._gemm_key] += 1
            return None
        stats["adaptive_selections"] += 1
        return AdaptiveMetadata(meta, self._full_moduli, stats)


class HipRNSBackend:
    """RNS backend on MI355X: one MFMA GEMM launch for all residue channels
    with the modular reduction, Garner reconstruction and signed correction
    in its epilogue."""

    name = "hip-rns-mfma"

    def __init__(self) -> None:
        if not torch.cuda.is_available():
            raise RuntimeError("no GPU is visible to this PyTorch (ROCm) installation")
        self._lib = _native.lib()
        self._device_cache: dict[tuple[int, tuple[int, ...]], _DeviceConstants] = {}
        self._quant_scratch: dict[tuple[int, int], torch.Tensor] = {}
        self._ws_bytes: dict[tuple[int, int, int], int] = {}
        self._stats: Counter[str] = Counter()

    # ------------------------------------------------------------------
    # Stats (cuda_backend.py:129-135)
    # ------------------------------------------------------------------
    def reset_stats(self) -> None:
        self._stats.clear()

    def stats_snapshot(self) -> dict[str, int]:
        return dict(self._stats)

    # ------------------------------------------------------------------
    # Constants (cuda_backend.py:137-166)
    # ------------------------------------------------------------------
    def _constants(self, device: torch.device, moduli: Iterable[int]) -> _DeviceConstants:
        mods = tuple(moduli)
        index = device.index if device.index is not None else torch.cuda.current_device()
        key = (index, mods)
        cached = self._device_cache.get(key)
        if cached is not None:
            return cached
        mods = validate_moduli(mods)
        if prod(mods) > 2**63 - 1:
            raise OverflowError("moduli product must fit signed int64")
        native = _native.make_moduli(mods)
        lut_host = torch.empty((len(mods), 4, 256), dtype=torch.int16)
        _native.check(self._lib.rnsmx_compact_lut(ctypes.byref(native), lut_host.data_ptr()))
        dev = torch.device("cuda", index)
        cached = _DeviceConstants(
            moduli=torch.tensor(mods, dtype=torch.int32, device=dev),
            compact_lut=lut_host.to(dev),
            modulus_product=prod(mods),
            native=native,
            native_ref=ctypes.byref(native),
        )
        self._device_cache[key] = cached
        return cached

    @staticmethod
    def _validate_matrix(matrix: torch.Tensor, name: str, ndim: int) -> None:
        """The layout every native entry point reads: a dense row-major
        device tensor of the expected rank."""
        problems = [text for bad, text in ((not matrix.is_cuda, "on the GPU"),
                                           (matrix.ndim != ndim, f"{ndim}-dimensional"),
                                           (not matrix.is_contiguous(), "contiguous"))
                    if bad]
        if problems:
            raise ValueError(f"{name} ({tuple(matrix.shape)}, {matrix.device}) must be "
                             + " and ".join(problems))

    # ------------------------------------------------------------------
    # Encoding (cuda_backend.py:188-200)
    # ------------------------------------------------------------------
    def encode_centered(self, values: torch.Tensor, moduli: Iterable[int]) -> torch.Tensor:
        """Encode int8/int16/int32 values as signed-int8 centered residues
        ``[R, *values.shape]``."""
        self._validate_matrix(values, "values", values.ndim)
        if values.dtype not in (torch.int8, torch.int16, torch.int32):
            raise ValueError("centered encoder supports int8, int16 and int32")
        consts = self._constants(values.device, moduli)
        self._stats["encode_centered_calls"] += 1
        self._stats["encode_centered_values"] += int(values.numel())
        r = len(consts.moduli)
        out = torch.empty((r,) + tuple(values.shape), dtype=torch.int8, device=values.device)
        n = int(values.numel())
        if n == 0:
            return out
        src = _aligned(values)
        _native.check(self._lib.rnsmx_encode_centered(
            src.data_ptr(), _native.dtype_code(values.dtype), 1, n, n, consts.native_ref,
            out.data_ptr(), None, None, _stream_handle(values.device)))
        return out

    # ------------------------------------------------------------------
    # Activation quantization (RNSLinear._symmetric_scale / _quantize,
    # rns_linear.py:154-166 of the reference)
    # ------------------------------------------------------------------
    def quantize_symmetric(self, values: torch.Tensor, quant_bits: int = 8):
        """Per-tensor symmetric quantization of float activations in two
        launches: ``(q, scale)`` with ``scale = max(amax|v| / qmax, eps)``
        ([1, 1] float32, the division rounded as the GPU reference rounds
        ``tensor / python_float``) and ``q = clamp(round(v / scale), ±qmax)``
        (int8 for 8 bits, int16 for 12 or 16), ``q`` shaped like ``values``.
        Bit-identical to the reference's torch chain for finite inputs."""
        if values.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise ValueError("quantize_symmetric expects float32, float16 or bfloat16 values")
        if not values.is_cuda:
            raise ValueError("values must be on a GPU")
        if quant_bits not in (8, 12, 16):
            raise ValueError("quant_bits must be 8, 12 or 16")
        x = values.contiguous()
        device = x.device
        q = torch.empty(x.shape, dtype=torch.int8 if quant_bits == 8 else torch.int16, device=device)
        scale = torch.empty((1, 1), dtype=torch.float32, device=device)
        stream = _stream_handle(device)
        index = device.index if device.index is not None else torch.cuda.current_device()
        scratch = self._quant_scratch.get((index, stream))
        if scratch is None:
            # per-block maxima passed between the two launches of one call
            scratch = torch.empty((_native.QUANT_SCRATCH,), dtype=torch.int32, device=device)
            self._quant_scratch[(index, stream)] = scratch
        _native.check(self._lib.rnsmx_quantize_symmetric(
            x.data_ptr(), _native.dtype_code(x.dtype), int(x.numel()), int(quant_bits),
            scratch.data_ptr(), scale.data_ptr(), q.data_ptr(), stream))
        return q, scale

    # ------------------------------------------------------------------
    # Bounds and selection (cuda_backend.py:205-261)
    # ------------------------------------------------------------------
    @staticmethod
    def accumulator_bound(k: int, moduli: Iterable[int]) -> int:
        mods = validate_moduli(moduli)
        return int(k) * (max(mods) - 1) ** 2

    @staticmethod
    def centered_accumulator_bound(k: int, moduli: Iterable[int]) -> int:
        return centered_accumulator_bound(k, moduli)

    def mfma_compatible(self, *, k: int, n: int, moduli: Iterable[int],
                        device: torch.device) -> bool:
        """The MFMA path takes any K and N (no multiple-of-4 rule) for 2..10
        channels whose int32 accumulators cannot overflow."""
        del n, device
        mods = validate_moduli(moduli)
        return (2 <= len(mods) <= _native.MAX_CHANNELS
                and self.centered_accumulator_bound(k, mods) <= 0x7FFFFFFF)

    def select_centered_kernel(self, *, k: int, n: int, moduli: Iterable[int],
                               requested: str = "auto", device: torch.device) -> str:
        if requested not in ("auto", KERNEL_NAME):
            raise ValueError(f"unknown kernel {requested!r}; this backend provides 'mfma'")
        if not self.mfma_compatible(k=k, n=n, moduli=moduli, device=device):
            raise ValueError("MFMA path constraints are not satisfied "
                             "(2..10 channels, K * max(floor(m/2))^2 < 2^31)")
        return KERNEL_NAME

    @staticmethod
    def supports_fused(prepared) -> bool:
        return getattr(prepared, "packed", None) is not None

    def bind_linear(self, prepared: PreparedRNSWeight, w_scale: torch.Tensor, bias: torch.Tensor | None,
                    quant_bits: int, adaptive: PreparedAdaptiveRNSWeight | None = None) -> LinearCall | None:
        """A ``LinearCall`` for ``RNSLinear.forward`` on this prepared weight
        (float32 ``w_scale`` [N] and ``bias`` [N] or None), or None when the
        one-call path cannot serve it: an adaptive weight whose device-side
        selection is not proven safe takes the synchronous selection, and a
        packed weight takes the quantize + packed GEMM calls."""
        if prepared.form != "planes":
            return None
        if adaptive is not None and not adaptive.device_selection_is_safe(
                torch.int8 if quant_bits == 8 else torch.int16):
            return None
        for name, t in (("w_scale", w_scale), ("bias", bias)):
            if t is not None and (t.dtype != torch.float32 or t.numel() != prepared.n
                                  or not t.is_contiguous() or t.device != prepared.packed.device):
                raise ValueError(f"{name} must be a contiguous float32 [N] tensor on the weight's device")
        return LinearCall(self, prepared, w_scale, bias, quant_bits, adaptive)

    def create_linear_scratch(self, call: LinearCall, rows: int, device: torch.device) -> torch.Tensor:
        """Zero-filled scratch for ``call`` at ``rows`` rows (the library's
        K-split counters at its start must be zero at first use)."""
        return torch.zeros((call.workspace_bytes(rows),), dtype=torch.uint8, device=device)

    # ------------------------------------------------------------------
    # Workspaces (cuda_backend.py:366-396)
    # ------------------------------------------------------------------
    def create_workspace(self, *, device: torch.device, channels: int, m: int, n: int,
                         k: int | None = None) -> RNSWorkspace:
        # zero-filled: the library's K-split arrival counters at its start
        # must be zero at first use (every call leaves them zero)
        scratch_bytes = _native.SPLIT_TICKETS * 4
        if k is not None:
            scratch_bytes = self._prepared_workspace_bytes(m, k, n, channels, None)
        return RNSWorkspace(
            accumulators=torch.zeros((max(scratch_bytes, 0),), dtype=torch.uint8, device=device),
            output=torch.empty((m, n), dtype=torch.int64, device=device),
            channels=channels,
            m=m,
            n=n,
        )

    @staticmethod
    def _check_workspace(workspace: RNSWorkspace, *, channels: int, m: int, n: int,
                         device: torch.device) -> None:
        """A workspace serves exactly the (channels, M, N) it was made for,
        on one device (``cuda_backend.py:385-396``)."""
        made_for = (workspace.channels, workspace.m, workspace.n)
        if made_for != (channels, m, n):
            raise ValueError(f"workspace made for (channels, M, N) = {made_for}, "
                             f"used for {(channels, m, n)}")
        devices = {workspace.accumulators.device, workspace.output.device}
        if devices != {device}:
            raise ValueError(f"workspace on {sorted(map(str, devices))}, operands on {device}")

    def _prepared_workspace_bytes(self, m: int, k: int, n: int, channels: int, plan) -> int:
        key = (m, k, n, channels, None if plan is None else plan.as_tuple())
        nbytes = self._ws_bytes.get(key)
        if nbytes is None:
            nbytes = int(self._lib.rnsmx_prepared_workspace_bytes(
                m, k, n, channels, None if plan is None else ctypes.byref(plan)))
            if nbytes < 0:
                raise ValueError("bad workspace shape")
            self._ws_bytes[key] = nbytes
        return nbytes

    def _packed_workspace_bytes(self, m: int, k: int, n: int, channels: int, plan) -> int:
        key = ("packed", m, k, n, channels, None if plan is None else plan.as_tuple())
        nbytes = self._ws_bytes.get(key)
        if nbytes is None:
            nbytes = int(self._lib.rnsmx_packed_workspace_bytes(
                m, k, n, channels, None if plan is None else ctypes.byref(plan)))
            if nbytes < 0:
                if plan is not None:  # the call itself reports why the plan does not fit
                    return self._packed_workspace_bytes(m, k, n, channels, None)
                raise ValueError("bad workspace shape")
            self._ws_bytes[key] = nbytes
        return nbytes

    @staticmethod
    def _scratch(workspace: RNSWorkspace, nbytes: int) -> torch.Tensor:
        if nbytes < 0:
            raise ValueError("bad workspace size")
        if workspace.accumulators.numel() < nbytes:
            # zero-filled for the arrival counters (see create_workspace)
            workspace.accumulators = torch.zeros(
                (nbytes,), dtype=torch.uint8, device=workspace.output.device)
        return workspace.accumulators

    # ------------------------------------------------------------------
    # Fused ops
    # ------------------------------------------------------------------
    def _residue_operands(self, a_residues: torch.Tensor, b_residues: torch.Tensor,
                          moduli: Iterable[int]) -> tuple[tuple[int, ...], int, int, int, int]:
        """Checks a pair of centered residue planes a [R, M, K], b [R, K, N]
        against each other and the moduli; returns (moduli, R, M, K, N)."""
        for name, planes in (("a_residues", a_residues), ("b_residues", b_residues)):
            self._validate_matrix(planes, name, 3)
            if planes.dtype != torch.int8:
                raise ValueError(f"{name} must hold centered int8 residues, not {planes.dtype}")
        if a_residues.device != b_residues.device:
            raise ValueError(f"a_residues is on {a_residues.device}, b_residues on {b_residues.device}")
        (ra, m, k), (rb, kb, n) = a_residues.shape, b_residues.shape
        if ra != rb or k != kb:
            raise ValueError(f"residue planes [{ra}, {m}, {k}] x [{rb}, {kb}, {n}] do not chain "
                             "(channels and K must agree)")
        mods = validate_moduli(moduli)
        if len(mods) != ra:
            raise ValueError(f"{len(mods)} moduli for {ra} residue channels")
        return mods, int(ra), int(m), int(k), int(n)

    def matmul_centered_fused(self, a_residues: torch.Tensor, b_residues: torch.Tensor,
                              moduli: Iterable[int], *, lut_channels: int = 0,
                              workspace: RNSWorkspace | None = None) -> torch.Tensor:
        """Residue planes a [R, M, K] and b [R, K, N] -> exact int64 [M, N]
        (``cuda_backend.py:398-459``).  Returns ``workspace.output``."""
        mods, channels, m, k, n = self._residue_operands(a_residues, b_residues, moduli)
        if lut_channels not in (0, 1, 2):
            raise ValueError(f"lut_channels is {lut_channels}; the table serves 0, 1 or 2 channels")
        device = a_residues.device
        if not self.mfma_compatible(k=k, n=n, moduli=mods, device=device):
            raise ValueError(f"no fused kernel for K={k} with moduli {mods}: 2..10 channels and "
                             "K * max(m // 2)^2 within int32 are required")
        if workspace is None:
            workspace = self.create_workspace(device=device, channels=channels, m=m, n=n)
        self._check_workspace(workspace, channels=channels, m=m, n=n, device=device)
        consts = self._constants(device, mods)
        scratch = self._scratch(
            workspace, int(self._lib.rnsmx_fused_workspace_bytes(m, k, n, channels)))
        self._stats["fused_gemm_calls"] += 1
        self._stats[f"fused_gemm_channels_{channels}"] += 1
        _native.check(self._lib.rnsmx_matmul_centered_fused_out(
            _aligned(a_residues).data_ptr(), b_residues.data_ptr(), m, k, n, consts.native_ref,
            consts.compact_lut.data_ptr(), lut_channels, scratch.data_ptr(), scratch.numel(),
            workspace.output.data_ptr(), _stream_handle(device)))
        return workspace.output

    def matmul_centered_residues(self, a_residues: torch.Tensor, b_residues: torch.Tensor,
                                 moduli: Iterable[int], *, kernel: str = "auto") -> torch.Tensor:
        """Residue-domain product [R, M, N] int8 (centered), as
        ``cuda_backend.py:300-344`` returns.  The exact integer product has
        the same residue in every channel as the per-channel modular GEMM
        (CRT reconstruction preserves residues), so this is the fused product
        re-encoded."""
        mods, _, _, k, n = self._residue_operands(a_residues, b_residues, moduli)
        self.select_centered_kernel(k=k, n=n, moduli=mods, requested=kernel, device=a_residues.device)
        exact = self.matmul_centered_fused(a_residues, b_residues, mods).clone()
        return self._encode_int64_centered(exact, mods)

    def _encode_int64_centered(self, values: torch.Tensor, mods: tuple[int, ...]) -> torch.Tensor:
        # int64 values are residue-reduced with torch integer ops (exact).
        mt = self._constants(values.device, mods).moduli.to(torch.int64).view(
            (-1,) + (1,) * values.ndim)
        r = torch.remainder(values.unsqueeze(0), mt)
        return torch.where(r > mt // 2, r - mt, r).to(torch.int8)

    def decode_garner(self, residues: torch.Tensor, moduli: Iterable[int]) -> torch.Tensor:
        """Centered int8 residues [R, *] -> int64 [*] (``cuda_backend.py:349-364``)."""
        self._validate_matrix(residues, "residues", residues.ndim)
        if residues.dtype != torch.int8:
            raise ValueError("Garner decoder expects centered int8 residues")
        consts = self._constants(residues.device, moduli)
        if residues.shape[0] != len(consts.moduli):
            raise ValueError("residue channel count does not match moduli")
        out = torch.empty(tuple(residues.shape[1:]), dtype=torch.int64, device=residues.device)
        count = int(out.numel())
        if count:
            _native.check(self._lib.rnsmx_decode_garner(
                residues.data_ptr(), count, consts.native_ref, out.data_ptr(),
                _stream_handle(residues.device)))
        return out

    def decode(self, residues: torch.Tensor, moduli: Iterable[int], *,
               signed: bool = True) -> torch.Tensor:
        """CRT decode with torch integer ops (the reference's legacy decoder,
        ``cuda_backend.py:706-731``)."""
        self._validate_matrix(residues, "residues", residues.ndim)
        if residues.dtype not in (torch.uint8, torch.int8):
            raise ValueError("decoder expects uint8 canonical or int8 centered residues")
        mods = validate_moduli(moduli)
        big_p = prod(mods)
        if big_p > (2**63 - 1) // 256:
            raise OverflowError("CRT product is too large for the int64 torch decoder")
        result = torch.zeros(residues.shape[1:], dtype=torch.int64, device=residues.device)
        for c, m in enumerate(mods):
            cof = big_p // m
            basis = (cof * pow(cof % m, -1, m)) % big_p
            canon = torch.remainder(residues[c].to(torch.int64), m)
            # canon * basis < 256 * P fits int64 by the check above
            result = torch.remainder(result + canon * basis, big_p)
        if signed:
            result = torch.where(result > big_p // 2, result - big_p, result)
        return result

    # ------------------------------------------------------------------
    # Prepared weights (cuda_backend.py:464-622)
    # ------------------------------------------------------------------
    def _prepare_nk(self, b_nk: torch.Tensor, mods: tuple[int, ...], k: int, n: int,
                    kernel: str) -> PreparedRNSWeight:
        consts = self._constants(b_nk.device, mods)
        r = len(mods)
        kp = (k + _native.K_ALIGN - 1) // _native.K_ALIGN * _native.K_ALIGN
        packed = torch.empty((r, (n + 15) // 16, kp // _native.K_ALIGN, 1024), dtype=torch.int8,
                             device=b_nk.device)
        absmax = torch.zeros((1,), dtype=torch.int32, device=b_nk.device)
        self._stats["encode_centered_calls"] += 1
        self._stats["encode_centered_values"] += int(b_nk.numel())
        _native.check(self._lib.rnsmx_prepare_weight(
            _aligned(b_nk).data_ptr(), _native.dtype_code(b_nk.dtype), n, k, consts.native_ref,
            packed.data_ptr(), absmax.data_ptr(), _stream_handle(b_nk.device)))
        return PreparedRNSWeight(moduli=mods, k=k, n=n, kernel=kernel, packed=packed,
                                 absmax=absmax)

    def _prepare_packed_nk(self, b_nk: torch.Tensor, mods: tuple[int, ...], k: int,
                           n: int) -> PreparedRNSWeight:
        if b_nk.dtype not in (torch.int8, torch.int16):
            raise ValueError("packed weights take int8/int16 values")
        if not 2 <= len(mods) <= 6:
            raise ValueError("packed weights take 2..6 channels")
        kp = (k + _native.K_ALIGN - 1) // _native.K_ALIGN * _native.K_ALIGN
        packed = torch.empty((2, (n + 15) // 16, kp // _native.K_ALIGN, 1024), dtype=torch.int8,
                             device=b_nk.device)
        absmax = torch.zeros((1,), dtype=torch.int32, device=b_nk.device)
        self._stats["pack_weight_calls"] += 1
        _native.check(self._lib.rnsmx_prepare_weight_packed(
            _aligned(b_nk).data_ptr(), _native.dtype_code(b_nk.dtype), n, k, packed.data_ptr(),
            absmax.data_ptr(), _stream_handle(b_nk.device)))
        return PreparedRNSWeight(moduli=mods, k=k, n=n, kernel=KERNEL_NAME, packed=packed,
                                 absmax=absmax, form="packed")

    def prepare_weight_packed(self, b: torch.Tensor, moduli: Iterable[int]) -> PreparedRNSWeight:
        """B [K, N] int8/int16 -> packed weight, 2 bytes per value for any
        channel count (2..6 channels).  No counterpart in the reference,
        whose prepared storage is one byte per channel (``README.md:26-36``
        names packed residues as the route to a memory saving)."""
        self._validate_matrix(b, "b", 2)
        mods = validate_moduli(moduli)
        return self._prepare_packed_nk(b.t().contiguous(), mods, int(b.shape[0]), int(b.shape[1]))

    def prepare_weight_packed_nk(self, w: torch.Tensor, moduli: Iterable[int]) -> PreparedRNSWeight:
        """``prepare_weight_packed(w.T)`` for a quantized nn.Linear weight
        W [N, K], without the transpose."""
        self._validate_matrix(w, "w", 2)
        mods = validate_moduli(moduli)
        return self._prepare_packed_nk(w, mods, int(w.shape[1]), int(w.shape[0]))

    def prepare_weight(self, b: torch.Tensor, moduli: Iterable[int]) -> PreparedRNSWeight:
        """B [K, N] int8/int16/int32 -> prepared centered residues."""
        self._validate_matrix(b, "b", 2)
        if b.dtype not in (torch.int8, torch.int16, torch.int32):
            raise ValueError("prepared weights support int8/int16/int32")
        mods = validate_moduli(moduli)
        k, n = int(b.shape[0]), int(b.shape[1])
        kernel = self.select_centered_kernel(k=k, n=n, moduli=mods, requested="auto",
                                             device=b.device)
        return self._prepare_nk(b.t().contiguous(), mods, k, n, kernel)

    def prepare_weight_nk(self, w: torch.Tensor, moduli: Iterable[int]) -> PreparedRNSWeight:
        """Same as ``prepare_weight(w.T)`` for a quantized nn.Linear weight
        W [N, K], without the transpose."""
        self._validate_matrix(w, "w", 2)
        if w.dtype not in (torch.int8, torch.int16, torch.int32):
            raise ValueError("prepared weights support int8/int16/int32")
        mods = validate_moduli(moduli)
        n, k = int(w.shape[0]), int(w.shape[1])
        kernel = self.select_centered_kernel(k=k, n=n, moduli=mods, requested="auto",
                                             device=w.device)
        return self._prepare_nk(w, mods, k, n, kernel)

    def _check_activation(self, a: torch.Tensor, prepared: PreparedRNSWeight) -> None:
        self._validate_matrix(a, "a", 2)
        if a.dtype not in (torch.int8, torch.int16, torch.int32):
            raise ValueError("a must be int8/int16/int32")
        if int(a.shape[1]) != prepared.k:
            raise ValueError("K dimension does not match prepared weight")
        if a.device != prepared.packed.device:
            raise ValueError("activation and prepared weight must share device")
        if not self.supports_fused(prepared):
            raise ValueError("prepared weight was not built by this backend")

    def matmul_prepared_fused(self, a: torch.Tensor, prepared_weight: PreparedRNSWeight, *,
                              lut_channels: int = 0, workspace: RNSWorkspace | None = None,
                              out: torch.Tensor | None = None, a_scale: torch.Tensor | None = None,
                              w_scale: torch.Tensor | None = None,
                              bias: torch.Tensor | None = None, plan=None) -> torch.Tensor:
        """a [M, K] int8/16/32 x prepared B -> exact int64 [M, N]
        (``cuda_backend.py:514-539``), returned as ``workspace.output``.

        With ``out`` (float32/float16/bfloat16 [M, N]) plus ``a_scale`` [1]
        and ``w_scale`` [N] (and optional ``bias`` [N], all float32), the
        epilogue instead writes ``((float)x * a_scale) * w_scale + bias`` in
        ``out``'s dtype, the float chain of ``RNSLinear.forward``.
        ``plan`` (kind, mb, nb, ks[, splits]) forces a kernel for this call
        (tuning and tests; results do not depend on it)."""
        return self._prepared_call(a, prepared_weight, lut_channels, workspace, None,
                                   out, a_scale, w_scale, bias, plan)

    def _prepared_call(self, a, prepared, lut_channels, workspace, adaptive, out,
                       a_scale, w_scale, bias, plan=None, count_channels=True):
        self._check_activation(a, prepared)
        if lut_channels not in (0, 1, 2):
            raise ValueError("lut_channels must be 0, 1 or 2")
        device = a.device
        m, k, n = int(a.shape[0]), prepared.k, prepared.n
        channels = len(prepared.moduli)
        consts = self._constants(device, prepared.moduli)
        if workspace is None:
            workspace = self.create_workspace(device=device, channels=channels, m=m, n=n, k=k)
        self._check_workspace(workspace, channels=channels, m=m, n=n, device=device)
        plan = _native.make_plan(plan)
        packed_form = prepared.form == "packed"
        if packed_form:
            scratch = self._scratch(workspace, self._packed_workspace_bytes(m, k, n, channels, plan))
        else:
            scratch = self._scratch(workspace, self._prepared_workspace_bytes(m, k, n, channels, plan))
        epi = None
        target = workspace.output
        if out is not None:
            if out.shape != (m, n) or not out.is_contiguous() or out.device != device:
                raise ValueError("out must be a contiguous [M, N] tensor on the same device")
            if a_scale is None or w_scale is None:
                raise ValueError("float output needs a_scale and w_scale")
            for name, t, size in (("a_scale", a_scale, 1), ("w_scale", w_scale, n),
                                  ("bias", bias, n)):
                if t is None:
                    continue
                if t.dtype != torch.float32 or t.numel() != size or not t.is_contiguous():
                    raise ValueError(f"{name} must be a contiguous float32 tensor of {size} values")
            epi = _native.Epilogue(
                _native.dtype_code(out.dtype), a_scale.data_ptr(), w_scale.data_ptr(),
                bias.data_ptr() if bias is not None else None)
            epi = ctypes.byref(epi)
            target = out
        self._stats["encode_centered_calls"] += 1
        self._stats["encode_centered_values"] += int(a.numel())
        self._stats["fused_gemm_calls"] += 1
        if count_channels:
            self._stats[f"fused_gemm_channels_{channels}"] += 1
        entry = self._lib.rnsmx_matmul_packed_fused if packed_form else self._lib.rnsmx_matmul_prepared_fused
        _native.check(entry(
            _aligned(a).data_ptr(), _native.dtype_code(a.dtype), m, k, n,
            prepared.packed.data_ptr(), consts.native_ref, consts.compact_lut.data_ptr(),
            lut_channels, adaptive, epi, None if plan is None else ctypes.byref(plan),
            scratch.data_ptr(), scratch.numel(), target.data_ptr(), _stream_handle(device)))
        return target

    def encode_activations(self, a: torch.Tensor, prepared_weight: PreparedRNSWeight,
                           out: torch.Tensor | None = None) -> torch.Tensor:
        """a [M, K] -> centered residues [R, M, kp], zero padded to the
        prepared weight's K alignment (the layout the GEMM reads)."""
        self._check_activation(a, prepared_weight)
        m, k = int(a.shape[0]), prepared_weight.k
        kp = prepared_weight.kp
        r = len(prepared_weight.moduli)
        if out is None:
            out = torch.empty((r, m, kp), dtype=torch.int8, device=a.device)
        elif out.shape != (r, m, kp) or out.dtype != torch.int8 or not out.is_contiguous():
            raise ValueError("out must be a contiguous int8 [R, M, kp] tensor")
        consts = self._constants(a.device, prepared_weight.moduli)
        self._stats["encode_centered_calls"] += 1
        self._stats["encode_centered_values"] += int(a.numel())
        _native.check(self._lib.rnsmx_encode_centered(
            _aligned(a).data_ptr(), _native.dtype_code(a.dtype), m, k, kp, consts.native_ref,
            out.data_ptr(), None, None, _stream_handle(a.device)))
        return out

    def matmul_residues_prepared(self, a_residues: torch.Tensor, prepared_weight: PreparedRNSWeight,
                                 *, lut_channels: int = 0, out: torch.Tensor | None = None,
                                 a_scale=None, w_scale=None, bias=None) -> torch.Tensor:
        """GEMM stage alone: residues from ``encode_activations`` x prepared
        weight -> int64 [M, N] (or the float epilogue into ``out``)."""
        if a_residues.ndim != 3 or a_residues.dtype != torch.int8 or not a_residues.is_contiguous():
            raise ValueError("a_residues must be a contiguous int8 [R, M, kp] tensor")
        r, m, kp = map(int, a_residues.shape)
        if r != len(prepared_weight.moduli) or kp != prepared_weight.kp:
            raise ValueError("a_residues do not match the prepared weight")
        if lut_channels not in (0, 1, 2):
            raise ValueError("lut_channels must be 0, 1 or 2")
        n = prepared_weight.n
        consts = self._constants(a_residues.device, prepared_weight.moduli)
        epi = None
        if out is None:
            out = torch.empty((m, n), dtype=torch.int64, device=a_residues.device)
        elif out.dtype != torch.int64:
            if a_scale is None or w_scale is None:
                raise ValueError("float output needs a_scale and w_scale")
            epi = ctypes.byref(_native.Epilogue(
                _native.dtype_code(out.dtype), a_scale.data_ptr(), w_scale.data_ptr(),
                bias.data_ptr() if bias is not None else None))
        if out.shape != (m, n) or not out.is_contiguous():
            raise ValueError("out must be a contiguous [M, N] tensor")
        self._stats["fused_gemm_calls"] += 1
        self._stats[f"fused_gemm_channels_{r}"] += 1
        _native.check(self._lib.rnsmx_matmul_residues_prepared(
            a_residues.data_ptr(), kp, m, prepared_weight.k, n, prepared_weight.packed.data_ptr(),
            consts.native_ref, consts.compact_lut.data_ptr(), lut_channels, epi, out.data_ptr(),
            _stream_handle(a_residues.device)))
        return out

    def matmul_prepared(self, a: torch.Tensor, prepared_weight: PreparedRNSWeight, *,
                        decode: bool = True, kernel: str = "auto") -> torch.Tensor:
        """Non-workspace entry (``cuda_backend.py:489-512``): the exact int64
        product, or its centered residues with ``decode=False``."""
        self._check_activation(a, prepared_weight)
        self.select_centered_kernel(k=prepared_weight.k, n=prepared_weight.n,
                                    moduli=prepared_weight.moduli, requested=kernel,
                                    device=a.device)
        exact = self.matmul_prepared_fused(a, prepared_weight).clone()
        return exact if decode else self._encode_int64_centered(exact, prepared_weight.moduli)

    def prepare_weight_adaptive(self, b: torch.Tensor, moduli: Iterable[int], *,
                                min_channels: int = 3, packed: bool = False) -> PreparedAdaptiveRNSWeight:
        """Encode once; every prefix variant shares the storage (residue
        planes, or with ``packed`` the 2-byte packed form)."""
        full = self.prepare_weight_packed(b, moduli) if packed else self.prepare_weight(b, moduli)
        return self._adaptive_from(full, min_channels)

    def prepare_weight_adaptive_nk(self, w: torch.Tensor, moduli: Iterable[int], *,
                                   min_channels: int = 3, packed: bool = False) -> PreparedAdaptiveRNSWeight:
        full = self.prepare_weight_packed_nk(w, moduli) if packed else self.prepare_weight_nk(w, moduli)
        return self._adaptive_from(full, min_channels)

    def _adaptive_from(self, full: PreparedRNSWeight, min_channels: int) -> PreparedAdaptiveRNSWeight:
        if not 2 <= min_channels <= len(full.moduli):
            raise ValueError("min_channels must be between 2 and full channel count")
        variants = {}
        for c in range(min_channels, len(full.moduli) + 1):
            prefix = full.moduli[:c]
            kernel = self.select_centered_kernel(k=full.k, n=full.n, moduli=prefix,
                                                 requested="auto", device=full.packed.device)
            # residue planes: the prefix's planes; packed bytes serve every prefix whole
            storage = full.packed if full.form == "packed" else full.packed[:c]
            variants[c] = PreparedRNSWeight(moduli=prefix, k=full.k, n=full.n, kernel=kernel,
                                            packed=storage, absmax=full.absmax, form=full.form)
        return PreparedAdaptiveRNSWeight(variants, full.moduli, full.absmax, min_channels)

    def _host_row_bound(self, a: torch.Tensor, max_abs_weight: int) -> int:
        """max_i sum_k |a_ik| * max|B|, read on the host (one synchronisation)."""
        self._validate_matrix(a, "a", 2)
        if a.dtype not in (torch.int8, torch.int16, torch.int32):
            raise ValueError(f"a must be an int8, int16 or int32 matrix, not {a.dtype}")
        row_l1 = a.to(torch.int64).abs().sum(dim=1)
        return safe_l1_dot_bound(int(row_l1.max()) if row_l1.numel() else 0, max_abs_weight)

    def select_adaptive_variant(self, a: torch.Tensor, prepared: PreparedAdaptiveRNSWeight):
        """Host-side selection with the reference's synchronising bound
        (``cuda_backend.py:577-600``): (variant, bound).  The device path of
        the fused adaptive call does not use it."""
        bound = self._host_row_bound(a, prepared.max_abs_weight)
        channels = minimal_prefix_channels(prepared.full_moduli, bound, min_channels=prepared.min_channels)
        for key in ("adaptive_selections", f"adaptive_channels_{channels}"):
            self._stats[key] += 1
        return prepared.variants[channels], bound

    def matmul_prepared_adaptive_fused(self, a: torch.Tensor, prepared: PreparedAdaptiveRNSWeight,
                                       *, lut_channels: int = 2,
                                       workspace_by_channels: dict | None = None,
                                       return_metadata: bool = False, out=None, a_scale=None,
                                       w_scale=None, bias=None, plan=None):
        """Adaptive channel prefix (``cuda_backend.py:602-622``).

        When the weight's preparation proves that no activation of ``a``'s
        dtype can exceed the full set (``device_selection_is_safe``), the
        prefix is chosen on the device inside the one GEMM launch, with no
        host synchronisation; the full-set workspace serves every prefix and
        the metadata is an ``AdaptiveMetadata`` read on demand.  Otherwise
        the selection is the reference's: the row bound is read on the host
        (one synchronisation), ``OverflowError`` is raised before anything
        is computed when no prefix holds it, and the chosen prefix runs as a
        fixed-channel call; the metadata is then a plain dict."""
        full_channels = len(prepared.full_moduli)
        if prepared.device_selection_is_safe(a.dtype):
            workspace = None if workspace_by_channels is None else workspace_by_channels.get(full_channels)
            meta = torch.empty((4,), dtype=torch.int64, device=a.device)
            adaptive = _native.Adaptive(prepared.min_channels, prepared.absmax.data_ptr(), meta.data_ptr())
            self._stats["adaptive_selections"] += 1
            result = self._prepared_call(a, prepared.variants[full_channels], lut_channels, workspace,
                                         ctypes.byref(adaptive), out, a_scale, w_scale, bias, plan,
                                         count_channels=False)
            if return_metadata:
                return result, AdaptiveMetadata(meta, prepared.full_moduli, self._stats)
            return result
        variant, bound = self.select_adaptive_variant(a, prepared)  # raises OverflowError
        channels = len(variant.moduli)
        workspace = None if workspace_by_channels is None else workspace_by_channels.get(channels)
        result = self._prepared_call(a, variant, min(lut_channels, channels), workspace, None, out,
                                     a_scale, w_scale, bias, plan)
        if return_metadata:
            return result, {"channels": channels, "bound": bound,
                            "capacity": (prod(variant.moduli) - 1) // 2}
        return result

    # ------------------------------------------------------------------
    # Continuous batching (cuda_backend.py:624-703)
    # ------------------------------------------------------------------
    def create_request_batch_workspace(self, *, device: torch.device, dtype: torch.dtype,
                                       rows_per_request: Sequence[int], k: int, channels: int,
                                       n: int) -> RNSRequestBatchWorkspace:
        """A staging buffer for the concatenated requests plus the fused
        workspace of the merged product (``cuda_backend.py:624-645``)."""
        rows = tuple(int(r) for r in rows_per_request)
        if len(rows) == 0 or min(rows) < 1:
            raise ValueError(f"every request needs at least one row, got {rows}")
        merged = sum(rows)
        return RNSRequestBatchWorkspace(
            activations=torch.empty((merged, k), dtype=dtype, device=device),
            fused=self.create_workspace(device=device, channels=channels, m=merged, n=n, k=k),
            rows_per_request=rows,
            k=int(k),
        )

    def matmul_prepared_fused_requests(self, requests: Sequence[torch.Tensor],
                                       prepared_weight: PreparedRNSWeight, *,
                                       lut_channels: int = 2,
                                       workspace: RNSRequestBatchWorkspace | None = None,
                                       clone_outputs: bool = False) -> tuple[torch.Tensor, ...]:
        """Continuous batching (``cuda_backend.py:647-703``): the requests'
        rows are stacked into one activation matrix (a single concatenation
        into the staging buffer), multiplied in one fused call, and handed
        back as row views of the merged output (copies with
        ``clone_outputs``)."""
        if len(requests) == 0:
            raise ValueError("no requests to batch")
        for index, request in enumerate(requests):
            self._validate_matrix(request, f"request {index}", 2)
        kinds = {(r.dtype, r.device) for r in requests}
        if len(kinds) != 1:
            raise ValueError(f"requests mix dtypes/devices: {sorted(map(str, kinds))}")
        widths = {int(r.shape[1]) for r in requests}
        if widths != {prepared_weight.k}:
            raise ValueError(f"request widths {sorted(widths)} differ from the weight's K = {prepared_weight.k}")
        rows = tuple(int(r.shape[0]) for r in requests)
        if workspace is None:
            (dtype, device), = kinds
            workspace = self.create_request_batch_workspace(
                device=device, dtype=dtype, rows_per_request=rows, k=prepared_weight.k,
                channels=len(prepared_weight.moduli), n=prepared_weight.n)
        if workspace.rows_per_request != rows or workspace.k != prepared_weight.k:
            raise ValueError(f"batch workspace holds rows {workspace.rows_per_request} x K={workspace.k}, "
                             f"requests are {rows} x K={prepared_weight.k}")
        torch.cat(tuple(requests), dim=0, out=workspace.activations)
        merged = self.matmul_prepared_fused(workspace.activations, prepared_weight,
                                            lut_channels=lut_channels, workspace=workspace.fused)
        bounds = list(itertools.accumulate(rows, initial=0))
        views = tuple(merged[lo:hi] for lo, hi in zip(bounds, bounds[1:]))
        self._stats["continuous_batch_calls"] += 1
        self._stats["continuous_batch_requests"] += len(rows)
        return tuple(v.clone() for v in views) if clone_outputs else views

    # ------------------------------------------------------------------
    # Convenience wrappers (cuda_backend.py:733-799): both integer operands
    # encoded here, then a residue-domain entry point
    # ------------------------------------------------------------------
    def _encode_operands(self, a: torch.Tensor, b: torch.Tensor, moduli: Iterable[int]):
        """Centered residue planes of an integer pair a [M, K], b [K, N] of
        one dtype: (a_res, b_res, moduli)."""
        self._validate_matrix(a, "a", 2)
        self._validate_matrix(b, "b", 2)
        if a.dtype not in (torch.int8, torch.int16, torch.int32):
            raise ValueError(f"a must be an int8, int16 or int32 matrix, not {a.dtype}")
        if b.dtype != a.dtype:
            raise ValueError(f"a is {a.dtype} but b is {b.dtype}; both need the same integer type")
        if a.shape[1] != b.shape[0]:
            raise ValueError(f"a {tuple(a.shape)} and b {tuple(b.shape)} do not chain over K")
        mods = validate_moduli(moduli)
        return self.encode_centered(a, mods), self.encode_centered(b, mods), mods

    def matmul_wide(self, a: torch.Tensor, b: torch.Tensor, moduli: Iterable[int], *,
                    decode: bool = True, kernel: str = "auto") -> torch.Tensor:
        """Exact a @ b as int64 (decode) or its centered residues [R, M, N]."""
        a_res, b_res, mods = self._encode_operands(a, b, moduli)
        if not decode:
            return self.matmul_centered_residues(a_res, b_res, mods, kernel=kernel)
        return self.matmul_centered_fused(a_res, b_res, mods).clone()

    def matmul_wide_fused(self, a: torch.Tensor, b: torch.Tensor, moduli: Iterable[int], *,
                          lut_channels: int = 0,
                          workspace: RNSWorkspace | None = None) -> torch.Tensor:
        """Exact a @ b into ``workspace.output`` (aliasing it, like
        ``matmul_centered_fused``)."""
        a_res, b_res, mods = self._encode_operands(a, b, moduli)
        return self.matmul_centered_fused(a_res, b_res, mods, lut_channels=lut_channels, workspace=workspace)

    def matmul_int8(self, a: torch.Tensor, b: torch.Tensor, moduli: Iterable[int], *,
                    decode: bool = True, kernel: str = "auto") -> torch.Tensor:
        """``matmul_wide`` restricted to int8 operands."""
        if torch.int8 != a.dtype or torch.int8 != b.dtype:
            raise ValueError(f"matmul_int8 takes int8 operands, got {a.dtype} and {b.dtype}")
        return self.matmul_wide(a, b, moduli, decode=decode, kernel=kernel)


def hip_extension_available() -> bool:
    return _native.available()
