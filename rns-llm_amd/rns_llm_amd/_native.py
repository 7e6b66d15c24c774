"""ctypes binding of librnsmx.so, the gfx950 C-ABI library (include/rnsmx.h).

The library is loaded from this package directory.  There is no fallback:
if it is missing or fails to load, every backend entry point raises
``RuntimeError``, the way the reference raises when its extension is not
built (``src/rns_llm/backends/cuda_backend.py:29-37``).
"""
from __future__ import annotations

import ctypes
import os
from functools import lru_cache

LIB_NAME = "librnsmx.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

MAX_CHANNELS = 10
K_ALIGN = 64
SPLIT_TICKETS = 16384  # RNSMX_SPLIT_TICKETS: 32-bit counters at the start of a workspace
NOALLOC_SCRATCH_BYTES = 16 << 20  # RNSMX_NOALLOC_SCRATCH_BYTES

OK, EINVAL, ERANGE, ELAUNCH, ESPACE = 0, 1, 2, 3, 4

INT8, INT16, INT32, INT64, FLOAT32, FLOAT16, BFLOAT16 = range(7)

# Every symbol include/rnsmx.h declares.
EXPORTED_SYMBOLS = (
    "rnsmx_last_error",
    "rnsmx_abi_version",
    "rnsmx_moduli_init",
    "rnsmx_compact_lut",
    "rnsmx_encode_centered",
    "rnsmx_fused_workspace_bytes",
    "rnsmx_matmul_centered_fused_out",
    "rnsmx_prepare_weight",
    "rnsmx_prepared_workspace_bytes",
    "rnsmx_matmul_prepared_fused",
    "rnsmx_matmul_prepared_fused_noalloc",
    "rnsmx_matmul_residues_prepared",
    "rnsmx_gemm_plan",
    "rnsmx_prepare_weight_packed",
    "rnsmx_packed_workspace_bytes",
    "rnsmx_matmul_packed_fused",
    "rnsmx_packed_plan",
    "rnsmx_quantize_symmetric",
    "rnsmx_linear_workspace_bytes",
    "rnsmx_linear_forward",
    "rnsmx_decode_garner",
)

QUANT_SCRATCH = 1025  # RNSMX_QUANT_SCRATCH


class Moduli(ctypes.Structure):
    """Mirror of ``rnsmx_moduli_t``."""

    _fields_ = [
        ("channels", ctypes.c_int32),
        ("moduli", ctypes.c_int32 * MAX_CHANNELS),
        ("magic", ctypes.c_uint32 * MAX_CHANNELS),
        ("c31", ctypes.c_uint32 * MAX_CHANNELS),
        ("qinv", ctypes.c_uint32 * MAX_CHANNELS),
        ("ucoef", (ctypes.c_uint32 * MAX_CHANNELS) * MAX_CHANNELS),
        ("prefix", ctypes.c_int64 * (MAX_CHANNELS + 1)),
        ("qk16", ctypes.c_int32 * MAX_CHANNELS),
        ("qk8", ctypes.c_uint32 * MAX_CHANNELS),
    ]


class Epilogue(ctypes.Structure):
    """Mirror of ``rnsmx_epilogue_t``."""

    _fields_ = [
        ("out_dtype", ctypes.c_int32),
        ("a_scale_dev", ctypes.c_void_p),
        ("w_scale_dev", ctypes.c_void_p),
        ("bias_dev", ctypes.c_void_p),
    ]


class Plan(ctypes.Structure):
    """Mirror of ``rnsmx_plan_t``: kind 0 = automatic; 1 stream, 2 MFMA,
    3 LDS-staged, 4 wide stream, 5 three-wave MFMA; tile blocks, ks, and
    the number of workgroups splitting K."""

    _fields_ = [
        ("kind", ctypes.c_int32),
        ("mb", ctypes.c_int32),
        ("nb", ctypes.c_int32),
        ("ks", ctypes.c_int32),
        ("splits", ctypes.c_int32),
        ("tail", ctypes.c_int32),
    ]

    def as_tuple(self) -> tuple[int, ...]:
        return (self.kind, self.mb, self.nb, self.ks, self.splits, self.tail)


def make_plan(plan) -> "Plan | None":
    """A ``Plan`` from a (kind, mb, nb, ks[, splits[, tail]]) tuple; None stays None."""
    if plan is None or isinstance(plan, Plan):
        return plan
    fields = tuple(int(v) for v in plan)
    fields += (1, 0)[len(fields) - 4:] if 4 <= len(fields) < 6 else ()
    if len(fields) != 6:
        raise ValueError("a plan is (kind, mb, nb, ks[, splits[, tail]])")
    return Plan(*fields)


class Adaptive(ctypes.Structure):
    """Mirror of ``rnsmx_adaptive_t``."""

    _fields_ = [
        ("min_channels", ctypes.c_int32),
        ("w_absmax_dev", ctypes.c_void_p),
        ("meta_dev", ctypes.c_void_p),
    ]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64

_SIGNATURES = {
    "rnsmx_last_error": (ctypes.c_char_p, []),
    "rnsmx_abi_version": (_I32, []),
    "rnsmx_moduli_init": (_I32, [_P, _I32, ctypes.POINTER(Moduli)]),
    "rnsmx_compact_lut": (_I32, [ctypes.POINTER(Moduli), _P]),
    "rnsmx_encode_centered": (
        _I32, [_P, _I32, _I64, _I64, _I64, ctypes.POINTER(Moduli), _P, _P, _P, _P]),
    "rnsmx_fused_workspace_bytes": (_I64, [_I64, _I64, _I64, _I32]),
    "rnsmx_matmul_centered_fused_out": (
        _I32, [_P, _P, _I32, _I32, _I32, ctypes.POINTER(Moduli), _P, _I32, _P, _I64, _P, _P]),
    "rnsmx_prepare_weight": (
        _I32, [_P, _I32, _I32, _I32, ctypes.POINTER(Moduli), _P, _P, _P]),
    "rnsmx_prepared_workspace_bytes": (_I64, [_I64, _I64, _I64, _I32, ctypes.POINTER(Plan)]),
    "rnsmx_matmul_prepared_fused": (
        _I32, [_P, _I32, _I32, _I32, _I32, _P, ctypes.POINTER(Moduli), _P, _I32,
               ctypes.POINTER(Adaptive), ctypes.POINTER(Epilogue), ctypes.POINTER(Plan),
               _P, _I64, _P, _P]),
    "rnsmx_matmul_prepared_fused_noalloc": (
        _I32, [_P, _I32, _I32, _I32, _I32, _P, ctypes.POINTER(Moduli), _P, _I32,
               ctypes.POINTER(Adaptive), ctypes.POINTER(Epilogue), ctypes.POINTER(Plan), _P, _P]),
    "rnsmx_matmul_residues_prepared": (
        _I32, [_P, _I64, _I32, _I32, _I32, _P, ctypes.POINTER(Moduli), _P, _I32,
               ctypes.POINTER(Epilogue), _P, _P]),
    "rnsmx_gemm_plan": (_I32, [_I64, _I64, _I64, _I32, _I32, ctypes.POINTER(Plan)]),
    "rnsmx_prepare_weight_packed": (_I32, [_P, _I32, _I32, _I32, _P, _P, _P]),
    "rnsmx_packed_workspace_bytes": (_I64, [_I64, _I64, _I64, _I32, ctypes.POINTER(Plan)]),
    "rnsmx_matmul_packed_fused": (
        _I32, [_P, _I32, _I32, _I32, _I32, _P, ctypes.POINTER(Moduli), _P, _I32,
               ctypes.POINTER(Adaptive), ctypes.POINTER(Epilogue), ctypes.POINTER(Plan),
               _P, _I64, _P, _P]),
    "rnsmx_packed_plan": (_I32, [_I64, _I64, _I64, _I32, ctypes.POINTER(Plan)]),
    "rnsmx_quantize_symmetric": (_I32, [_P, _I32, _I64, _I32, _P, _P, _P, _P]),
    "rnsmx_linear_workspace_bytes": (_I64, [_I64, _I64, _I64, _I32, _I32]),
    "rnsmx_linear_forward": (
        _I32, [_P, _I32, _I32, _I32, _I32, _I32, _P, ctypes.POINTER(Moduli), _P, _P,
               ctypes.POINTER(Adaptive), _P, _I64, _P, _P]),
    "rnsmx_decode_garner": (_I32, [_P, _I64, ctypes.POINTER(Moduli), _P, _P]),
}

ABI_VERSION = 5


class NativeError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"rnsmx native library is not built ({LIB_PATH} missing); run "
            "`python -c 'import __graft_entry__ as g; g.build()'` at the repo root")
    handle = ctypes.CDLL(LIB_PATH)
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = handle.rnsmx_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"librnsmx ABI version {version}, expected {ABI_VERSION}")
    return handle


def available() -> bool:
    try:
        lib()
    except (RuntimeError, OSError):
        return False
    return True


def check(rc: int) -> None:
    """Raise on a non-zero status: ValueError for argument errors (the
    reference's Python-level checks), OverflowError for range errors, and
    RuntimeError for launch failures."""
    if rc == OK:
        return
    message = lib().rnsmx_last_error().decode("utf-8", "replace")
    if rc == EINVAL:
        raise ValueError(message)
    if rc == ERANGE:
        raise OverflowError(message)
    raise NativeError(rc, message)


def make_moduli(moduli) -> Moduli:
    mods = tuple(int(m) for m in moduli)
    arr = (ctypes.c_int32 * max(1, len(mods)))(*mods)
    out = Moduli()
    check(lib().rnsmx_moduli_init(ctypes.cast(arr, _P), len(mods), ctypes.byref(out)))
    return out


_DTYPE_CODES: dict = {}


def dtype_code(dtype) -> int:
    if not _DTYPE_CODES:
        import torch

        _DTYPE_CODES.update({
            torch.int8: INT8,
            torch.int16: INT16,
            torch.int32: INT32,
            torch.int64: INT64,
            torch.float32: FLOAT32,
            torch.float16: FLOAT16,
            torch.bfloat16: BFLOAT16,
        })
    code = _DTYPE_CODES.get(dtype)
    if code is None:
        raise ValueError(f"unsupported dtype {dtype}")
    return code
