"""Builds librnsmx.so (gfx950) in this package directory with hipcc.

Every translation unit is compiled to an object in parallel, then linked.
The GEMM kernels are split into parts (rnsmx_gemm_part.hip, built once per
channel capacity and part) so no single object dominates the build."""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)                 # rns-llm_amd/
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
OBJDIR = os.path.join(ROOT, "_build")
OUT = os.path.join(PKG, "librnsmx.so")
GEMM_CAPACITIES = (3, 4, 6, 10)
GEMM_PARTS = 6
# (source, object name, extra flags)
UNITS = [("rnsmx_kernels.hip", "rnsmx_kernels", []), ("rnsmx_host.cpp", "rnsmx_host", [])] + [
    ("rnsmx_gemm_part.hip", f"rnsmx_gemm_r{r}_p{p}", [f"-DRNSMX_RCAP={r}", f"-DRNSMX_PART={p}"])
    for r in GEMM_CAPACITIES for p in range(GEMM_PARTS)]
ARCH = os.environ.get("RNSMX_OFFLOAD_ARCH", "gfx950")
NOISE = "packed-fp32-ops"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        # packed fp32 VALU ops stay off for all device code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
        "-I", INCLUDE, "-I", CSRC,
    ]


def compile_command(source: str, obj: str, extra: list[str]) -> list[str]:
    return [hipcc(), *flags(), *extra, "-c", os.path.join(CSRC, source), "-o", obj]


def link_command(objs: list[str], out: str) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs,
            "-Wl,-rpath,/opt/rocm/lib", "-o", out]


def _run(cmd: list[str]) -> tuple[int, str, list[str]]:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if NOISE not in ln]
    return proc.returncode, "\n".join(msgs), cmd


def build(verbose: bool = False) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    objs = [os.path.join(OBJDIR, name + ".o") for _, name, _ in UNITS]
    jobs = min(len(UNITS), max(1, min(16, os.cpu_count() or 1)))
    # the longest units first, so the tail of the build stays short
    order = sorted(range(len(UNITS)), key=lambda i: UNITS[i][0] != "rnsmx_gemm_part.hip")
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(_run, [compile_command(UNITS[i][0], objs[i], UNITS[i][2]) for i in order]))
    for rc, msgs, cmd in results:
        if rc != 0:
            sys.stderr.write(msgs + "\n")
            raise RuntimeError(f"hipcc failed ({rc}): {' '.join(cmd)}")
        if verbose and msgs:
            sys.stderr.write(msgs + "\n")
    tmp = OUT + ".tmp"
    rc, msgs, cmd = _run(link_command(objs, tmp))
    if rc != 0:
        sys.stderr.write(msgs + "\n")
        raise RuntimeError(f"hipcc link failed ({rc}): {' '.join(cmd)}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
