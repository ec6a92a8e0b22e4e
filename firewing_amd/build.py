"""Build libfirewing_hip_moe.so in-tree with hipcc for gfx950.

Every translation unit is compiled with -ffp-contract=off (no multiply-add
contraction: the exact-order kernels depend on it), with f32 denormals kept,
and without packed-FP32 instructions.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
ROOT = PKG.parent
LIB = PKG / "libfirewing_hip_moe.so"
ARCH = os.environ.get("FIREWING_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")
    return path


def _compile(args: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(args), flush=True)
    res = subprocess.run(args, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-6000:]}")


HOST_CHECK = PKG / "_build" / "zstd_host_check"


def host_check(verbose: bool = False) -> Path:
    """Compile tests/zstd_host_check.cpp (fw_zstd.h's format core on the host,
    g++ with AddressSanitizer) into _build/."""
    (PKG / "_build").mkdir(exist_ok=True)
    rocm = Path(hipcc()).resolve().parent.parent
    _compile(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
              "-D__HIP_PLATFORM_AMD__", "-I", str(rocm / "include"), "-I", str(CSRC),
              str(ROOT / "tests" / "zstd_host_check.cpp"), "-o", str(HOST_CHECK)], verbose)
    return HOST_CHECK


def build(verbose: bool = False) -> Path:
    """Compile the host/stateless translation unit and one decode-kernel unit
    per token count in parallel, then link the shared library in place."""
    from concurrent.futures import ThreadPoolExecutor

    out_dir = PKG / "_build"
    out_dir.mkdir(exist_ok=True)
    include = ["-I", str(ROOT / "include"), "-I", str(CSRC)]
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    units = [(CSRC / "fw_moe.hip", [], out_dir / "fw_moe.o"),
             (CSRC / "fw_safetensors.cpp", [], out_dir / "fw_safetensors.o"),
             (CSRC / "fw_zstd.hip", [], out_dir / "fw_zstd.o")]
    for nt in (1, 2, 3, 4):
        units.append((CSRC / "fw_decode_kernels.hip", [f"-DFW_NT={nt}"], out_dir / f"fw_decode_t{nt}.o"))
    jobs = [[hipcc(), *compile_flags, *include, *defs, "-c", str(src), "-o", str(obj)] for src, defs, obj in units]
    workers = max(1, min(len(jobs), os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for f in [pool.submit(_compile, j, verbose) for j in jobs]:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _compile([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *[str(o) for _, _, o in units], "-o", str(tmp)],
             verbose)
    os.replace(tmp, LIB)
    # the zstd format core on the host under AddressSanitizer, for tests/test_zstd_host.py
    host_check(verbose)
    # stand-alone C++ driver of the decode step (for profilers), next to the library
    drv = PKG / "fw_decode_bench"
    _compile([hipcc(), "-O2", "-std=c++17", *include, str(CSRC / "fw_decode_bench.cpp"), "-o", str(drv),
              "-L", str(PKG), "-lfirewing_hip_moe", f"-Wl,-rpath,{PKG}", "-Wl,-rpath,$ORIGIN"], verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
