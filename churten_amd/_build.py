"""Ahead-of-time build of the native parts of churten_amd.

Two artefacts, both built in-tree so they travel with the source tree:

* ``churten_amd/lib/libchurten_optim.so`` -- the gfx950 HIP kernels and the
  C ABI of ``include/churten_optim.h``, compiled with ``hipcc`` directly (no
  hipify step, no torch headers).
* ``churten_amd/kernels/_C.so`` -- the ``torchstrap`` operator library: the
  schemas plus the GPU dispatch-key wrappers that call the C ABI, compiled with
  ``g++`` against torch's headers and linked to the library above through an
  ``$ORIGIN`` rpath.

Run ``python -m churten_amd._build`` or ``__graft_entry__.build()``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
KERNELS_DIR = PKG / "kernels"

LIB = LIB_DIR / "libchurten_optim.so"
BENCH_LIB = LIB_DIR / "libchurten_bench.so"
EXT = KERNELS_DIR / "_C.so"

ARCH = "gfx950"

# -O3 with hipcc's default contraction (-ffp-contract=fast) and correctly
# rounded fp32 divide/sqrt: the element math is checked bit-for-bit against
# torch's ROCm kernels, which are built the same way. Packed-fp32 instructions
# are disabled for every HIP compile in this project.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        sys.stderr.write(proc.stderr)
        raise RuntimeError(f"build step failed ({proc.returncode}): {cmd[0]}")
    noisy = [
        ln
        for ln in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in ln and ln.strip()
    ]
    if verbose and noisy:
        print("\n".join(noisy), flush=True)


def build_library(verbose: bool = False) -> Path:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    _run(
        [_hipcc(), *HIPCC_FLAGS, str(CSRC / "optim_kernels.hip"), str(CSRC / "rows.hip"),
         "-o", str(tmp)],
        verbose,
    )
    os.replace(tmp, LIB)
    return LIB


# The CPU kernels state every fused multiply-add explicitly (std::fma) and
# must not gain or lose any: -ffp-contract=off. AVX2/FMA as the reference's
# CPU build (its setup.py:58-60), which the element formulations reproduce.
CPU_KERNEL_FLAGS = ["-O3", "-mavx2", "-mfma", "-ffp-contract=off", "-fno-math-errno"]


def build_extension(verbose: bool = False, sanitize: bool = False) -> Path:
    """``sanitize``: host code with AddressSanitizer and UBSan (load it with
    their runtimes preloaded; for the CPU tests)."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], "/opt/rocm/include"]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    common = [
        "g++",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-function",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C",
        *[f"-isystem{p}" for p in incs],
    ]
    san = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-g"] if sanitize else []
    common[1:1] = san
    build_dir = PKG / "_objs"
    build_dir.mkdir(exist_ok=True)
    objs = []
    for src, flags in (("torch_ops.cpp", ["-O2"]), ("cpu_kernels.cpp", CPU_KERNEL_FLAGS)):
        obj = build_dir / (Path(src).stem + ".o")
        _run([*common, *flags, "-c", str(CSRC / src), "-o", str(obj)], verbose)
        objs.append(str(obj))
    tmp = EXT.with_suffix(".so.tmp")
    _run(
        [
            "g++",
            *san,
            "-shared",
            *objs,
            "-o",
            str(tmp),
            f"-L{LIB_DIR}",
            "-lchurten_optim",
            f"-L{torch_lib}",
            "-lc10",
            "-lc10_hip",
            "-ltorch_cpu",
            "-ltorch",
            "-Wl,-rpath,$ORIGIN/../lib",
            f"-Wl,-rpath,{torch_lib}",
        ],
        verbose,
    )
    os.replace(tmp, EXT)
    return EXT


def build_bench_library(verbose: bool = False) -> Path:
    """The measurement aid bench.py loads (bench_kernels.hip); not the product ABI."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = BENCH_LIB.with_suffix(".so.tmp")
    _run([_hipcc(), *HIPCC_FLAGS, str(CSRC / "bench_kernels.hip"), "-o", str(tmp)], verbose)
    os.replace(tmp, BENCH_LIB)
    return BENCH_LIB


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_bench_library(verbose)
    build_extension(verbose)


if __name__ == "__main__":
    build(verbose=True)
