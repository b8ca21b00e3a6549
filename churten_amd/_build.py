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
from concurrent.futures import ThreadPoolExecutor
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


# The library's translation units: the optimizers' entry points (Adam's
# dense and segmented ones apart), so that each compiles only its own
# policies and drivers and they compile in parallel; the shared entry points;
# the row copies.
LIB_SOURCES = ("abi_adam.hip", "abi_adam_segments.hip", "abi_sgd.hip", "abi_adagrad.hip",
               "optim_kernels.hip", "rows.hip")
OBJ_DIR = PKG / "_objs"


def _parallel(jobs: list, workers: int | None = None) -> None:
    """Runs the zero-argument callables in ``jobs`` concurrently (each one
    drives a compiler process) and re-raises the first failure."""
    if not jobs:
        return
    n = workers or min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=n) as pool:
        for fut in [pool.submit(j) for j in jobs]:
            fut.result()


def _library_objects(verbose: bool) -> tuple:
    OBJ_DIR.mkdir(exist_ok=True)
    objs, jobs = [], []
    for src in LIB_SOURCES:
        obj = OBJ_DIR / (Path(src).stem + ".hip.o")
        objs.append(obj)
        cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
        jobs.append(lambda cmd=cmd: _run(cmd, verbose))
    return objs, jobs


def _link_library(objs: list, verbose: bool) -> Path:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", *map(str, objs), "-o", str(tmp)],
         verbose)
    os.replace(tmp, LIB)
    return LIB


def build_library(verbose: bool = False) -> Path:
    objs, jobs = _library_objects(verbose)
    _parallel(jobs)
    return _link_library(objs, verbose)


# The CPU kernels state every fused multiply-add explicitly (std::fma) and
# must not gain or lose any: -ffp-contract=off. AVX2/FMA as the reference's
# CPU build (its setup.py:58-60), which the element formulations reproduce.
CPU_KERNEL_FLAGS = ["-O3", "-mavx2", "-mfma", "-ffp-contract=off", "-fno-math-errno"]


def _extension_objects(verbose: bool, sanitize: bool = False):
    import torch
    from torch.utils import cpp_extension

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
    common[1:1] = _sanitize_flags(sanitize)
    OBJ_DIR.mkdir(exist_ok=True)
    objs, jobs = [], []
    for src, flags in (("torch_ops.cpp", ["-O2"]), ("cpu_kernels.cpp", CPU_KERNEL_FLAGS)):
        obj = OBJ_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmd = [*common, *flags, "-c", str(CSRC / src), "-o", str(obj)]
        jobs.append(lambda cmd=cmd: _run(cmd, verbose))
    return objs, jobs


def _sanitize_flags(sanitize: bool) -> list:
    return ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-g"] if sanitize else []


def _link_extension(objs: list, verbose: bool, sanitize: bool = False) -> Path:
    import torch

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    tmp = EXT.with_suffix(".so.tmp")
    _run(
        [
            "g++",
            *_sanitize_flags(sanitize),
            "-shared",
            *map(str, objs),
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


def build_extension(verbose: bool = False, sanitize: bool = False) -> Path:
    """``sanitize``: host code with AddressSanitizer and UBSan (load it with
    their runtimes preloaded; for the CPU tests). Links against the library
    already built."""
    objs, jobs = _extension_objects(verbose, sanitize)
    _parallel(jobs)
    return _link_extension(objs, verbose, sanitize)


def build_bench_library(verbose: bool = False) -> Path:
    """The measurement aid bench.py loads (bench_kernels.hip); not the product ABI."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = BENCH_LIB.with_suffix(".so.tmp")
    _run([_hipcc(), *HIPCC_FLAGS, "-shared", str(CSRC / "bench_kernels.hip"), "-o", str(tmp)],
         verbose)
    os.replace(tmp, BENCH_LIB)
    return BENCH_LIB


def build(verbose: bool = False) -> None:
    """Every compile runs concurrently; the library is linked once its objects
    are there, the operator extension after it (it links against it)."""
    lib_objs, lib_jobs = _library_objects(verbose)
    ext_objs, ext_jobs = _extension_objects(verbose)
    _parallel([*lib_jobs, lambda: build_bench_library(verbose), *ext_jobs])
    _link_library(lib_objs, verbose)
    _link_extension(ext_objs, verbose)


if __name__ == "__main__":
    build(verbose=True)
