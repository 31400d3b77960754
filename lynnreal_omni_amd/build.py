"""Build liblynnreal_amd.so, the gfx950 HIP library of the W8A8 path, in-tree.

Usage: python -m lynnreal_omni_amd.build  (or build() from Python).

Every .hip file under csrc/ is compiled for gfx950 only, in parallel, and
linked into lynnreal_omni_amd/liblynnreal_amd.so; csrc/pycall.c becomes the
CPython module _pycall beside it. The library is written to
a temporary name and renamed into place, so a process that has the old one
loaded keeps a valid mapping.
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sysconfig

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
OBJ = HERE / "_build"
LIBRARY = HERE / "liblynnreal_amd.so"

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # IEEE semantics: no FMA contraction, correctly rounded fp32 divide/sqrt.
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # Never emit packed fp32 arithmetic (device pass; the host pass ignores it).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP toolchain is required to build")
    return path


# Per-file flags. The GEMM keeps at most 128 accumulators per wave and wants
# them in VGPRs: with the default heuristic LLVM puts MFMA accumulators in
# AGPRs and copies them between AGPRs and VGPRs inside the k-loop.
FILE_FLAGS = {"gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: pathlib.Path, extra: list[str]) -> pathlib.Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [hipcc(), *FLAGS, *FILE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    return obj


PYCALL = HERE / ("_pycall" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))


def build_pycall() -> pathlib.Path:
    """Compile csrc/pycall.c, the CPython fast-call shim of the integer-argument
    entry points, with the host C compiler (no GPU code in it)."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler found for csrc/pycall.c")
    tmp = PYCALL.with_name(PYCALL.name + f".tmp{os.getpid()}")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", f"-I{sysconfig.get_paths()['include']}",
           str(CSRC / "pycall.c"), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"pycall.c failed:\n{proc.stderr}")
    os.replace(tmp, PYCALL)
    return PYCALL


ABI_CONSUMER = ROOT / "tests" / "abi_host" / "c_abi_consumer"


def build_abi_consumer() -> pathlib.Path:
    """Compile tests/abi_host/c_abi_consumer.cpp, a C++ host program that uses
    the library through include/lynnreal_amd.h alone (host code, no GPU code),
    against the library built here; a GPU test runs it."""
    cxx = shutil.which("g++") or shutil.which("c++")
    src = ABI_CONSUMER.with_suffix(".cpp")
    if cxx is None or not src.exists():
        raise RuntimeError("no C++ compiler or no tests/abi_host/c_abi_consumer.cpp")
    rocm = pathlib.Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    tmp = ABI_CONSUMER.with_name(ABI_CONSUMER.name + f".tmp{os.getpid()}")
    cmd = [cxx, "-O2", "-std=c++17", "-ffp-contract=off", "-Wall", "-D__HIP_PLATFORM_AMD__",
           f"-I{rocm / 'include'}", f"-I{ROOT / 'include'}", str(src), "-o", str(tmp),
           f"-L{HERE}", "-llynnreal_amd", f"-L{rocm / 'lib'}", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN/../../lynnreal_omni_amd", f"-Wl,-rpath,{rocm / 'lib'}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"c_abi_consumer.cpp failed:\n{proc.stderr}")
    os.replace(tmp, ABI_CONSUMER)
    return ABI_CONSUMER


def build(extra: list[str] | None = None, jobs: int = 8) -> pathlib.Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library (and
    the CPython fast-call shim beside it)."""
    extra = list(extra or [])
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda s: _compile(s, extra), sources))
    tmp = LIBRARY.with_name(LIBRARY.name + f".tmp{os.getpid()}")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    build_pycall()
    build_abi_consumer()
    return LIBRARY


if __name__ == "__main__":
    print(build())
