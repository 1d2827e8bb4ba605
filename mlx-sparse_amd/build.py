"""Build recipe for the MI355X library and its Python binding.

Produces, in-tree (so the built files travel with the source tree):

- ``mlx_sparse/libmsx_sparse.so``: the C-ABI library (``include/msx_sparse.h``)
  - HIP kernels compiled by hipcc for gfx950, plus the host CPU path;
- ``mlx_sparse/_ext.<abi>.so``: the pybind11 module over the C++ primitive
  layer in ``src/``, linked to the library with an ``$ORIGIN`` rpath.

Run ``python mlx-sparse_amd/build.py`` (or ``__graft_entry__.build()``).
Objects go to ``mlx-sparse_amd/_build/``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
INCLUDE = REPO / "include"
CSRC = PKG_ROOT / "csrc"
SRC = PKG_ROOT / "src"
OUT_DIR = PKG_ROOT / "mlx_sparse"
BUILD = PKG_ROOT / "_build"

ARCH = os.environ.get("MSX_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# Device code: -ffp-contract=off keeps products and sums separately rounded
# (the reference CPU arithmetic); packed fp32 instructions are disabled.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wextra",
             f"-I{INCLUDE}", f"-I{CSRC}", f"-I{SRC}"]

LIB_NAME = "libmsx_sparse.so"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line  # host pass does not know the feature
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def _ext_suffix() -> str:
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def build(verbose: bool = True) -> Path:
    """Compile every source and link both shared objects.  Returns OUT_DIR."""
    BUILD.mkdir(parents=True, exist_ok=True)
    hip_srcs = sorted(CSRC.glob("*.hip"))
    cpu_srcs = sorted(CSRC.glob("*.cpp"))
    jobs = []
    for s in hip_srcs:
        jobs.append([HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(BUILD / (s.stem + ".o"))])
    for s in cpu_srcs:
        jobs.append(["g++", *CXX_FLAGS, "-c", str(s), "-o", str(BUILD / (s.stem + ".o"))])

    import pybind11  # noqa: PLC0415 - build-time dependency only

    py_inc = sysconfig.get_paths()["include"]
    bind_srcs = [SRC / "bindings.cpp", SRC / "common" / "validate.cpp",
                 SRC / "sparse" / "csr_matvec" / "csr_matvec.cpp",
                 SRC / "sparse" / "csr_matmul" / "csr_matmul.cpp",
                 SRC / "sparse" / "csr_batched_matvec" / "csr_batched_matvec.cpp",
                 SRC / "sparse" / "csr_batched_matmul" / "csr_batched_matmul.cpp",
                 SRC / "sparse" / "csr_adjoint" / "csr_adjoint.cpp",
                 SRC / "linalg" / "csr_cg.cpp", SRC / "linalg" / "csr_krylov.cpp"]
    bind_objs = []
    for s in bind_srcs:
        o = BUILD / ("bind_" + s.stem + ".o")
        bind_objs.append(o)
        jobs.append(["g++", *CXX_FLAGS, "-fvisibility=hidden", f"-I{pybind11.get_include()}",
                     f"-I{py_inc}", "-c", str(s), "-o", str(o)])

    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(_run, jobs))

    lib = OUT_DIR / LIB_NAME
    objs = [str(BUILD / (s.stem + ".o")) for s in hip_srcs + cpu_srcs]
    tmp = lib.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs, "-pthread"])
    os.replace(tmp, lib)

    ext = OUT_DIR / ("_ext" + _ext_suffix())
    tmp = ext.with_suffix(".tmp")
    _run(["g++", "-shared", "-fPIC", "-o", str(tmp), *map(str, bind_objs),
          f"-L{OUT_DIR}", "-lmsx_sparse", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, ext)
    if verbose:
        print(f"built {lib.relative_to(REPO)} and {ext.relative_to(REPO)}")
    return OUT_DIR


if __name__ == "__main__":
    build()
    sys.exit(0)
