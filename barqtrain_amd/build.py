"""Build recipe for the native parts of barqtrain_amd, in-tree.

* ``libbarq_kv.so`` -- the gfx950 HIP kernels and their C ABI (include/barq_kv.h), compiled by
  ``hipcc --offload-arch=gfx950`` only.
* ``barqtrain_cuda<EXT_SUFFIX>`` -- the host-only torch extension module (csrc/barq_kv_torch.cpp)
  that the loader imports under the reference's module name; compiled by ``g++`` against the
  installed torch headers and linked to ``libbarq_kv.so`` through ``$ORIGIN``.

Run ``python -m barqtrain_amd.build`` (or ``__graft_entry__.build()``).  No GPU is needed.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
LIB_NAME = "libbarq_kv.so"
EXT_NAME = "barqtrain_cuda"
OFFLOAD_ARCH = "gfx950"
HIP_SOURCES = ("barq_kv.hip", "barq_kv_attention.hip", "barq_kv_quant.hip")
HIP_HEADERS = ("fastdiv.h", "barq_kv_fp8.h", "barq_kv_commit.h")
HOST_SOURCES = ("barq_kv_torch.cpp",)


def source_files() -> tuple[Path, ...]:
    """Every file the build reads: the HIP sources and headers, the binding, the C ABI header."""
    return tuple(CSRC / f for f in HIP_SOURCES + HIP_HEADERS + HOST_SOURCES) + (INCLUDE / "barq_kv.h",)

# Packed fp32 instructions stay off in every HIP compile (none are needed: the kernels only
# move bits, but the flag keeps the compiler from forming them).
HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def lib_path() -> Path:
    return PKG_DIR / LIB_NAME


def ext_path() -> Path:
    return PKG_DIR / (EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH") or os.environ.get("ROCM_HOME") or "/opt/rocm"
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: the gfx950 kernels cannot be built")
    return found


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build_library(verbose: bool = False) -> Path:
    """Compile the HIP kernels and C ABI into barqtrain_amd/libbarq_kv.so."""
    out = lib_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [_hipcc(), *HIP_FLAGS, "-shared", f"-I{INCLUDE}", f"-I{CSRC}",
           *[str(CSRC / name) for name in HIP_SOURCES], "-o", str(tmp)]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build_extension(verbose: bool = False) -> Path:
    """Compile the torch binding module barqtrain_cuda next to the library."""
    import torch
    from torch.utils import cpp_extension

    out = ext_path()
    tmp = out.with_name(out.name + ".tmp")
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    rocm = os.environ.get("ROCM_PATH") or "/opt/rocm"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{p}" for p in cpp_extension.include_paths(device_type="cuda")],
        f"-I{rocm}/include", f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
        *(str(CSRC / f) for f in HOST_SOURCES),
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-ltorch_hip",
        f"-L{PKG_DIR}", "-lbarq_kv", "-Wl,-rpath,$ORIGIN",
        "-o", str(tmp),
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_extension(verbose)


def is_built() -> bool:
    return lib_path().exists() and ext_path().exists()


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(f"built {lib_path()} and {ext_path()}")
