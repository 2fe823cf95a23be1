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


def object_dir() -> Path:
    return PKG_DIR / "_build"


def build_library(verbose: bool = False, defines: tuple[str, ...] = (), out: Path | None = None) -> Path:
    """Compile the HIP kernels and C ABI into barqtrain_amd/libbarq_kv.so: every source to an
    object in parallel (the sources are independent), then one link.  `defines` (``NAME=VALUE``)
    and `out` build an alternative library from the same sources."""
    out = out or lib_path()
    objs = object_dir()
    objs.mkdir(exist_ok=True)
    tag = "" if not defines else "-" + "-".join(d.replace("=", "_") for d in defines)
    procs = []
    for name in HIP_SOURCES:
        obj = objs / (Path(name).stem + tag + ".o")
        cmd = [_hipcc(), *HIP_FLAGS, "-c", f"-I{INCLUDE}", f"-I{CSRC}", *(f"-D{d}" for d in defines),
               str(CSRC / name), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for cmd, _, proc in procs:
        text = proc.communicate()[0]
        if proc.returncode != 0:
            failed.append(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{text}")
    if failed:
        raise RuntimeError("\n".join(failed))
    tmp = out.with_suffix(".so.tmp")
    _run([_hipcc(), *HIP_FLAGS, "-shared", *(str(o) for _, o, _ in procs), "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def _extension_commands(obj: Path, tmp: Path) -> tuple[list[str], list[str]]:
    """(compile, link) commands of the torch binding module."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    rocm = os.environ.get("ROCM_PATH") or "/opt/rocm"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    compile_cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-c",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{p}" for p in cpp_extension.include_paths(device_type="cuda")],
        f"-I{rocm}/include", f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
        *(str(CSRC / f) for f in HOST_SOURCES), "-o", str(obj),
    ]
    link_cmd = [
        os.environ.get("CXX", "g++"), "-shared", str(obj),
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-ltorch_hip",
        f"-L{PKG_DIR}", "-lbarq_kv", "-Wl,-rpath,$ORIGIN",
        "-o", str(tmp),
    ]
    return compile_cmd, link_cmd


def build_extension(verbose: bool = False, compiled: subprocess.Popen | None = None) -> Path:
    """Compile the torch binding module barqtrain_cuda next to the library (its object may
    already be compiling: `compiled`, started by build())."""
    out = ext_path()
    tmp = out.with_name(out.name + ".tmp")
    object_dir().mkdir(exist_ok=True)
    obj = object_dir() / "barq_kv_torch.o"
    compile_cmd, link_cmd = _extension_commands(obj, tmp)
    if compiled is None:
        _run(compile_cmd, verbose)
    else:
        text = compiled.communicate()[0]
        if compiled.returncode != 0:
            raise RuntimeError(f"build step failed ({compiled.returncode}): {' '.join(compile_cmd)}\n{text}")
    _run(link_cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    """Both parts; the binding's object compiles while the HIP sources do."""
    object_dir().mkdir(exist_ok=True)
    compile_cmd, _ = _extension_commands(object_dir() / "barq_kv_torch.o", ext_path())
    if verbose:
        print(" ".join(compile_cmd), flush=True)
    ext_proc = subprocess.Popen(compile_cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    try:
        build_library(verbose)
    except BaseException:
        ext_proc.kill()
        ext_proc.wait()
        raise
    build_extension(verbose, compiled=ext_proc)


def is_built() -> bool:
    return lib_path().exists() and ext_path().exists()


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(f"built {lib_path()} and {ext_path()}")
