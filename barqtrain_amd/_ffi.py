"""Native backend loader, with the contract of the reference's python/barqtrain/_ffi.py:104-183.

Order (``load_cuda_backend``):

1. import a pre-installed module named ``barqtrain_cuda`` (_ffi.py:117-121);
2. otherwise, unless an earlier build failed or ``BARQTRAIN_AUTO_BUILD`` is off (:123-127),
   load the in-tree build ``barqtrain_amd/barqtrain_cuda*.so`` -- building it first with
   ``barqtrain_amd.build`` (hipcc for gfx950, g++ for the binding) when it is absent, the
   counterpart of the reference's JIT ``cpp_extension.load`` (:164-178);
3. otherwise ``None``; a failed build is memoised (:180-183) and a later import is still retried.

The module is memoised in ``_CUDA_BACKEND``.  The name keeps the reference's "cuda": on
ROCm PyTorch a GPU tensor's device type is ``cuda``.  The Rust data-pipeline half of the
reference loader (:186-228) belongs to the training path and is not part of this package.
"""

from __future__ import annotations

import importlib
import importlib.util
import os
import shutil
import sys
import warnings
from pathlib import Path
from types import ModuleType
from typing import Optional


def _hip_sources() -> tuple[Path, ...]:
    """The files the in-tree build compiles (its own list, so the two cannot drift apart)."""
    from barqtrain_amd.build import source_files

    return source_files()


_CUDA_BACKEND: Optional[ModuleType] = None
_CUDA_BUILD_FAILED = False


def _env_enabled(name: str, default: str = "1") -> bool:
    """Same parsing as the reference (_ffi.py:36-38): 0/false/no/off disable."""
    value = os.environ.get(name, default).strip().lower()
    return value not in {"0", "false", "no", "off"}


def _detect_cuda_home() -> Optional[str]:
    """GPU toolkit root (reference _ffi.py:41-81).

    ``CUDA_HOME`` / ``CUDA_PATH`` are honoured first, as in the reference; on this stack the
    toolkit is ROCm, found next through ``ROCM_PATH`` / ``ROCM_HOME``, torch's ``ROCM_HOME``,
    ``hipcc`` on ``PATH`` and ``/opt/rocm``.
    """
    for env_name in ("CUDA_HOME", "CUDA_PATH", "ROCM_PATH", "ROCM_HOME"):
        home = os.environ.get(env_name)
        if home and Path(home).exists():
            return home
    try:
        import torch.utils.cpp_extension as cpp_extension

        home = getattr(cpp_extension, "ROCM_HOME", None)
        if home and Path(home).exists():
            return home
    except Exception:
        pass
    hipcc = shutil.which("hipcc")
    if hipcc:
        return str(Path(hipcc).resolve().parents[1])
    if Path("/opt/rocm").exists():
        return "/opt/rocm"
    return None


def _load_in_tree() -> Optional[ModuleType]:
    from barqtrain_amd import build

    path = build.ext_path()
    if not path.exists():
        return None
    import torch  # noqa: F401  -- torch's HIP runtime must be the one the module binds to

    spec = importlib.util.spec_from_file_location("barqtrain_cuda", str(path))
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    sys.modules["barqtrain_cuda"] = module
    return module


def load_cuda_backend() -> Optional[ModuleType]:
    """Return the ``barqtrain_cuda`` module (HIP kernels for gfx950), or ``None``."""
    global _CUDA_BACKEND, _CUDA_BUILD_FAILED
    if _CUDA_BACKEND is not None:
        return _CUDA_BACKEND

    try:
        _CUDA_BACKEND = importlib.import_module("barqtrain_cuda")
        return _CUDA_BACKEND
    except ImportError:
        pass

    if _CUDA_BUILD_FAILED:
        return None
    if not _env_enabled("BARQTRAIN_AUTO_BUILD", "1"):
        return None

    missing = [src for src in _hip_sources() if not src.exists()]
    if missing:
        warnings.warn(
            "BarqTrain HIP sources missing, skipping the GPU backend: "
            + ", ".join(str(p) for p in missing)
        )
        return None

    try:
        module = _load_in_tree()
        if module is None:
            if _detect_cuda_home() is None:
                warnings.warn("BarqTrain HIP build skipped because no ROCm toolkit was found.")
                return None
            from barqtrain_amd import build

            build.build(verbose=_env_enabled("BARQTRAIN_VERBOSE_BUILD", "0"))
            module = _load_in_tree()
        _CUDA_BACKEND = module
        return _CUDA_BACKEND
    except Exception as exc:
        _CUDA_BUILD_FAILED = True
        warnings.warn(f"BarqTrain HIP backend build/load failed: {exc}")
        return None
