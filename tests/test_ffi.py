"""Loader contract of the reference's python/barqtrain/_ffi.py (tests/test_ffi.py:12-39 of
BarqTrain): toolkit-home detection prefers the environment, and a missing backend is retried
after a late install even when auto-build is off."""

import types

from barqtrain import _ffi


def test_toolkit_home_prefers_environment(monkeypatch, tmp_path):
    home = tmp_path / "toolkit"
    home.mkdir()
    monkeypatch.setenv("CUDA_HOME", str(home))
    assert _ffi._detect_cuda_home() == str(home)


def test_rocm_home_from_environment(monkeypatch, tmp_path):
    home = tmp_path / "rocm"
    home.mkdir()
    for name in ("CUDA_HOME", "CUDA_PATH"):
        monkeypatch.delenv(name, raising=False)
    monkeypatch.setenv("ROCM_PATH", str(home))
    assert _ffi._detect_cuda_home() == str(home)


def test_backend_import_retried_after_late_install(monkeypatch):
    module = types.SimpleNamespace(__name__="barqtrain_cuda")
    real_import = _ffi.importlib.import_module
    attempts = {"n": 0}

    def fake_import(name):
        if name == "barqtrain_cuda":
            attempts["n"] += 1
            if attempts["n"] == 1:
                raise ImportError("not installed yet")
            return module
        return real_import(name)

    monkeypatch.setattr(_ffi, "_CUDA_BACKEND", None)
    monkeypatch.setattr(_ffi, "_CUDA_BUILD_FAILED", False)
    monkeypatch.setattr(_ffi, "_env_enabled", lambda name, default="1": False)
    monkeypatch.setattr(_ffi.importlib, "import_module", fake_import)
    assert _ffi.load_cuda_backend() is None
    assert _ffi.load_cuda_backend() is module


def test_failed_build_is_memoised(monkeypatch):
    def no_module(name):
        raise ImportError(name)

    monkeypatch.setattr(_ffi, "_CUDA_BACKEND", None)
    monkeypatch.setattr(_ffi, "_CUDA_BUILD_FAILED", True)
    monkeypatch.setattr(_ffi.importlib, "import_module", no_module)
    assert _ffi.load_cuda_backend() is None


def test_env_switch_parsing(monkeypatch):
    for off in ("0", "false", "No", " off "):
        monkeypatch.setenv("BARQTRAIN_X", off)
        assert _ffi._env_enabled("BARQTRAIN_X") is False
    monkeypatch.setenv("BARQTRAIN_X", "1")
    assert _ffi._env_enabled("BARQTRAIN_X") is True
    monkeypatch.delenv("BARQTRAIN_X")
    assert _ffi._env_enabled("BARQTRAIN_X", "0") is False


def test_in_tree_module_loads_without_gpu(monkeypatch):
    """With the in-tree build present, the loader returns the module on a CPU-only host."""
    from barqtrain_amd import build

    if not build.is_built():
        build.build()
    monkeypatch.setattr(_ffi, "_CUDA_BACKEND", None)
    monkeypatch.setattr(_ffi, "_CUDA_BUILD_FAILED", False)
    monkeypatch.delenv("BARQTRAIN_AUTO_BUILD", raising=False)
    mod = _ffi.load_cuda_backend()
    assert mod is not None and hasattr(mod, "paged_kv_append_") and hasattr(mod, "pool_update_")
