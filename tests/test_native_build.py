"""The native library without a GPU: it loads, exports exactly what include/barq_kv.h declares,
the torch binding module loads, and the kernels' invariant-divisor arithmetic is exact."""

import ctypes
import subprocess

import pytest

from barqtrain_amd import _capi, build


@pytest.fixture(scope="module")
def built():
    if not build.is_built():
        build.build()
    return True


def test_library_exports_every_header_function(built):
    lib = ctypes.CDLL(str(build.lib_path()))
    declared = _capi.header_functions()
    assert len(declared) == 25
    for name in declared:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(build.lib_path())], capture_output=True, text=True).stdout
    exported = sorted({line.split()[-1] for line in out.splitlines() if " T barq_kv_" in line})
    assert exported == declared


def test_ctypes_signatures_cover_header(built):
    assert sorted(_capi._SIGNATURES) == _capi.header_functions()
    lib = _capi.load_library()
    assert lib.barq_kv_version().decode().endswith("gfx950")
    assert lib.barq_kv_status_string(1).decode().startswith("invalid")


def test_invalid_arguments_rejected_without_gpu(built):
    """Argument validation happens on the host before any HIP call."""
    lib = _capi.load_library()
    assert lib.barq_kv_pool_reset(None, None, None) == 1
    # the known-state update checks the caller's state before anything else
    assert lib.barq_kv_update_known(None, None, None, 1, 1, 0, 0, 0, None, None, 1, 0, 0, 0, None, None, 0, None) == 1
    assert lib.barq_kv_update_known(None, None, None, 0, 1, 0, 0, 0, None, None, 1, 0, 0, 0, None, None, -1, None) == 1
    pool = _capi.BarqKVPool()
    assert lib.barq_kv_append(ctypes.byref(pool), None, None, 1, 1, 0, 0, 0, None) == 1
    assert lib.barq_kv_append_dense(None, None, None, None, None, 1, 1, 1, 1, 1, 1, 1, 2, 0, 0, 0, None) == 1


def _fake_pool():
    """A pool descriptor with plausible geometry and non-null, never-dereferenced addresses:
    only calls that return before any launch may be made with it."""
    addr = 0x7F0000000000
    return _capi.BarqKVPool(addr, addr + 2**30, addr + 2**31, addr + 2**31 + 2**20,
                            addr + 2**31 + 2**21, addr + 2**31 + 2**22, addr + 2**31 + 2**23,
                            addr + 2**31 + 2**24, 64, 4, 8, 16, 8, 128, 2)


def test_empty_work_returns_ok_before_any_launch(built):
    """No-op calls (no rows, no tokens and no output extent) succeed whatever the pointers,
    including the null data pointer of an empty output tensor."""
    lib = _capi.load_library()
    p = ctypes.byref(_fake_pool())
    assert lib.barq_kv_update(p, None, None, 0, 3, 0, 0, 0, None, None, 0, 0, 0, 0, 0, None) == 0
    assert lib.barq_kv_gather(p, None, None, 2, 0, 0, 0, 0, 0, None) == 0
    assert lib.barq_kv_gather(p, None, None, 0, 5, 0, 0, 0, 0, None) == 0
    assert lib.barq_kv_append(p, None, None, 3, 0, 0, 0, 0, None) == 0
    assert lib.barq_kv_crop(p, 0, 5, None) == 0
    assert lib.barq_kv_free_rows(p, None, 0, None) == 0


def test_bad_geometry_rejected_before_any_launch(built):
    lib = _capi.load_library()
    p = ctypes.byref(_fake_pool())
    a = 0x7F1000000000
    # an update whose output extent cannot hold the new tokens
    assert lib.barq_kv_update(p, a, a, 2, 5, 0, 0, 0, a, a, 4, 0, 0, 0, 0, None) == 1
    # output extent beyond the capacity (8 blocks x 16 = 128 positions)
    assert lib.barq_kv_gather(p, a, a, 2, 129, 0, 0, 0, 0, None) == 1
    # more rows than the pool holds, negative sizes, unknown flags
    assert lib.barq_kv_append(p, a, a, 5, 1, 0, 0, 0, None) == 1
    assert lib.barq_kv_append(p, a, a, 1, -1, 0, 0, 0, None) == 1
    assert lib.barq_kv_gather(p, a, a, 1, 4, 0, 0, 0, 64, None) == 1
    # missing data pointers when there is work
    assert lib.barq_kv_append(p, None, a, 1, 1, 0, 0, 0, None) == 1
    assert lib.barq_kv_gather(p, None, a, 1, 4, 0, 0, 0, 0, None) == 1
    # ctrl words must be 256-byte aligned
    bad = _fake_pool()
    bad.ctrl += 4
    assert lib.barq_kv_pool_reset(ctypes.byref(bad), None, None) == 1


def header_define(name: str) -> int:
    """Value of an integer #define of include/barq_kv.h, expressions of earlier defines allowed."""
    import re

    defs = {}
    for m in re.finditer(r"^#define (BARQ_KV_\w+) (.+?)(?:\s*/\*.*)?$", _capi.HEADER.read_text(), flags=re.M):
        expr = m.group(2).strip()
        for k, v in defs.items():
            expr = re.sub(rf"\b{k}\b", str(v), expr)
        try:
            defs[m.group(1)] = int(eval(expr, {"__builtins__": {}}))
        except Exception:
            pass
    return defs[name]


def test_torch_binding_module_surface(built):
    import importlib.util

    import torch  # noqa: F401

    spec = importlib.util.spec_from_file_location("barqtrain_cuda", str(build.ext_path()))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    for name in ("paged_kv_append_", "pool_reset_", "pool_append_", "pool_gather", "pool_update_",
                 "pool_crop_", "pool_free_rows_", "pool_copy_rows_"):
        assert callable(getattr(mod, name)), name
    from barqtrain_amd import paged

    assert mod.CTRL_WORDS == paged.CTRL_WORDS == header_define("BARQ_KV_CTRL_WORDS")


def test_loader_lists_every_native_source():
    """The loader's missing-source check names exactly the files the build reads."""
    from barqtrain_amd import _ffi

    listed = {p.resolve() for p in _ffi._hip_sources()}
    on_disk = {p.resolve() for p in build.CSRC.iterdir() if p.suffix in (".hip", ".h", ".cpp")}
    on_disk |= {p.resolve() for p in build.INCLUDE.glob("*.h")}
    assert listed == on_disk


def test_library_is_gfx950_only(built, tmp_path):
    """The fatbin embedded in the library holds one device code object, for gfx950."""
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", str(build.lib_path()), str(fatbin)],
                   check=True)
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o", f"--input={fatbin}"],
                         capture_output=True, text=True, check=True).stdout.split()
    devices = [t for t in out if "amdgcn" in t]
    assert devices == ["hipv4-amdgcn-amd-amdhsa--gfx950"], out


FASTDIV_CHECK = r"""
#include <cstdio>
#include <cstdint>
#include "fastdiv.h"
int main() {
  const uint32_t ds[] = {1, 2, 3, 5, 7, 10, 16, 24, 48, 64, 80, 96, 127, 128, 160, 255, 256, 257, 516, 1000,
                         1026, 4097, 65535, 65536, 65537, 1u << 20, (1u << 20) + 1, 2147483647u, 2147483648u,
                         3000000019u, 4294967295u};
  uint64_t bad = 0, n_checked = 0;
  for (uint32_t d : ds) {
    FastDiv f = FastDiv::make(d);
    uint32_t probes[] = {0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d, 4294967295u, 4294967294u, 2147483647u, 2147483648u};
    for (uint32_t n : probes) { n_checked++; if (f.div(n) != n / d) bad++; }
    for (uint64_t n = 0; n < 300000; ++n) { n_checked++; if (f.div((uint32_t)n) != (uint32_t)n / d) bad++; }
    uint64_t x = 0x9E3779B97F4A7C15ull ^ d;
    for (int i = 0; i < 300000; ++i) {
      x ^= x << 13; x ^= x >> 7; x ^= x << 17;
      uint32_t n = (uint32_t)x; n_checked++;
      if (f.div(n) != n / d) bad++;
    }
  }
  printf("%llu %llu\n", (unsigned long long)bad, (unsigned long long)n_checked);
  return bad != 0;
}
"""


def test_fastdiv_is_exact(tmp_path):
    src = tmp_path / "fd.cpp"
    src.write_text(FASTDIV_CHECK)
    exe = tmp_path / "fd"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{build.CSRC}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    bad, checked = map(int, out.stdout.split())
    assert bad == 0 and checked > 10_000_000
