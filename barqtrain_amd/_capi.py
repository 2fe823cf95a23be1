"""ctypes view of the C ABI in include/barq_kv.h (libbarq_kv.so).

This is how a non-torch host (or a test) calls the kernels: plain device pointers, sizes and a
HIP stream handle.  ``torch`` is imported before the library is opened so that the library
binds to the HIP runtime torch already loaded.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path
from typing import Optional

from barqtrain_amd import build

HEADER = build.INCLUDE / "barq_kv.h"

c_i64 = ctypes.c_int64
c_ptr = ctypes.c_void_p


class BarqKVPool(ctypes.Structure):
    """struct barq_kv_pool"""

    _fields_ = [
        ("key_pages", c_ptr),
        ("value_pages", c_ptr),
        ("block_table", c_ptr),
        ("seq_lens", c_ptr),
        ("high_water", c_ptr),
        ("free_pages", c_ptr),
        ("ctrl", c_ptr),
        ("page_shares", c_ptr),
        ("num_pages", c_i64),
        ("max_batch", c_i64),
        ("max_blocks", c_i64),
        ("page_size", c_i64),
        ("kv_heads", c_i64),
        ("head_dim", c_i64),
        ("elem_bytes", c_i64),
    ]


class BarqKVCold(ctypes.Structure):
    """struct barq_kv_cold"""

    _fields_ = [
        ("key_codes", c_ptr),
        ("value_codes", c_ptr),
        ("key_scales", c_ptr),
        ("value_scales", c_ptr),
        ("free_cold", c_ptr),
        ("cold_shares", c_ptr),
        ("num_cold", c_i64),
        ("window", c_i64),
        ("element_type", c_i64),
    ]


_POOL = ctypes.POINTER(BarqKVPool)
_COLD = ctypes.POINTER(BarqKVCold)

_SIGNATURES = {
    "barq_kv_version": (ctypes.c_char_p, []),
    "barq_kv_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "barq_kv_append_dense": (ctypes.c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr] + [c_i64] * 11 + [c_ptr]),
    "barq_kv_pool_reset": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_ptr, c_ptr]),
    "barq_kv_append": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_ptr, c_ptr] + [c_i64] * 5 + [c_ptr]),
    "barq_kv_gather": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_ptr, c_ptr] + [c_i64] * 6 + [c_ptr]),
    "barq_kv_update": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_ptr, c_ptr] + [c_i64] * 5
                       + [c_ptr, c_ptr] + [c_i64] * 5 + [c_ptr]),
    "barq_kv_update_known": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_ptr, c_ptr] + [c_i64] * 5
                             + [c_ptr, c_ptr] + [c_i64] * 4 + [c_ptr, c_ptr, c_i64, c_ptr]),
    "barq_kv_crop": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_i64, c_i64, c_ptr]),
    "barq_kv_free_rows": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_ptr, c_i64, c_ptr]),
    "barq_kv_copy_rows": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), ctypes.POINTER(BarqKVPool), c_ptr, c_i64, c_ptr]),
    "barq_kv_select_rows": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_ptr, c_i64, c_ptr, c_i64, c_ptr]),
    "barq_kv_select_rows_layers": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_i64, c_ptr, c_i64, c_ptr, c_i64,
                                                  c_ptr]),
    "barq_kv_select_workspace_words": (c_i64, [ctypes.POINTER(BarqKVPool), c_i64, c_i64]),
    "barq_kv_attention_workspace_bytes": (c_i64, [ctypes.POINTER(BarqKVPool)] + [c_i64] * 5),
    "barq_kv_decode_attention": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_ptr] + [c_i64] * 6 + [c_ptr]
                                 + [c_i64] * 3 + [ctypes.c_float] + [c_i64] * 3 + [c_ptr, c_i64, c_ptr]),
    "barq_kv_decode_attention_noalloc": (ctypes.c_int, [ctypes.POINTER(BarqKVPool), c_ptr] + [c_i64] * 6 + [c_ptr]
                                         + [c_i64] * 3 + [ctypes.c_float] + [c_i64] * 3 + [c_ptr]),
    "barq_kv_cold_reset": (ctypes.c_int, [_POOL, _COLD, c_ptr]),
    "barq_kv_compress": (ctypes.c_int, [_POOL, _COLD, c_i64, c_ptr]),
    "barq_kv_gather_cold": (ctypes.c_int, [_POOL, _COLD, c_ptr, c_ptr] + [c_i64] * 6 + [c_ptr]),
    "barq_kv_update_cold": (ctypes.c_int, [_POOL, _COLD, c_ptr, c_ptr] + [c_i64] * 5 + [c_ptr, c_ptr]
                            + [c_i64] * 5 + [c_ptr]),
    "barq_kv_free_rows_cold": (ctypes.c_int, [_POOL, _COLD, c_ptr, c_i64, c_ptr]),
    "barq_kv_select_rows_cold_layers": (ctypes.c_int, [_POOL, _COLD, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_ptr]),
    "barq_kv_crop_cold": (ctypes.c_int, [_POOL, _COLD, c_i64, c_i64, c_ptr]),
    "barq_kv_decode_attention_cold": (ctypes.c_int, [_POOL, _COLD, c_ptr] + [c_i64] * 6 + [c_ptr] + [c_i64] * 3
                                      + [ctypes.c_float] + [c_i64] * 3 + [c_ptr, c_i64, c_ptr]),
}

_LIB: Optional[ctypes.CDLL] = None


def header_functions(header: Path = HEADER) -> list[str]:
    """Names of the functions the header declares."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(barq_kv_\w+)\s*\(", text, flags=re.M)))


def load_library(path: Optional[Path] = None) -> ctypes.CDLL:
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    import torch  # noqa: F401  -- share torch's HIP runtime

    lib = ctypes.CDLL(str(path or build.lib_path()))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


class CapiError(RuntimeError):
    pass


def check(rc: int) -> None:
    if rc != 0:
        msg = load_library().barq_kv_status_string(rc).decode()
        raise CapiError(f"barq_kv call failed: {rc} ({msg})")


def pool_struct(pool) -> BarqKVPool:
    """struct barq_kv_pool for a barqtrain_amd.paged.PagePool."""
    return BarqKVPool(
        pool.key_pages.data_ptr(), pool.value_pages.data_ptr(), pool.block_table.data_ptr(),
        pool.seq_lens.data_ptr(), pool.high_water.data_ptr(), pool.free_pages.data_ptr(),
        pool.ctrl.data_ptr(), pool.page_shares.data_ptr(), pool.num_pages, pool.max_batch,
        pool.max_blocks, pool.page_size,
        pool.kv_heads, pool.head_dim, pool.key_pages.element_size(),
    )


def current_stream() -> int:
    import torch

    return torch.cuda.current_stream().cuda_stream
