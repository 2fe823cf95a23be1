"""Import-compatible name for code written against the reference package ``barqtrain``.

``barqtrain.kv_cache``, ``barqtrain._ffi`` and ``barqtrain.patch_models`` are the very module
objects of ``barqtrain_amd`` (so patching ``barqtrain.kv_cache._get_cuda_backend`` patches the
function the cache uses); the top-level names of the reference's KV-cache path are re-exported
(python/barqtrain/__init__.py:26,48,71-72).
"""

import sys as _sys

import barqtrain_amd as _impl
from barqtrain_amd import _ffi, kv_cache, patch_models

for _name, _module in (("_ffi", _ffi), ("kv_cache", kv_cache), ("patch_models", patch_models)):
    _sys.modules[f"{__name__}.{_name}"] = _module

from barqtrain_amd.kv_cache import BarqPagedKVCache, create_paged_kv_cache  # noqa: E402
from barqtrain_amd.patch_models import patch_inference  # noqa: E402

__version__ = _impl.__version__

__all__ = ["BarqPagedKVCache", "create_paged_kv_cache", "patch_inference", "__version__"]
