"""barqtrain_amd: BarqTrain's paged KV-cache path, native to MI355X (gfx950).

Python surface (mirrors the reference's ``barqtrain`` package for this path):
``kv_cache.BarqPagedKVCacheLayer``, ``kv_cache.BarqPagedKVCache``, ``create_paged_kv_cache``,
``maybe_prepare_paged_kv_generate_kwargs``, ``paged_kv_supported_for_model``,
``patch_models.patch_inference`` and the loader ``_ffi.load_cuda_backend``.
Native code: ``libbarq_kv.so`` (HIP kernels + C ABI, include/barq_kv.h) and the torch binding
module ``barqtrain_cuda``, both built in-tree by ``barqtrain_amd.build``.
"""

__version__ = "0.1.0"

from barqtrain_amd.kv_cache import (  # noqa: E402
    BarqPagedKVCache,
    BarqPagedKVCacheLayer,
    PagedKVCapacityError,
    PagedKVPoolExhausted,
    create_paged_kv_cache,
    maybe_prepare_paged_kv_generate_kwargs,
    paged_kv_supported_for_model,
)
from barqtrain_amd.patch_models import patch_inference  # noqa: E402

__all__ = [
    "BarqPagedKVCache",
    "BarqPagedKVCacheLayer",
    "PagedKVCapacityError",
    "PagedKVPoolExhausted",
    "create_paged_kv_cache",
    "maybe_prepare_paged_kv_generate_kwargs",
    "paged_kv_supported_for_model",
    "patch_inference",
    "__version__",
]
