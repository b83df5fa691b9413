"""MI355X-native paged KV-cache path of the aojsd/GPU_Offloading MoE engine.

Host side (PyTorch-ROCm, this package) keeps the engine's cache-manager API;
every kernel is hand-written HIP for gfx950 in ``csrc/`` and reached through
the C ABI of ``include/kvc.h`` (``lib/libkvc.so``).

Modules:
  ops        reshape_and_cache_flash, gather_kv, merge_attention_states,
             compute_slot_mapping, copy_page_indices, block gather/scatter, swap
  decode     BatchDecodeWithPagedKVCacheWrapper (plan / run)
  kv_cache   PagedKVCache: caches, block table, page pool, step setup, swap
  allocator  PageAllocator protocol, PagePool, pages_needed
  workloads  seeded synthetic workloads of the benchmark configurations
  build      compiles libkvc.so
"""
from .allocator import PageAllocator, PagePool, pages_needed  # noqa: F401

__version__ = "0.1.0"


def __getattr__(name):
    # Lazy imports keep `import gpu_offloading_amd` cheap (no torch) for the
    # allocator-only users, e.g. CPU scheduler tests.
    if name in ("ops", "decode", "kv_cache", "workloads", "build", "_lib"):
        import importlib
        return importlib.import_module(f".{name}", __name__)
    if name == "PagedKVCache":
        from .kv_cache import PagedKVCache
        return PagedKVCache
    if name == "BatchDecodeWithPagedKVCacheWrapper":
        from .decode import BatchDecodeWithPagedKVCacheWrapper
        return BatchDecodeWithPagedKVCacheWrapper
    raise AttributeError(name)
