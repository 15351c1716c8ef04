"""pkv -- MI355X (gfx950) paged-KV decode path behind mlx-one's cache interface.

Compute runs only in libpkv.so (hand-written HIP, C ABI in include/pkv.h);
this package keeps the reference's Python names (``quantize_page``,
``SegmentedPageArena``, ``PersistentPageTable``, ``PagedKVCache``,
``PagedBatchCache``, ``paged_attention``, ``CacheManager``) around it.
"""

__version__ = "0.1.0"
