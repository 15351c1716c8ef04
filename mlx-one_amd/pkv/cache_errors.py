"""Exceptions of the paged cache runtime.

The class names and their bases are the reference's
(src/mlx_one/engine/cache_errors.py:1-37): callers at the drop-in boundary
catch them by name, and a full arena is also a ``MemoryError``.
"""


class CacheError(RuntimeError):
    """Root of every error raised by the cache runtime."""


class CacheCapacityError(CacheError, MemoryError):
    """No room under the cache's byte budget (or in its page arena);
    ``retryable`` says whether freeing memory can make the call succeed."""

    def __init__(self, message: str, *, retryable: bool = True) -> None:
        super().__init__(message)
        self.retryable = retryable


class CacheTopologyUnsupported(CacheError):
    """The model's layer layout is one this cache cannot hold."""


class PrefixReuseUnsupported(CacheError):
    """The request cannot take pages from the shared prefix store."""


class KVQuantizationUnsupported(CacheError):
    """The requested key/value precision or its pairing is not offered."""


class CacheCorruptionError(CacheError):
    """Page ownership records disagree (unknown, freed or foreign ids,
    negative counts)."""
