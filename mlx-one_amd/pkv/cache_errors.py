"""Cache runtime failures, as in the reference (src/mlx_one/engine/cache_errors.py:1-37)."""


class CacheError(RuntimeError):
    """Base class for cache-runtime failures."""


class CacheCapacityError(CacheError, MemoryError):
    """The configured cache budget cannot satisfy an allocation."""

    def __init__(self, message: str, *, retryable: bool = True) -> None:
        super().__init__(message)
        self.retryable = retryable


class CacheTopologyUnsupported(CacheError):
    """The cache plan cannot serve the requested layer topology."""


class PrefixReuseUnsupported(CacheError):
    """Cached prefixes cannot be reused for this request."""


class KVQuantizationUnsupported(CacheError):
    """A requested KV quantization/backend combination is unsupported."""


class CacheCorruptionError(CacheError):
    """Internal block or reference metadata is inconsistent."""
