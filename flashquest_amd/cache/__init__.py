"""Persistent quantised KV caches (src/flashquest/cache/): preallocated
per-layer buffers in the packed layout the decode kernels read."""
from .persistent_int4 import PersistentInt4KVCache
from .persistent_int8 import PersistentInt8KVCache
from .persistent_turbo import PersistentTurboKVCache

__all__ = ["PersistentInt4KVCache", "PersistentInt8KVCache", "PersistentTurboKVCache"]
