"""Device-side plumbing shared by the quant modules: the cache of tiled weights built for the
functional linear entry points."""

from __future__ import annotations

import threading
import weakref

import torch


class TensorKeyedCache:
    """Cache of values derived from tensors.

    An entry is keyed by the source tensors' identity (storage pointer, shape, strides, dtype,
    device) plus the caller's extra key, and stores the version counters it was built from. A
    call after an in-place update (a version counter moved) rebuilds the value and replaces the
    entry, so a tensor updated N times holds one derived value, not N. An entry is dropped when a
    source tensor is garbage-collected; the finalizer is registered once, when the key is
    inserted."""

    def __init__(self) -> None:
        self._d: dict[tuple, tuple[tuple, object]] = {}
        self._lock = threading.Lock()

    @staticmethod
    def _key(tensors: tuple[torch.Tensor, ...], extra: tuple) -> tuple:
        parts = tuple((t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype, str(t.device)) for t in tensors)
        return (parts, extra)

    def get(self, tensors: tuple[torch.Tensor, ...], extra: tuple, build):
        key = self._key(tensors, extra)
        versions = tuple(t._version for t in tensors)
        with self._lock:
            hit = self._d.get(key)
        if hit is not None and hit[0] == versions:
            return hit[1]
        val = build()
        with self._lock:
            fresh = key not in self._d
            self._d[key] = (versions, val)
        if fresh:
            for t in tensors:
                weakref.finalize(t, self._d.pop, key, None)
        return val

    def __len__(self) -> int:
        return len(self._d)

    def clear(self) -> None:
        with self._lock:
            self._d.clear()
