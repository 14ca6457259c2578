"""Device-side plumbing shared by the quant modules: the cache of tiled weights built for the
functional linear entry points."""

from __future__ import annotations

import threading
import weakref

import torch


class TensorKeyedCache:
    """Cache of values derived from tensors, keyed by storage pointer, version counter and shape.

    An entry is dropped when any source tensor is garbage-collected, and is rebuilt when a source
    tensor is modified in place (its version counter moves)."""

    def __init__(self) -> None:
        self._d: dict[tuple, object] = {}
        self._lock = threading.Lock()

    @staticmethod
    def _key(tensors: tuple[torch.Tensor, ...], extra: tuple) -> tuple:
        parts = []
        for t in tensors:
            parts.append((t.data_ptr(), t._version, tuple(t.shape), tuple(t.stride()), t.dtype, str(t.device)))
        return (tuple(parts), extra)

    def get(self, tensors: tuple[torch.Tensor, ...], extra: tuple, build):
        key = self._key(tensors, extra)
        with self._lock:
            hit = self._d.get(key)
        if hit is not None:
            return hit
        val = build()
        with self._lock:
            self._d[key] = val
        for t in tensors:
            weakref.finalize(t, self._d.pop, key, None)
        return val

    def clear(self) -> None:
        with self._lock:
            self._d.clear()
