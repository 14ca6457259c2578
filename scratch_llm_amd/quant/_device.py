"""Device-side plumbing shared by the quant modules: split-K workspaces and the cache of tiled
weights built for the functional linear entry points."""

from __future__ import annotations

import threading
import weakref

import torch

from scratch_llm_amd import _lib

_ws_lock = threading.Lock()
_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """A zero-initialised, 256-byte aligned int32 buffer of at least ``nbytes`` for the current
    stream of ``device``. The linear kernels leave its counter prefix zero after every call, so the
    buffer is reused across calls on that stream; a larger request replaces it with a fresh one."""
    if nbytes <= 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(), _lib.stream_ptr(device))
    with _ws_lock:
        buf = _workspaces.get(key)
        if buf is None or buf.numel() * 4 < nbytes:
            size = max(nbytes, 1 << 20)
            buf = torch.zeros((size + 3) // 4, dtype=torch.int32, device=device)
            _workspaces[key] = buf
    return buf


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
