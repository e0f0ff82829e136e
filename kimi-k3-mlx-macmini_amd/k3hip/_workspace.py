"""Caller-side workspaces for the persistent kernels.

The C-ABI allocates nothing.  Kernels that synchronise across the grid keep a few
counters at the head of their workspace; those must be zero before the first launch and
the kernels leave them zero afterwards.  Concurrent launches must not share a workspace,
so workspaces are kept per (device, stream).
"""
from __future__ import annotations

import threading

import torch

_lock = threading.Lock()
_cache: dict[tuple, torch.Tensor] = {}


def get(device: torch.device, nbytes: int, tag: str = "") -> torch.Tensor:
    """A zero-initialised uint8 device buffer of at least nbytes for the current stream."""
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index, stream, tag)
    with _lock:
        buf = _cache.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 4096), dtype=torch.uint8, device=device)
            _cache[key] = buf
    return buf


def error_flag(buf: torch.Tensor) -> int:
    """The kernel-side error word (word 2 of the header); nonzero after a barrier timeout."""
    return int(buf[8:12].view(torch.int32).item())


def clear() -> None:
    with _lock:
        _cache.clear()
