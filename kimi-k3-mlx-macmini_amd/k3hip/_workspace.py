"""Caller-side workspaces for the multi-launch kernels.

The C-ABI allocates nothing.  Intermediate records (the expert's act vector, router
records, split-T partials, grouping lists) live in a workspace the caller passes in.
Concurrent launches must not share a workspace, so workspaces are kept per (device,
stream, user).
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


def clear() -> None:
    with _lock:
        _cache.clear()
