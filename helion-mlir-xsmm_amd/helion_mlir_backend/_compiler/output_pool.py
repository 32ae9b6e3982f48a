"""Fresh output tensors of the kernels: an HBM buffer pool on the GPU.

The reference pools large CPU outputs in mmap'd blocks reused without page
faults (``_compiler/output_pool.py:243-329``). On a ROCm device the same job --
reuse device blocks by size so a steady stream of calls allocates nothing new
-- is done by torch's stream-ordered caching allocator, which this module
fronts with the reference's API: ``empty``, ``empty_like``,
``set_output_pool``, ``release`` and ``output_pool_stats``. Blocks are kept
per stream, so a buffer freed by one call is reused by the next call on that
stream without synchronization.
"""

from __future__ import annotations

import os
import threading

import torch

OUTPUT_POOL_ENV = "HELION_MLIR_OUTPUT_POOL_BYTES"
DEFAULT_MAX_BYTES = 64 << 30
MIN_BYTES = 4 << 20

_lock = threading.Lock()
_requests = [0]


def _default_max_bytes() -> int:
    value = os.environ.get(OUTPUT_POOL_ENV, "").strip()
    if not value:
        return DEFAULT_MAX_BYTES
    try:
        return max(0, int(value))
    except ValueError:
        return DEFAULT_MAX_BYTES


_max_bytes = _default_max_bytes()


def empty(sizes: tuple[int, ...] | list[int], *, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """``torch.empty(sizes, dtype=dtype, device=device)``; device tensors come
    from the caching allocator's free blocks when one fits."""
    if torch.device(device).type == "cuda":
        _requests[0] += 1
    return torch.empty(tuple(sizes), dtype=dtype, device=device)


def empty_like(x: torch.Tensor, *, dtype: torch.dtype | None = None) -> torch.Tensor:
    """A contiguous ``torch.empty`` of ``x``'s shape (and device)."""
    return empty(tuple(x.shape), dtype=x.dtype if dtype is None else dtype, device=x.device)


def set_output_pool(max_bytes: int) -> None:
    """Keep at most ``max_bytes`` of free device blocks: beyond it the cached
    blocks are returned to the device (0 returns them all now)."""
    global _max_bytes
    with _lock:
        _max_bytes = max(0, int(max_bytes))
    _settle()


def _settle() -> None:
    if not torch.cuda.is_available():
        return
    free = torch.cuda.memory_reserved() - torch.cuda.memory_allocated()
    if free > _max_bytes:
        torch.cuda.empty_cache()


def release() -> None:
    """Return every free cached device block now."""
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


def enabled() -> bool:
    return _max_bytes > 0


def output_pool_stats() -> dict[str, int]:
    """Pool counters in the reference's keys: ``hits`` (outputs served from a
    cached block), ``misses`` (new device allocations), ``free_blocks``,
    ``free_bytes`` and ``max_bytes``."""
    stats = torch.cuda.memory_stats() if torch.cuda.is_available() else {}
    allocs = int(stats.get("allocation.all.allocated", 0))
    segments = int(stats.get("segment.all.allocated", 0))
    reserved = int(stats.get("reserved_bytes.all.current", 0))
    active = int(stats.get("active_bytes.all.current", 0))
    return {
        "hits": max(0, allocs - segments),
        "misses": segments,
        "free_blocks": int(stats.get("inactive_split.all.current", 0)),
        "free_bytes": max(0, reserved - active),
        "max_bytes": _max_bytes,
        "requests": _requests[0],
    }
