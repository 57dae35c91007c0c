"""Token-chunk heuristic (reference ``utils/resolver.py:5-62``).

The numbers this module returns are part of the public contract: the
reference's unit tests assert them (``test/unit/test_resolver.py``).  In this
build a "chunk" bounds the backward staging workspace instead of the per-chunk
logits buffer: ``num_chunks`` token chunks of the reference map to
``num_chunks`` vocabulary chunks of the fused kernels (see
``ops._engine.vocab_chunk_for``), so asking for more chunks still means less
memory, which is what the OOM retry in :mod:`.dispatcher` relies on.
"""
from __future__ import annotations

import math

from ._autotune import DEFAULT_MAX_FUSED_SIZE

__all__ = ["DEFAULT_MAX_FUSED_SIZE", "is_power_of_two", "resolve_chunk_size"]


def is_power_of_two(value: int) -> bool:
    """True for 1, 2, 4, ... (reference ``utils/resolver.py:5-6``)."""
    return value > 0 and (value & (value - 1)) == 0


def _is_auto_chunk_size(chunk_size) -> bool:
    """Values that mean "choose for me" (reference ``utils/resolver.py:9-16``)."""
    if chunk_size is None or chunk_size in ("auto", "dynamic"):
        return True
    if isinstance(chunk_size, bool):
        return False
    return isinstance(chunk_size, (int, float)) and chunk_size <= 0


def _chunks_from_raw(raw: float) -> int:
    """Power-of-two chunk count for a memory-pressure score
    (reference ``utils/resolver.py:20-24``): 1 below 1.5, else
    ``2 ** (floor(log2(raw / 1.5)) + 1)``."""
    if raw < 1.5:
        return 1
    return 2 ** (int(math.floor(math.log2(raw / 1.5))) + 1)


def resolve_chunk_size(BT, chunk_size_arg, V=None, max_chunks=None, num_chunks=None):
    """Return ``(chunk_size, num_chunks)`` for ``BT`` rows
    (reference ``utils/resolver.py:28-62``).

    * explicit ``num_chunks``: rows per chunk rounded up, capped at ``BT``;
    * automatic with a vocabulary size: pressure
      ``max((BT/1024) * (V/32768)**2, BT/4096)`` mapped to a power of two and
      clamped to ``BT // 512`` useful chunks (default cap twice that);
    * automatic without ``V``: one chunk;
    * explicit ``chunk_size``: clamped to ``BT``.
    """
    bt = int(BT)
    if bt == 0:
        raise ValueError("BT (batch x sequence length) must be > 0.")

    if num_chunks is not None:
        if not _is_auto_chunk_size(chunk_size_arg):
            raise ValueError("chunk_size and num_chunks are mutually exclusive.")
        wanted = int(num_chunks)
        if wanted < 1:
            raise ValueError(f"num_chunks must be >= 1, got {num_chunks}")
        n = min(wanted, bt)
        if max_chunks is not None and n > int(max_chunks):
            raise ValueError(
                f"num_chunks must be <= max_chunks, got num_chunks={num_chunks}, max_chunks={max_chunks}"
            )
        return -(-bt // n), n

    if _is_auto_chunk_size(chunk_size_arg):
        if V is None:
            return bt, 1
        useful = max(1, bt // 512)
        cap = 2 * useful if max_chunks is None else int(max_chunks)
        pressure = max((bt / 1024.0) * (float(V) / 32768.0) ** 2, bt / 4096.0)
        n = min(cap, useful, _chunks_from_raw(pressure), bt)
        return -(-bt // n), n

    size = min(int(chunk_size_arg), bt)
    return size, -(-bt // size)
