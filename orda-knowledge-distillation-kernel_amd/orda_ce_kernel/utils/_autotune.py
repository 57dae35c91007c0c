"""Launch-configuration policy for gfx950.

The reference picks a Triton ``(BLOCK_SIZE, num_warps)`` pair per mode and can
autotune it with ``triton.testing.do_bench`` (reference
``utils/_autotune.py:19-340``).  This build has no Triton: every kernel runs
the same MFMA tile, and the few knobs that remain are fixed per shape in
:data:`GFX950_TILES`.  ``KernelConfig.autotune`` is accepted and ignored.
``DEFAULT_MAX_FUSED_SIZE`` keeps the reference's value (``:32``) because it is
a public default that is validated as a power of two.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

__all__ = ["DEFAULT_MAX_FUSED_SIZE", "GFX950_TILES", "TileConfig", "tile_config", "_is_oom_error"]

DEFAULT_MAX_FUSED_SIZE = 65536 // 2


class TileConfig(NamedTuple):
    """Geometry of the fused MFMA tile (all kernels of ``liborda_ce.so``)."""

    vocab_rows: int       # vocabulary rows per workgroup tile (MFMA M)
    token_rows: int       # tokens per workgroup tile (MFMA N, student + teacher halves)
    k_bytes: int          # bytes of the hidden dimension staged per K step
    waves: int            # wavefronts per workgroup
    mfma: str             # MFMA instruction of the bf16 / fp16 path


# One entry per compute dtype: the tile is fixed in the library; the table
# documents it and is what tests compare against.
GFX950_TILES: dict[torch.dtype, TileConfig] = {
    torch.bfloat16: TileConfig(256, 128, 128, 4, "v_mfma_f32_32x32x16_bf16"),
    torch.float16: TileConfig(256, 128, 128, 4, "v_mfma_f32_32x32x16_f16"),
    torch.float32: TileConfig(256, 128, 128, 4, "v_mfma_f32_32x32x2_f32"),
}


def tile_config(dtype: torch.dtype) -> TileConfig:
    """Fixed gfx950 tile for ``dtype``."""
    try:
        return GFX950_TILES[dtype]
    except KeyError as exc:
        raise ValueError(f"no gfx950 tile for dtype {dtype}") from exc


def _is_oom_error(exc) -> bool:
    """Device out-of-memory, recognised by type or message
    (reference ``utils/_autotune.py`` / ``utils/dispatcher.py:13-23``)."""
    oom_type = getattr(torch.cuda, "OutOfMemoryError", None)
    if oom_type is not None and isinstance(exc, oom_type):
        return True
    text = str(exc).lower()
    return any(
        marker in text
        for marker in ("cuda out of memory", "cuda error: out of memory", "hip out of memory", "hip error: out of memory")
    )
