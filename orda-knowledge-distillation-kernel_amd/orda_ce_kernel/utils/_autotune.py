"""Launch-configuration policy for gfx950.

The reference picks a Triton ``(BLOCK_SIZE, num_warps)`` pair per mode from
``DEFAULT_CONFIGS`` and can autotune it with ``triton.testing.do_bench``
(reference ``utils/_autotune.py:34-46,94-106,255-340``).  This build has no
Triton and no run-time tuning: the MFMA tile is fixed per engine
(:data:`ENGINE_TILES`), and the launch geometry around it -- tokens per
chunk, scan workgroups, the grad-hidden split-K count -- comes from a fixed
gfx950 table inside ``liborda_ce.so`` (``csrc/launch_table.hpp``, one row
per measured shape, a rule for the rest).  :func:`launch_plan` asks the
library which plan a call would use.  ``KernelConfig.autotune`` is accepted
and ignored.  ``DEFAULT_MAX_FUSED_SIZE`` keeps the reference's value
(``:32``) because it is a public default that is validated as a power of
two.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

__all__ = ["DEFAULT_MAX_FUSED_SIZE", "ENGINE_TILES", "EngineTile", "engine_tile", "launch_plan", "_is_oom_error"]

DEFAULT_MAX_FUSED_SIZE = 65536 // 2


class EngineTile(NamedTuple):
    """Geometry of the MFMA engine that runs the GEMM-shaped kernels."""

    engine: str           # "ring" (4 waves, 5-slot LDS ring) or "two-stage" (8 waves, 2 LDS stages)
    tile_m: int           # workgroup tile rows (vocabulary rows in the scan)
    tile_n: int           # workgroup tile columns (tokens in the scan: student + teacher)
    k_bytes: int          # bytes of K staged per step
    waves: int            # wavefronts per workgroup
    wave_tile: tuple[int, int]
    lds_bytes: int        # LDS per workgroup (one workgroup per CU)
    mfma: str             # MFMA instruction


# The 16-bit kernels of the default schedule (scan, grad W, grad hidden) run
# the ring engine; fp32 and the two-phase schedule the two-stage engine.
ENGINE_TILES: dict[torch.dtype, EngineTile] = {
    torch.bfloat16: EngineTile("ring", 256, 256, 128, 4, (128, 128), 160 * 1024, "v_mfma_f32_32x32x16_bf16"),
    torch.float16: EngineTile("ring", 256, 256, 128, 4, (128, 128), 160 * 1024, "v_mfma_f32_32x32x16_f16"),
    torch.float32: EngineTile("two-stage", 256, 256, 128, 8, (128, 64), 128 * 1024, "v_mfma_f32_32x32x2_f32"),
}


def engine_tile(dtype: torch.dtype) -> EngineTile:
    """The MFMA engine tile for ``dtype``."""
    try:
        return ENGINE_TILES[dtype]
    except KeyError as exc:
        raise ValueError(f"no gfx950 engine for dtype {dtype}") from exc


def launch_plan(problem) -> dict:
    """The launch plan the library picks for an ``orda_problem_t``
    (``_native.Problem``): ``table_entry`` (-1 = rule), ``token_chunk``,
    ``grad_hidden_splits``, ``scan_workgroups``, ...  Host-side only."""
    from .. import _native

    return _native.plan_info(problem)


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
