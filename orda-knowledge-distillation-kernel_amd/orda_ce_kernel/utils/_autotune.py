"""Launch-configuration policy for gfx950.

The reference picks a Triton ``(BLOCK_SIZE, num_warps)`` pair per mode from
``DEFAULT_CONFIGS`` and can autotune it with ``triton.testing.do_bench``
(reference ``utils/_autotune.py:34-46,94-106,255-340``).  This build has no
Triton and no run-time tuning: the MFMA tiles are fixed in the HIP kernels,
and the launch geometry around them -- tokens per chunk, scan workgroups,
the grad-hidden split-K count -- comes from a fixed gfx950 table inside
``liborda_ce.so`` (``csrc/launch_table.hpp``, one row per measured shape)
and a rule for the shapes it does not list (``make_plan`` in
``csrc/abi.hip``); ``_native.plan_info`` reports the plan a call would use.
``KernelConfig.autotune`` is accepted and ignored.
``DEFAULT_MAX_FUSED_SIZE`` keeps the reference's value (``:32``) because it
is a public default that is validated as a power of two.
"""
from __future__ import annotations

import torch

__all__ = ["DEFAULT_MAX_FUSED_SIZE", "_is_oom_error"]

DEFAULT_MAX_FUSED_SIZE = 65536 // 2


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
