"""Argument checks shared by the mode entry points and autograd Functions.

The messages match the reference's (``ops/tied_teacher.py:594-636`` and the
analogues in ``separate_teacher.py`` / ``precomputed_teacher.py``), because
callers and tests match on them.
"""
from __future__ import annotations

import torch

from ..utils.resolver import is_power_of_two

__all__ = ["check_scalars", "check_common", "check_labels_in_range"]


def check_scalars(*, student_ce_weight, kl_weight, kl_temperature, max_fused_size, teacher_ce_weight=None,
                  reduction=None, max_chunks=None) -> None:
    if student_ce_weight < 0.0:
        raise ValueError(f"student_ce_weight must be >= 0.0, got {student_ce_weight}")
    if kl_weight < 0.0:
        raise ValueError(f"kl_weight must be >= 0.0, got {kl_weight}")
    if kl_temperature <= 0.0:
        raise ValueError(f"kl_temperature must be > 0.0, got {kl_temperature}")
    if teacher_ce_weight is not None and teacher_ce_weight < 0.0:
        raise ValueError(f"teacher_ce_weight must be >= 0.0, got {teacher_ce_weight}")
    if reduction is not None and reduction not in ("mean", "sum"):
        raise ValueError(f"reduction must be 'mean' or 'sum', got {reduction!r}")
    if max_chunks is not None and max_chunks < 1:
        raise ValueError(f"max_chunks must be >= 1, got {max_chunks}")
    if max_fused_size < 1:
        raise ValueError(f"max_fused_size must be >= 1, got {max_fused_size}")
    if not is_power_of_two(int(max_fused_size)):
        raise ValueError(f"max_fused_size must be a power of two, got {max_fused_size}")


def check_common(student_hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor):
    """Shape / dtype checks on the student operands; returns (BT, H, V)."""
    if student_hidden.ndim != 2:
        raise ValueError(f"student_hidden must be 2D, got shape={tuple(student_hidden.shape)}")
    BT, H = student_hidden.shape
    if weight.ndim != 2 or weight.shape[1] != H:
        raise ValueError(f"weight must have shape (V, {H}), got {tuple(weight.shape)}")
    if labels is None:
        raise ValueError("labels is required")
    if labels.shape != (BT,):
        raise ValueError(f"labels must have shape ({BT},), got {tuple(labels.shape)}")
    if labels.dtype != torch.long:
        raise ValueError(f"labels must have dtype torch.long, got {labels.dtype}")
    return BT, H, weight.shape[0]


def check_labels_in_range(labels: torch.Tensor, V: int, ignore_index: int) -> None:
    """Host-synchronising label check of the ``debug`` profile."""
    ok = (labels == ignore_index) | ((labels >= 0) & (labels < V))
    if not bool(ok.all()):
        bad = labels[~ok].tolist()[:5]
        raise ValueError(
            f"labels contains values outside [0, {V}) and not equal to ignore_index={ignore_index}: {bad}"
        )
