"""Separate teacher: teacher logits come from its own ``(hidden_t, W_t)``.

Mirrors the reference's ``ops/separate_teacher.py`` interface:
``SeparateStudentCEFunction`` (``:488-740``, teacher CE off, no teacher
gradients), ``SeparateFullCEFunction`` (``:743-1020``, teacher CE on, with
``hidden_t`` / ``W_t`` gradients) and ``separate_distillation_loss``
(``:1024-1121``), which picks the full Function when
``teacher_ce_weight > 0`` (``:1102``).  Same ``.apply`` order, defaults and
messages, plus one optional trailing ``divergence`` argument.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from .._runtime import default_compute_dtype
from ..utils.resolver import DEFAULT_MAX_FUSED_SIZE
from ._checks import check_common, check_labels_in_range, check_scalars
from ._engine import (FusedCall, cast_to, fused_backward, fused_forward, grads_in_forward, require_native,
                      token_chunk_for, vocab_chunk_for)

__all__ = ["SeparateFullCEFunction", "SeparateStudentCEFunction", "separate_distillation_loss"]


def _separate_call(student_hidden, teacher_hidden, weight, teacher_weight, labels, *, student_ce_weight,
                   ignore_index, reduction, chunk_size, kl_weight, kl_temperature, teacher_ce_weight, max_chunks,
                   divergence, full, use_fp32_accum=None):
    BT = student_hidden.shape[0]
    V = weight.shape[0]
    dtype = default_compute_dtype(weight, teacher_weight, student_hidden, teacher_hidden)
    need = (student_hidden.requires_grad, weight.requires_grad, full and teacher_hidden.requires_grad,
            full and teacher_weight.requires_grad)
    return FusedCall(
        mode="separate",
        student_hidden=student_hidden.contiguous().to(dtype),
        weight=weight.contiguous().to(dtype),
        labels=labels.contiguous(),
        teacher_hidden=teacher_hidden.contiguous().to(dtype),
        teacher_weight=teacher_weight.contiguous().to(dtype),
        teacher_logits=None,
        student_ce_weight=float(student_ce_weight),
        teacher_ce_weight=float(teacher_ce_weight),
        kl_weight=float(kl_weight),
        kl_temperature=float(kl_temperature),
        ignore_index=int(ignore_index),
        reduction=reduction,
        vocab_chunk=vocab_chunk_for(BT, V, chunk_size, max_chunks),
        divergence=divergence,
        compute_teacher_ce=full,
        need_grad_student_hidden=need[0],
        need_grad_weight=need[1],
        need_grad_teacher_hidden=need[2],
        need_grad_teacher_weight=need[3],
        grads_in_forward=grads_in_forward("separate", use_fp32_accum, divergence, any(need)),
        token_chunk=token_chunk_for(chunk_size),
    )


class SeparateStudentCEFunction(torch.autograd.Function):
    @staticmethod
    def forward(
        ctx,
        student_hidden,
        teacher_hidden,
        weight,
        teacher_weight,
        labels,
        student_ce_weight=1.0,
        ignore_index=-100,
        reduction="mean",
        chunk_size=None,
        use_fp32_accum=None,
        kl_weight=0.0,
        kl_temperature=1.0,
        teacher_ce_weight=0.0,
        max_chunks=None,
        max_fused_size=DEFAULT_MAX_FUSED_SIZE,
        autotune=False,
        validate_labels=True,
        divergence=None,
    ):
        if float(teacher_ce_weight) != 0.0:
            raise ValueError("SeparateStudentCEFunction requires teacher_ce_weight=0.0")
        check_scalars(
            student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
            max_fused_size=max_fused_size,
        )
        require_native("separate_distillation_loss")
        if labels.dtype != torch.long:
            raise ValueError(f"labels must have dtype torch.long, got {labels.dtype}")
        ctx.compute_grad = student_hidden.requires_grad or weight.requires_grad
        ctx.dtypes = (student_hidden.dtype, weight.dtype)
        call = _separate_call(
            student_hidden, teacher_hidden, weight, teacher_weight, labels, student_ce_weight=student_ce_weight,
            ignore_index=ignore_index, reduction=reduction, chunk_size=chunk_size, kl_weight=kl_weight,
            kl_temperature=kl_temperature, teacher_ce_weight=0.0, max_chunks=max_chunks, divergence=divergence,
            full=False, use_fp32_accum=use_fp32_accum,
        )
        loss, ce_s, ce_t, kl = fused_forward(ctx, call)
        ctx.mark_non_differentiable(ce_s, ce_t, kl)
        return loss, ce_s, ce_t, kl

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output, _gs=None, _gt=None, _gkl=None):
        if grad_output is None or not ctx.compute_grad:
            return (None,) * 18
        g_hs, g_w, _, _ = fused_backward(ctx, grad_output)
        d_hs, d_w = ctx.dtypes
        return (cast_to(g_hs, d_hs), None, cast_to(g_w, d_w)) + (None,) * 15


class SeparateFullCEFunction(torch.autograd.Function):
    @staticmethod
    def forward(
        ctx,
        student_hidden,
        teacher_hidden,
        weight,
        teacher_weight,
        labels,
        student_ce_weight=1.0,
        ignore_index=-100,
        reduction="mean",
        chunk_size=None,
        use_fp32_accum=None,
        kl_weight=0.0,
        kl_temperature=1.0,
        teacher_ce_weight=1.0,
        max_chunks=None,
        max_fused_size=DEFAULT_MAX_FUSED_SIZE,
        autotune=False,
        validate_labels=True,
        divergence=None,
    ):
        if float(teacher_ce_weight) <= 0.0:
            raise ValueError("SeparateFullCEFunction requires teacher_ce_weight > 0.0")
        check_scalars(
            student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
            max_fused_size=max_fused_size,
        )
        require_native("separate_distillation_loss")
        if labels.dtype != torch.long:
            raise ValueError(f"labels must have dtype torch.long, got {labels.dtype}")
        ctx.compute_grad = (
            student_hidden.requires_grad or teacher_hidden.requires_grad
            or weight.requires_grad or teacher_weight.requires_grad
        )
        ctx.dtypes = (student_hidden.dtype, teacher_hidden.dtype, weight.dtype, teacher_weight.dtype)
        call = _separate_call(
            student_hidden, teacher_hidden, weight, teacher_weight, labels, student_ce_weight=student_ce_weight,
            ignore_index=ignore_index, reduction=reduction, chunk_size=chunk_size, kl_weight=kl_weight,
            kl_temperature=kl_temperature, teacher_ce_weight=teacher_ce_weight, max_chunks=max_chunks,
            divergence=divergence, full=True, use_fp32_accum=use_fp32_accum,
        )
        loss, ce_s, ce_t, kl = fused_forward(ctx, call)
        ctx.mark_non_differentiable(ce_s, ce_t, kl)
        return loss, ce_s, ce_t, kl

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output, _gs=None, _gt=None, _gkl=None):
        if grad_output is None or not ctx.compute_grad:
            return (None,) * 18
        g_hs, g_w, g_ht, g_wt = fused_backward(ctx, grad_output)
        d_hs, d_ht, d_w, d_wt = ctx.dtypes
        return (cast_to(g_hs, d_hs), cast_to(g_ht, d_ht), cast_to(g_w, d_w), cast_to(g_wt, d_wt)) + (None,) * 14


@torch._dynamo.disable
def separate_distillation_loss(
    student_hidden: torch.Tensor,
    teacher_hidden: torch.Tensor | None,
    weight: torch.Tensor,
    teacher_weight: torch.Tensor | None,
    labels: torch.Tensor,
    student_ce_weight: float = 1.0,
    ignore_index: int = -100,
    reduction: str = "mean",
    chunk_size=None,
    use_fp32_accum: bool | None = None,
    kl_weight: float = 0.0,
    kl_temperature: float = 1.0,
    teacher_ce_weight: float | None = None,
    max_chunks: int | None = None,
    max_fused_size: int = DEFAULT_MAX_FUSED_SIZE,
    autotune: bool = False,
    validate_labels: bool = True,
    divergence=None,
):
    """Separate-teacher loss on the HIP path; ``teacher_ce_weight`` defaults
    to 0.0 (reference ``ops/separate_teacher.py:559``)."""
    w_t = 0.0 if teacher_ce_weight is None else float(teacher_ce_weight)
    require_native("separate_distillation_loss")
    BT, H, V = check_common(student_hidden, weight, labels)
    if teacher_hidden is None:
        raise ValueError("separate_distillation_loss requires teacher_hidden")
    if teacher_hidden.ndim != 2 or teacher_hidden.shape[0] != BT:
        raise ValueError(
            f"teacher_hidden must have shape (BT, teacher_hidden_dim), got {tuple(teacher_hidden.shape)}"
        )
    Ht = teacher_hidden.shape[1]
    if teacher_weight is None:
        raise ValueError("separate_distillation_loss requires teacher_weight")
    if teacher_weight.shape != (V, Ht):
        raise ValueError(f"teacher_weight must have shape ({V}, {Ht}), got {tuple(teacher_weight.shape)}")
    check_scalars(
        student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
        max_fused_size=max_fused_size, teacher_ce_weight=w_t, reduction=reduction, max_chunks=max_chunks,
    )
    device = student_hidden.device
    if device.type != "cuda":
        raise ValueError(f"tensors must be CUDA/HIP tensors, got device={device}")
    if labels.device != device or weight.device != device:
        raise ValueError("labels and weight must be on the same device as student_hidden")
    if teacher_hidden.device != device or teacher_weight.device != device:
        raise ValueError("teacher_hidden and teacher_weight must be on the same device as student_hidden")
    if validate_labels:
        check_labels_in_range(labels, V, ignore_index)
    function = SeparateFullCEFunction if w_t > 0.0 else SeparateStudentCEFunction
    return function.apply(
        student_hidden, teacher_hidden, weight, teacher_weight, labels, student_ce_weight, ignore_index,
        reduction, chunk_size, use_fp32_accum, kl_weight, kl_temperature, w_t, max_chunks, max_fused_size,
        autotune, validate_labels, divergence,
    )
