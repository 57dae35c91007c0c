"""Tied teacher: student and teacher share the LM-head weight ``W``.

Mirrors the reference's ``ops/tied_teacher.py`` interface
(``TiedCEFunction`` ``:287-564``, ``tied_distillation_loss`` ``:568-655``):
same positional ``.apply`` order, defaults, checks and messages, plus one
optional trailing ``divergence`` argument.  The arithmetic runs in the fused
HIP kernels of ``liborda_ce.so`` (:mod:`._engine`).

Loss (per non-ignored row, then mean or sum):
``w_s CE(x_s) + w_t CE(x_t) + w_kl T^2 D(softmax(x_t/T) || softmax(x_s/T))``
with ``x_s = h_s W^T``, ``x_t = h_t W^T``; the divergence gradient reaches the
student only (the teacher distribution is detached), the teacher CE gradient
reaches ``h_t`` and ``W``.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from .._runtime import default_compute_dtype
from ..utils.resolver import DEFAULT_MAX_FUSED_SIZE
from ._checks import check_common, check_labels_in_range, check_scalars
from ._engine import (FusedCall, cast_to, fused_backward, fused_forward, grads_in_forward, require_native,
                      token_chunk_for, vocab_chunk_for)

__all__ = ["TiedCEFunction", "tied_distillation_loss"]


class TiedCEFunction(torch.autograd.Function):
    @staticmethod
    def forward(
        ctx,
        student_hidden,
        teacher_hidden,
        weight,
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
        require_native("tied_distillation_loss")
        check_scalars(
            student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
            max_fused_size=max_fused_size,
        )
        if labels.dtype != torch.long:
            raise ValueError(f"labels must have dtype torch.long, got {labels.dtype}")
        BT = student_hidden.shape[0]
        V = weight.shape[0]
        ctx.compute_grad = student_hidden.requires_grad or teacher_hidden.requires_grad or weight.requires_grad
        ctx.dtypes = (student_hidden.dtype, teacher_hidden.dtype, weight.dtype)
        dtype = default_compute_dtype(weight, student_hidden, teacher_hidden)
        call = FusedCall(
            mode="tied",
            student_hidden=student_hidden.contiguous().to(dtype),
            weight=weight.contiguous().to(dtype),
            labels=labels.contiguous(),
            teacher_hidden=teacher_hidden.contiguous().to(dtype),
            teacher_weight=None,
            teacher_logits=None,
            student_ce_weight=float(student_ce_weight),
            teacher_ce_weight=float(teacher_ce_weight),
            kl_weight=float(kl_weight),
            kl_temperature=float(kl_temperature),
            ignore_index=int(ignore_index),
            reduction=reduction,
            vocab_chunk=vocab_chunk_for(BT, V, chunk_size, max_chunks),
            divergence=divergence,
            compute_teacher_ce=float(teacher_ce_weight) != 0.0,
            need_grad_student_hidden=student_hidden.requires_grad,
            need_grad_weight=weight.requires_grad,
            need_grad_teacher_hidden=teacher_hidden.requires_grad,
            grads_in_forward=grads_in_forward("tied", use_fp32_accum, divergence, ctx.compute_grad),
            token_chunk=token_chunk_for(chunk_size),
        )
        loss, ce_s, ce_t, kl = fused_forward(ctx, call)
        ctx.mark_non_differentiable(ce_s, ce_t, kl)
        return loss, ce_s, ce_t, kl

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output, _gs=None, _gt=None, _gkl=None):
        if grad_output is None or not ctx.compute_grad:
            return (None,) * 17
        g_hs, g_w, g_ht, _ = fused_backward(ctx, grad_output)
        d_hs, d_ht, d_w = ctx.dtypes
        return (cast_to(g_hs, d_hs), cast_to(g_ht, d_ht), cast_to(g_w, d_w)) + (None,) * 14


@torch._dynamo.disable
def tied_distillation_loss(
    student_hidden: torch.Tensor,
    teacher_hidden: torch.Tensor | None,
    weight: torch.Tensor,
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
    """Tied-teacher loss on the HIP path; returns ``(loss, student_ce,
    teacher_ce, kl)``.  ``teacher_ce_weight`` defaults to 1.0 (reference
    ``ops/tied_teacher.py:587``)."""
    w_t = 1.0 if teacher_ce_weight is None else float(teacher_ce_weight)
    require_native("tied_distillation_loss")
    BT, H, V = check_common(student_hidden, weight, labels)
    if teacher_hidden is None:
        raise ValueError("tied_distillation_loss requires teacher_hidden")
    if teacher_hidden.shape != (BT, H):
        raise ValueError(
            f"teacher_hidden.shape={tuple(teacher_hidden.shape)} does not match student_hidden.shape={(BT, H)}"
        )
    check_scalars(
        student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
        max_fused_size=max_fused_size, teacher_ce_weight=w_t, reduction=reduction, max_chunks=max_chunks,
    )
    device = student_hidden.device
    if device.type != "cuda":
        raise ValueError(f"tensors must be CUDA/HIP tensors, got device={device}")
    if labels.device != device or weight.device != device or teacher_hidden.device != device:
        raise ValueError("labels, weight and teacher_hidden must be on the same device as student_hidden")
    if validate_labels:
        check_labels_in_range(labels, V, ignore_index)
    return TiedCEFunction.apply(
        student_hidden, teacher_hidden, weight, labels, student_ce_weight, ignore_index, reduction,
        chunk_size, use_fp32_accum, kl_weight, kl_temperature, w_t, max_chunks, max_fused_size, autotune,
        validate_labels, divergence,
    )
