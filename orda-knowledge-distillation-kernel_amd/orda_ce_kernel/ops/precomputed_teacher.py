"""Precomputed teacher: teacher logits ``[N x V]`` given, or a frozen
``(teacher_hidden, teacher_weight)`` pair.

Mirrors the reference's ``ops/precomputed_teacher.py`` interface
(``PrecomputedCEFunction`` ``:239-523``, ``precomputed_distillation_loss``
``:527-651``): same ``.apply`` order, defaults, checks and messages, plus one
optional trailing ``divergence`` argument.

Given logits are streamed by the fused kernels in their own dtype (bf16,
fp16 or fp32; other float dtypes are read as fp32); the reference casts them
to the compute dtype first (``:340-348``), which only loses precision.  The
teacher is frozen: it gets no gradient.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from .._runtime import default_compute_dtype
from ..utils.resolver import DEFAULT_MAX_FUSED_SIZE
from ._checks import check_common, check_labels_in_range, check_scalars
from ._engine import (FusedCall, cast_to, fused_backward, fused_forward, grads_in_forward, require_native,
                      token_chunk_for, vocab_chunk_for)

__all__ = ["PrecomputedCEFunction", "precomputed_distillation_loss"]


def _forward(ctx, student_hidden, weight, logits_teacher, labels, student_ce_weight, ignore_index, reduction,
             chunk_size, kl_weight, kl_temperature, teacher_ce_weight, max_chunks, max_fused_size, teacher_hidden,
             teacher_weight, divergence, use_fp32_accum=None):
    check_scalars(
        student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
        max_fused_size=max_fused_size,
    )
    require_native("precomputed_distillation_loss")
    if labels.dtype != torch.long:
        raise ValueError(f"labels must have dtype torch.long, got {labels.dtype}")
    BT = student_hidden.shape[0]
    V = weight.shape[0]
    use_teacher = float(kl_weight) != 0.0 or float(teacher_ce_weight) != 0.0
    if logits_teacher is not None:
        mode = "precomputed_logits"
        dtype = default_compute_dtype(weight, student_hidden, *( [logits_teacher] if use_teacher else []))
        th = tw = None
    elif teacher_hidden is not None and teacher_weight is not None:
        mode = "precomputed_hidden"
        dtype = default_compute_dtype(weight, student_hidden, *([teacher_hidden] if use_teacher else []))
        th = teacher_hidden.detach().contiguous().to(dtype)
        tw = teacher_weight.detach().contiguous().to(dtype)
    else:
        raise ValueError("PrecomputedCEFunction requires logits_teacher or (teacher_hidden, teacher_weight)")
    ctx.compute_grad = student_hidden.requires_grad or weight.requires_grad
    ctx.dtypes = (student_hidden.dtype, weight.dtype)
    call = FusedCall(
        mode=mode,
        student_hidden=student_hidden.contiguous().to(dtype),
        weight=weight.contiguous().to(dtype),
        labels=labels.contiguous(),
        teacher_hidden=th,
        teacher_weight=tw,
        teacher_logits=None if logits_teacher is None else logits_teacher.detach(),
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
        # (logits of another dtype are taken as the compute dtype holds them
        # in either schedule, as the reference casts each chunk,
        # ops/precomputed_teacher.py:343-348)
        grads_in_forward=grads_in_forward(mode, use_fp32_accum, divergence, ctx.compute_grad),
        token_chunk=token_chunk_for(chunk_size),
    )
    loss, ce_s, ce_t, kl = fused_forward(ctx, call)
    ctx.mark_non_differentiable(ce_s, ce_t, kl)
    return loss, ce_s, ce_t, kl


def _backward(ctx, grad_output):
    if grad_output is None or not ctx.compute_grad:
        return (None,) * 19
    g_hs, g_w, _, _ = fused_backward(ctx, grad_output)
    d_hs, d_w = ctx.dtypes
    return (cast_to(g_hs, d_hs), cast_to(g_w, d_w)) + (None,) * 17


class PrecomputedCEFunction(torch.autograd.Function):
    @staticmethod
    def forward(
        ctx,
        student_hidden,
        weight,
        logits_teacher,
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
        teacher_hidden=None,
        teacher_weight=None,
        validate_labels=True,
        divergence=None,
    ):
        if float(teacher_ce_weight) != 0.0:
            raise ValueError("PrecomputedCEFunction requires teacher_ce_weight=0.0")
        return _forward(ctx, student_hidden, weight, logits_teacher, labels, student_ce_weight, ignore_index,
                        reduction, chunk_size, kl_weight, kl_temperature, 0.0, max_chunks, max_fused_size,
                        teacher_hidden, teacher_weight, divergence, use_fp32_accum)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output, _gs=None, _gt=None, _gkl=None):
        return _backward(ctx, grad_output)


class PrecomputedTeacherCEFunction(torch.autograd.Function):
    """Like :class:`PrecomputedCEFunction` but also reports the teacher's CE
    (no teacher gradient: the teacher is frozen).  The reference only has this
    through its unfused torch fallback (``api.py:392-397``); ``backend='auto'``
    on HIP tensors uses this Function instead."""

    @staticmethod
    def forward(ctx, student_hidden, weight, logits_teacher, labels, student_ce_weight=1.0, ignore_index=-100,
                reduction="mean", chunk_size=None, use_fp32_accum=None, kl_weight=0.0, kl_temperature=1.0,
                teacher_ce_weight=0.0, max_chunks=None, max_fused_size=DEFAULT_MAX_FUSED_SIZE, autotune=False,
                teacher_hidden=None, teacher_weight=None, validate_labels=True, divergence=None):
        if float(teacher_ce_weight) < 0.0:
            raise ValueError(f"teacher_ce_weight must be >= 0.0, got {teacher_ce_weight}")
        return _forward(ctx, student_hidden, weight, logits_teacher, labels, student_ce_weight, ignore_index,
                        reduction, chunk_size, kl_weight, kl_temperature, float(teacher_ce_weight), max_chunks,
                        max_fused_size, teacher_hidden, teacher_weight, divergence, use_fp32_accum)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output, _gs=None, _gt=None, _gkl=None):
        return _backward(ctx, grad_output)


def _check_precomputed(student_hidden, weight, logits_teacher, labels, teacher_hidden, teacher_weight):
    BT, H, V = check_common(student_hidden, weight, labels)
    if logits_teacher is not None:
        if logits_teacher.shape != (BT, V):
            raise ValueError(f"logits_teacher must have shape ({BT}, {V}), got {tuple(logits_teacher.shape)}")
        if logits_teacher.requires_grad:
            raise ValueError(
                "precomputed_distillation_loss requires logits_teacher without gradients; "
                "use SeparateTeacher when the teacher path needs gradients"
            )
    elif teacher_hidden is not None and teacher_weight is not None:
        if teacher_hidden.ndim != 2 or teacher_hidden.shape[0] != BT:
            raise ValueError(f"teacher_hidden must have shape (BT, D_t), got {tuple(teacher_hidden.shape)}")
        if teacher_weight.shape != (V, teacher_hidden.shape[1]):
            raise ValueError(
                f"teacher_weight must have shape ({V}, {teacher_hidden.shape[1]}), got {tuple(teacher_weight.shape)}"
            )
        if teacher_hidden.requires_grad or teacher_weight.requires_grad:
            raise ValueError("teacher_hidden and teacher_weight must not require gradients")
    else:
        raise ValueError(
            "precomputed_distillation_loss requires logits_teacher or (teacher_hidden, teacher_weight)"
        )
    return BT, H, V


def _check_devices(student_hidden, labels, weight, logits_teacher, teacher_hidden, teacher_weight):
    device = student_hidden.device
    if device.type != "cuda":
        raise ValueError(f"tensors must be CUDA/HIP tensors, got device={device}")
    others = [labels, weight] + [x for x in (logits_teacher, teacher_hidden, teacher_weight) if x is not None]
    if any(x.device != device for x in others):
        raise ValueError("all tensors must be on the same device as student_hidden")


@torch._dynamo.disable
def precomputed_distillation_loss(
    student_hidden: torch.Tensor,
    weight: torch.Tensor,
    logits_teacher: torch.Tensor | None = None,
    labels: torch.Tensor = None,
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
    teacher_hidden: torch.Tensor | None = None,
    teacher_weight: torch.Tensor | None = None,
    validate_labels: bool = True,
    divergence=None,
):
    """Precomputed-teacher loss on the HIP path; requires
    ``teacher_ce_weight`` 0 like the reference (``:603-604``)."""
    w_t = 0.0 if teacher_ce_weight is None else float(teacher_ce_weight)
    require_native("precomputed_distillation_loss")
    if student_hidden.ndim != 2:
        raise ValueError(f"student_hidden must be 2D, got shape={tuple(student_hidden.shape)}")
    BT, H, V = _check_precomputed(student_hidden, weight, logits_teacher, labels, teacher_hidden, teacher_weight)
    if w_t != 0.0:
        raise ValueError("Triton precomputed_distillation_loss requires teacher_ce_weight=0.0")
    check_scalars(
        student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
        max_fused_size=max_fused_size, reduction=reduction, max_chunks=max_chunks,
    )
    _check_devices(student_hidden, labels, weight, logits_teacher, teacher_hidden, teacher_weight)
    if validate_labels:
        check_labels_in_range(labels, V, ignore_index)
    return PrecomputedCEFunction.apply(
        student_hidden, weight, logits_teacher, labels, student_ce_weight, ignore_index, reduction, chunk_size,
        use_fp32_accum, kl_weight, kl_temperature, w_t, max_chunks, max_fused_size, autotune, teacher_hidden,
        teacher_weight, validate_labels, divergence,
    )


@torch._dynamo.disable
def precomputed_distillation_loss_with_teacher_ce(
    student_hidden, weight, logits_teacher=None, labels=None, student_ce_weight=1.0, ignore_index=-100,
    reduction="mean", chunk_size=None, use_fp32_accum=None, kl_weight=0.0, kl_temperature=1.0,
    teacher_ce_weight=None, max_chunks=None, max_fused_size=DEFAULT_MAX_FUSED_SIZE, autotune=False,
    teacher_hidden=None, teacher_weight=None, validate_labels=True, divergence=None,
):
    """Precomputed teacher with its CE reported (HIP path of
    ``backend='auto'`` when ``teacher_ce_weight != 0``)."""
    w_t = 0.0 if teacher_ce_weight is None else float(teacher_ce_weight)
    require_native("precomputed_distillation_loss")
    _, _, V = _check_precomputed(student_hidden, weight, logits_teacher, labels, teacher_hidden, teacher_weight)
    check_scalars(
        student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
        max_fused_size=max_fused_size, teacher_ce_weight=w_t, reduction=reduction, max_chunks=max_chunks,
    )
    _check_devices(student_hidden, labels, weight, logits_teacher, teacher_hidden, teacher_weight)
    if validate_labels:
        check_labels_in_range(labels, V, ignore_index)
    return PrecomputedTeacherCEFunction.apply(
        student_hidden, weight, logits_teacher, labels, student_ce_weight, ignore_index, reduction, chunk_size,
        use_fp32_accum, kl_weight, kl_temperature, w_t, max_chunks, max_fused_size, autotune, teacher_hidden,
        teacher_weight, validate_labels, divergence,
    )
