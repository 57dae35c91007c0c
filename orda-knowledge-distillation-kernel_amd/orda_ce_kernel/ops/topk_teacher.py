"""Top-k teacher: a precomputed teacher stored as its k most likely
vocabulary ids and their log-probabilities per token.

The reference caches a precomputed teacher as full ``[N x V]`` logits, or as
hidden states plus its LM head (reference
``test/benchmark/src/_train.py:56-99``), and its precomputed path streams the
whole ``[N x V]`` tensor (``ops/precomputed_teacher.py:336-356``): 2.10 GB per
pass at 8192 tokens and a 128256-row vocabulary in bf16.  A top-k teacher
keeps ``k`` (id, log-probability) pairs per token instead -- 12 bytes each,
about 1.5 MB at k = 64 for the same tokens.

The teacher distribution it stands for is the teacher renormalised over its
k ids (zero elsewhere): at temperature T, ``p_t = softmax(logprobs / T)``
over the ids.  Divergences that stay finite with a teacher that is zero off
its ids and whose student gradient is sparse in the same way are supported:
forward KL (the reference's) and soft-target CE, whose gradient in the
student's logits at temperature T is ``p_s - p_t`` (dense ``p_s``, ``p_t`` on
the k ids).  There is no teacher CE and no teacher gradient.

Kernels: the student scan (logits and softmax statistics, no teacher), then a
per-token pass over the k ids (the student logit at each id as an fp32 dot
product, the renormalised teacher, the divergence row), the dense dlogits
pass with a zero teacher, and a scatter of ``-p_t`` into the k ids' dlogits;
the gradient GEMMs are the other modes'.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from .._runtime import default_compute_dtype
from ..divergences import resolve_divergence
from ..utils.resolver import DEFAULT_MAX_FUSED_SIZE
from ._checks import check_common, check_labels_in_range, check_scalars
from ._engine import FusedCall, cast_to, fused_backward, fused_forward, require_native, token_chunk_for

__all__ = ["TOPK_DIVERGENCES", "TopKCEFunction", "check_topk_teacher", "topk_distillation_loss"]

TOPK_DIVERGENCES = ("forward_kl", "soft_target_ce")


def check_topk_teacher(indices: torch.Tensor, logprobs: torch.Tensor, BT: int, V: int, divergence) -> None:
    """Shape, dtype and divergence checks of a top-k teacher."""
    if indices.ndim != 2 or indices.shape[0] != BT:
        raise ValueError(f"TopKTeacher.indices must have shape (BT, k), got {tuple(indices.shape)}")
    if indices.dtype not in (torch.int64, torch.int32):
        raise ValueError(f"TopKTeacher.indices must have an integer dtype (int64 / int32), got {indices.dtype}")
    k = indices.shape[1]
    if not 1 <= k <= V:
        raise ValueError(f"TopKTeacher needs 1 <= k <= vocab ({V}), got k={k}")
    if logprobs.shape != indices.shape:
        raise ValueError(
            f"TopKTeacher.logprobs must have the shape of indices {tuple(indices.shape)}, got {tuple(logprobs.shape)}"
        )
    if not logprobs.is_floating_point():
        raise ValueError(f"TopKTeacher.logprobs must be floating point, got {logprobs.dtype}")
    if logprobs.requires_grad:
        raise ValueError("TopKTeacher.logprobs must not require gradients")
    name = resolve_divergence(divergence).name
    if name not in TOPK_DIVERGENCES:
        raise ValueError(f"a TopKTeacher supports the divergences {TOPK_DIVERGENCES}, got {name!r}")


class TopKCEFunction(torch.autograd.Function):
    @staticmethod
    def forward(
        ctx,
        student_hidden,
        weight,
        topk_indices,
        topk_logprobs,
        labels,
        student_ce_weight=1.0,
        ignore_index=-100,
        reduction="mean",
        chunk_size=None,
        kl_weight=0.0,
        kl_temperature=1.0,
        max_chunks=None,
        max_fused_size=DEFAULT_MAX_FUSED_SIZE,
        divergence=None,
    ):
        require_native("topk_distillation_loss")
        check_scalars(student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
                      max_fused_size=max_fused_size)
        ctx.compute_grad = student_hidden.requires_grad or weight.requires_grad
        ctx.dtypes = (student_hidden.dtype, weight.dtype)
        dtype = default_compute_dtype(weight, student_hidden)
        call = FusedCall(
            mode="topk",
            student_hidden=student_hidden.contiguous().to(dtype),
            weight=weight.contiguous().to(dtype),
            labels=labels.contiguous(),
            teacher_hidden=None,
            teacher_weight=None,
            teacher_logits=None,
            student_ce_weight=float(student_ce_weight),
            teacher_ce_weight=0.0,
            kl_weight=float(kl_weight),
            kl_temperature=float(kl_temperature),
            ignore_index=int(ignore_index),
            reduction=reduction,
            vocab_chunk=0,
            divergence=divergence,
            compute_teacher_ce=False,
            need_grad_student_hidden=student_hidden.requires_grad,
            need_grad_weight=weight.requires_grad,
            # the top-k teacher's sparse pass runs inside the token-chunk
            # schedule, with or without gradients
            grads_in_forward=True,
            token_chunk=token_chunk_for(chunk_size),
            topk_indices=topk_indices.contiguous().to(torch.int64),
            topk_logprobs=topk_logprobs.detach().contiguous().to(torch.float32),
        )
        loss, ce_s, ce_t, kl = fused_forward(ctx, call)
        ctx.mark_non_differentiable(ce_s, ce_t, kl)
        return loss, ce_s, ce_t, kl

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output, _gs=None, _gt=None, _gkl=None):
        if grad_output is None or not ctx.compute_grad:
            return (None,) * 14
        g_hs, g_w, _, _ = fused_backward(ctx, grad_output)
        d_hs, d_w = ctx.dtypes
        return (cast_to(g_hs, d_hs), cast_to(g_w, d_w)) + (None,) * 12


@torch._dynamo.disable
def topk_distillation_loss(
    student_hidden: torch.Tensor,
    weight: torch.Tensor,
    topk_indices: torch.Tensor,
    topk_logprobs: torch.Tensor,
    labels: torch.Tensor,
    student_ce_weight: float = 1.0,
    ignore_index: int = -100,
    reduction: str = "mean",
    chunk_size=None,
    kl_weight: float = 0.0,
    kl_temperature: float = 1.0,
    max_chunks: int | None = None,
    max_fused_size: int = DEFAULT_MAX_FUSED_SIZE,
    validate_labels: bool = True,
    divergence=None,
):
    """Top-k-teacher loss on the HIP path; returns ``(loss, student_ce,
    teacher_ce, kl)`` (``teacher_ce`` is 0: the teacher has no CE term)."""
    require_native("topk_distillation_loss")
    BT, H, V = check_common(student_hidden, weight, labels)
    check_topk_teacher(topk_indices, topk_logprobs, BT, V, divergence)
    check_scalars(student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
                  max_fused_size=max_fused_size, reduction=reduction, max_chunks=max_chunks)
    device = student_hidden.device
    if device.type != "cuda":
        raise ValueError(f"tensors must be CUDA/HIP tensors, got device={device}")
    if validate_labels:
        check_labels_in_range(labels, V, ignore_index)
    return TopKCEFunction.apply(
        student_hidden, weight, topk_indices, topk_logprobs, labels, student_ce_weight, ignore_index, reduction,
        chunk_size, kl_weight, kl_temperature, max_chunks, max_fused_size, divergence,
    )
