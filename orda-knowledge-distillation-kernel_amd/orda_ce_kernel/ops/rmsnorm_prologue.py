"""The extension entry: the student's final RMSNorm fused in front of the
loss, and/or the scan's logits GEMM on fp8 operands.

The reference's producer normalises the last hidden states before the LM
head, ``y = x * rsqrt(mean(x^2) + eps) * w`` (reference
``test/benchmark/src/core.py:7-14``, applied at ``:135``), and hands ``y`` to
the loss; autograd then runs the norm's backward as separate kernels over
``[N x H]`` tensors.  Here the loss takes ``x`` and the norm weight and, per
token chunk of the gradients-in-forward schedule:

* ``k_rmsnorm_fwd`` forms the chunk's ``y`` (fp32 arithmetic, rounded once
  to the compute dtype) and its ``rsqrt`` per row; every GEMM of the chunk
  (logits, label logits, grad W) reads that ``y``;
* after the grad-hidden GEMM has written ``dloss/dy`` for the chunk,
  ``k_rmsnorm_dgamma`` adds ``sum_t dy * x * r`` to an fp32 accumulator of
  the norm weight's gradient (fixed order: bit-stable) and ``k_rmsnorm_bwd``
  turns ``dloss/dy`` into ``dloss/dx = r (w dy) - x r^3 <w dy, x> / H`` in
  place.

Every teacher mode and divergence works unchanged (only the student's rows
are transformed).  No counterpart in the reference's loss API: an extension
(``distillation_loss(..., student_norm=StudentRMSNorm(weight, eps))``).

``logits_gemm="fp8"`` (``ORDA_FP8_LOGITS``): the scan's logits GEMM takes W
and the chunk's hidden rows rounded to OCP e4m3 with one power-of-two scale
per row (``v_mfma_scale_f32_32x32x64_f8f6f4`` applies the scales), so the
losses, softmax statistics and dlogits come from those logits; the gradient
GEMMs keep the compute dtype.  With or without the norm; ``norm_weight`` may
be None.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch.autograd.function import once_differentiable

from .._runtime import default_compute_dtype
from ._engine import FusedCall, cast_to, fused_backward, fused_forward, require_native

__all__ = ["NormedCall", "RMSNormPrologueFunction"]


@dataclass(frozen=True)
class NormedCall:
    """The non-differentiable part of a normed loss call."""

    mode: str                   # tied / separate / precomputed_logits / precomputed_hidden / topk
    teacher_logits: torch.Tensor | None
    topk_indices: torch.Tensor | None
    topk_logprobs: torch.Tensor | None
    student_ce_weight: float
    teacher_ce_weight: float
    kl_weight: float
    kl_temperature: float
    ignore_index: int
    reduction: str
    divergence: object
    token_chunk: int
    eps: float
    fp8_logits: bool = False


class RMSNormPrologueFunction(torch.autograd.Function):
    """``(x, norm_weight, weight, teacher_hidden, teacher_weight, labels,
    spec)`` → ``(loss, student_ce, teacher_ce, kl)``; gradients for ``x``,
    ``norm_weight``, ``weight`` and (teacher CE) the teacher's tensors."""

    @staticmethod
    def forward(ctx, x, norm_weight, weight, teacher_hidden, teacher_weight, labels, spec: NormedCall):
        require_native("the fused RMSNorm prologue / fp8 logits")
        trainable_teacher = spec.mode in ("tied", "separate")
        ht_grad = trainable_teacher and teacher_hidden is not None and teacher_hidden.requires_grad
        wt_grad = spec.mode == "separate" and teacher_weight is not None and teacher_weight.requires_grad
        nw_grad = norm_weight is not None and norm_weight.requires_grad
        ctx.compute_grad = x.requires_grad or nw_grad or weight.requires_grad or ht_grad or wt_grad
        ctx.dtypes = (x.dtype, None if norm_weight is None else norm_weight.dtype, weight.dtype,
                      None if teacher_hidden is None else teacher_hidden.dtype,
                      None if teacher_weight is None else teacher_weight.dtype)
        ops = [t for t in (weight, x, teacher_hidden, teacher_weight) if t is not None]
        dtype = default_compute_dtype(*ops)
        cast = lambda t: None if t is None else t.contiguous().to(dtype)  # noqa: E731
        lt = spec.teacher_logits
        call = FusedCall(
            mode=spec.mode,
            student_hidden=cast(x),
            weight=cast(weight),
            labels=labels.contiguous(),
            teacher_hidden=None if spec.mode in ("precomputed_logits", "topk") else cast(teacher_hidden),
            teacher_weight=cast(teacher_weight) if spec.mode in ("separate", "precomputed_hidden") else None,
            # (precomputed logits in the compute dtype, as the reference casts
            # them, ops/precomputed_teacher.py:340-348)
            teacher_logits=None if lt is None else lt.detach().to(dtype),
            student_ce_weight=float(spec.student_ce_weight),
            teacher_ce_weight=float(spec.teacher_ce_weight),
            kl_weight=float(spec.kl_weight),
            kl_temperature=float(spec.kl_temperature),
            ignore_index=int(spec.ignore_index),
            reduction=spec.reduction,
            vocab_chunk=0,
            divergence=spec.divergence,
            compute_teacher_ce=float(spec.teacher_ce_weight) != 0.0,
            need_grad_student_hidden=x.requires_grad,
            need_grad_weight=weight.requires_grad,
            need_grad_teacher_hidden=ht_grad,
            need_grad_teacher_weight=wt_grad,
            # the prologue lives in the token-chunk schedule, with or without
            # gradients
            grads_in_forward=True,
            token_chunk=spec.token_chunk,
            topk_indices=None if spec.topk_indices is None else spec.topk_indices.contiguous().to(torch.int64),
            topk_logprobs=None if spec.topk_logprobs is None
            else spec.topk_logprobs.detach().contiguous().to(torch.float32),
            student_norm_weight=None if norm_weight is None else cast(norm_weight.detach()),
            norm_eps=float(spec.eps),
            need_grad_student_norm_weight=nw_grad,
            fp8_logits=bool(spec.fp8_logits),
        )
        loss, ce_s, ce_t, kl = fused_forward(ctx, call)
        ctx.mark_non_differentiable(ce_s, ce_t, kl)
        return loss, ce_s, ce_t, kl

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output, _gs=None, _gt=None, _gkl=None):
        if grad_output is None or not ctx.compute_grad:
            return (None,) * 7
        g_x, g_w, g_ht, g_wt, g_nw = fused_backward(ctx, grad_output, with_norm=True)
        d_x, d_nw, d_w, d_ht, d_wt = ctx.dtypes
        return (cast_to(g_x, d_x), cast_to(g_nw, d_nw), cast_to(g_w, d_w), cast_to(g_ht, d_ht),
                cast_to(g_wt, d_wt), None, None)
