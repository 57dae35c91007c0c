"""``torch.compile``-friendly entry point.

The reference's ``distillation_loss`` is a graph break under ``torch.compile``
(``@torch._dynamo.disable``, reference ``api.py:339``), and so is this
package's drop-in :func:`orda_ce_kernel.distillation_loss`, which keeps that
contract.  This module exposes the same loss as ``torch.library`` custom ops,
so a compiled training step traces through it in one graph:

* ``orda_ce::fused_loss`` runs ``orda_forward`` with the gradients computed
  inside forward (the default schedule) and returns the four loss components
  and the four gradients (empty tensors where not requested) as outputs;
* its autograd formula multiplies those gradients by ``grad_output`` (out of
  place, in the gradient's dtype: no tensor handed out is changed later);
* a fake (meta) implementation gives the output shapes, so Dynamo/AOT
  tracing never runs the kernels.

Differences from the drop-in entry: no OOM retry with more chunks (the chunk
is the reference's auto chunk, or ``chunk_size``), and the compute dtype comes
from the inputs, not from an enclosing autocast region.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .api import (DistillationLossOutput, _resolve_teacher_ce_weight, _teacher_mode_and_tensors, _validate_teacher)
from .divergences import Divergence, resolve_divergence

__all__ = ["distillation_loss"]

_GRAD_SLOTS = 4  # student hidden, weight, teacher hidden, teacher weight


def _mode_name(mode: str, teacher_logits) -> str:
    if mode == "precomputed":
        return "precomputed_logits" if teacher_logits is not None else "precomputed_hidden"
    return mode


def _compute_dtype(student_hidden, weight, teacher_hidden, teacher_weight, teacher_logits, use_teacher: bool):
    """The inputs' compute dtype by the reference's rule without autocast
    (``_runtime.py:61-80``): bf16 if any input is bf16, then fp16, then fp32."""
    ts = [t for t in (weight, student_hidden, teacher_hidden, teacher_weight) if t is not None]
    if teacher_logits is not None and use_teacher:
        ts.append(teacher_logits)
    floats = {t.dtype for t in ts if t.is_floating_point()}
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        if dt in floats:
            return dt
    return torch.bfloat16


@torch.library.custom_op("orda_ce::fused_loss", mutates_args=())
def fused_loss(
    student_hidden: torch.Tensor,
    weight: torch.Tensor,
    labels: torch.Tensor,
    teacher_hidden: Optional[torch.Tensor],
    teacher_weight: Optional[torch.Tensor],
    teacher_logits: Optional[torch.Tensor],
    mode: str,
    student_ce_weight: float,
    teacher_ce_weight: float,
    kl_weight: float,
    kl_temperature: float,
    ignore_index: int,
    reduction: str,
    divergence: str,
    div_alpha: float,
    div_beta: float,
    need_grads: list[bool],
    chunk_size: int,
) -> list[torch.Tensor]:
    """Loss components and gradients of one fused evaluation (see module doc).
    ``div_alpha`` / ``div_beta`` NaN = the divergence's default;
    ``chunk_size`` 0 = the reference's auto chunk."""
    from .ops._engine import FusedCall, run_fused_call, token_chunk_for
    from .utils.resolver import resolve_chunk_size

    use_teacher = kl_weight != 0.0 or teacher_ce_weight != 0.0
    dtype = _compute_dtype(student_hidden, weight, teacher_hidden, teacher_weight, teacher_logits, use_teacher)
    BT, H = student_hidden.shape
    V = weight.shape[0]
    cs = chunk_size if chunk_size > 0 else resolve_chunk_size(BT, None, V=V)[0]
    nan_none = lambda x: None if math.isnan(x) else float(x)  # noqa: E731
    div = resolve_divergence(Divergence(divergence, nan_none(div_alpha), nan_none(div_beta)))
    grads_teacher = mode in ("tied", "separate") and teacher_ce_weight != 0.0
    need = [bool(need_grads[0]), bool(need_grads[1]), bool(need_grads[2]) and grads_teacher,
            bool(need_grads[3]) and grads_teacher and mode == "separate"]
    cast = lambda t: None if t is None else t.detach().contiguous().to(dtype)  # noqa: E731
    lt = None
    if teacher_logits is not None:
        lt = teacher_logits.detach()
        if lt.dtype != dtype and lt.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            lt = lt.float()
    call = FusedCall(
        mode=mode, student_hidden=cast(student_hidden), weight=cast(weight), labels=labels.contiguous(),
        teacher_hidden=cast(teacher_hidden), teacher_weight=cast(teacher_weight), teacher_logits=lt,
        student_ce_weight=float(student_ce_weight), teacher_ce_weight=float(teacher_ce_weight),
        kl_weight=float(kl_weight), kl_temperature=float(kl_temperature), ignore_index=int(ignore_index),
        reduction=reduction, vocab_chunk=0, divergence=div, compute_teacher_ce=teacher_ce_weight != 0.0,
        need_grad_student_hidden=need[0], need_grad_weight=need[1], need_grad_teacher_hidden=need[2],
        need_grad_teacher_weight=need[3],
        # gradients inside forward; given logits of another dtype take the
        # two-phase schedule, which computes no gradients here
        grads_in_forward=any(need) and (lt is None or lt.dtype == dtype),
        token_chunk=token_chunk_for(cs),
    )
    if any(need) and not call.grads_in_forward:
        raise ValueError("orda_ce::fused_loss: precomputed teacher logits must be in the compute dtype "
                         f"({dtype}) when gradients are requested; got {lt.dtype}")
    outs, grads, _ = run_fused_call(call)
    widths = (H, H, H if mode == "tied" else (teacher_hidden.shape[1] if teacher_hidden is not None else 0),
              teacher_hidden.shape[1] if teacher_hidden is not None else 0)
    res = list(outs)
    for g, width in zip(grads, widths):
        if g is None:
            res.append(student_hidden.new_empty((0,), dtype=dtype))
        else:
            res.append(g[:, :width] if g.shape[1] != width else g)
    return res


@fused_loss.register_fake
def _fused_loss_fake(student_hidden, weight, labels, teacher_hidden, teacher_weight, teacher_logits, mode,
                     student_ce_weight, teacher_ce_weight, kl_weight, kl_temperature, ignore_index, reduction,
                     divergence, div_alpha, div_beta, need_grads, chunk_size):
    use_teacher = kl_weight != 0.0 or teacher_ce_weight != 0.0
    dtype = _compute_dtype(student_hidden, weight, teacher_hidden, teacher_weight, teacher_logits, use_teacher)
    grads_teacher = mode in ("tied", "separate") and teacher_ce_weight != 0.0
    need = [need_grads[0], need_grads[1], need_grads[2] and grads_teacher,
            need_grads[3] and grads_teacher and mode == "separate"]
    res = [student_hidden.new_empty((), dtype=torch.float32) for _ in range(4)]
    for flag, ref in zip(need, (student_hidden, weight, teacher_hidden, teacher_weight)):
        res.append(ref.new_empty(ref.shape, dtype=dtype) if (flag and ref is not None)
                   else student_hidden.new_empty((0,), dtype=dtype))
    return res


def _setup_context(ctx, inputs, output):
    ctx.save_for_backward(*output[4:4 + _GRAD_SLOTS])
    ctx.input_dtypes = tuple(None if inputs[i] is None else inputs[i].dtype for i in (0, 1, 3, 4))


def _backward(ctx, grads):
    g_loss = grads[0]
    saved = ctx.saved_tensors
    res = []
    for g, dt in zip(saved, ctx.input_dtypes):
        if g.numel() == 0 or dt is None:
            res.append(None)
        else:
            # (grad_output is applied in the gradient's dtype: no fp32 copy of
            # a [V x H] gradient)
            res.append((g * g_loss).to(dt))
    d_hs, d_w, d_ht, d_wt = res
    # one gradient per op input (None for labels, logits and the scalars)
    return (d_hs, d_w, None, d_ht, d_wt) + (None,) * 13


fused_loss.register_autograd(_backward, setup_context=_setup_context)


def distillation_loss(
    student_hidden: torch.Tensor,
    weight: torch.Tensor,
    labels: torch.Tensor,
    teacher,
    *,
    student_ce_weight: float = 1.0,
    teacher_ce_weight: float | None = None,
    kl_weight: float = 0.0,
    kl_temperature: float = 1.0,
    ignore_index: int = -100,
    reduction: str = "mean",
    divergence: str | Divergence = "forward_kl",
    chunk_size: int | None = None,
) -> DistillationLossOutput:
    """:func:`orda_ce_kernel.distillation_loss` (same loss, arguments and
    defaults; ``chunk_size`` as ``KernelConfig.chunk_size``) as custom ops
    that ``torch.compile`` traces without a graph break.  HIP tensors only."""
    if reduction not in ("mean", "sum"):
        raise ValueError(f"reduction must be 'mean' or 'sum', got {reduction!r}")
    if kl_temperature <= 0.0:
        raise ValueError(f"kl_temperature must be > 0.0, got {kl_temperature}")
    if student_ce_weight < 0.0 or kl_weight < 0.0 or (teacher_ce_weight is not None and teacher_ce_weight < 0.0):
        raise ValueError("loss weights must be >= 0.0")
    if labels.dtype != torch.long:
        raise ValueError(f"labels must have dtype torch.long, got {labels.dtype}")
    mode, t_hidden, t_weight, t_logits = _teacher_mode_and_tensors(teacher)
    _validate_teacher(mode=mode, teacher_hidden=t_hidden, teacher_weight=t_weight, teacher_logits=t_logits,
                      student_hidden=student_hidden, weight=weight)
    w_t = _resolve_teacher_ce_weight(mode, teacher_ce_weight)
    if mode == "precomputed" and w_t != 0.0:
        raise ValueError("a PrecomputedTeacher has no gradient path: teacher_ce_weight must be 0.0")
    div = resolve_divergence(divergence)
    need = [student_hidden.requires_grad, weight.requires_grad,
            t_hidden is not None and t_hidden.requires_grad and mode != "precomputed",
            t_weight is not None and t_weight.requires_grad and mode == "separate"]
    outs = fused_loss(
        student_hidden, weight, labels, t_hidden, t_weight, t_logits, _mode_name(mode, t_logits),
        float(student_ce_weight), float(w_t), float(kl_weight), float(kl_temperature), int(ignore_index),
        reduction, div.name, float("nan") if div.alpha is None else float(div.alpha),
        float("nan") if div.beta is None else float(div.beta), need, int(chunk_size or 0),
    )
    return DistillationLossOutput(outs[0], outs[1].detach(), outs[2].detach(), outs[3].detach())
