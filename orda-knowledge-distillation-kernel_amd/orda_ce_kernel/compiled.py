"""``torch.compile``-friendly entry point.

The reference's ``distillation_loss`` is a graph break under ``torch.compile``
(``@torch._dynamo.disable``, reference ``api.py:339``), and so is this
package's drop-in :func:`orda_ce_kernel.distillation_loss`, which keeps that
contract.  This module exposes the same loss as ``torch.library`` custom ops,
so a compiled training step traces through it in one graph:

* ``orda_ce::fused_loss`` runs ``orda_forward`` with the gradients computed
  inside forward (the default schedule) and returns the four loss components,
  the five gradients (empty tensors where not requested) and a one-element
  record of the factor already applied to them (1);
* its autograd formula multiplies those gradients by ``grad_output`` in
  place (``orda_ce::scale_grads_``, the library's scaling kernel, which
  leaves them untouched when the factor is 1) and returns them, so no second
  gradient-sized buffer is allocated (grad W is 1.05 GB at the headline
  shape).  Under ``torch.compile`` a second backward through a retained
  graph multiplies by the new ``grad_output`` over the recorded one, and
  autograd copies a gradient it cannot take over (the retained graph still
  holds it), so tensors already handed out never change; called eagerly,
  the first backward hands the buffers over and a second one recomputes
  them, as the drop-in does;
* a fake (meta) implementation gives the output shapes, so Dynamo/AOT
  tracing never runs the kernels.

As in the drop-in entry, the compute dtype follows an enclosing autocast
region (``_runtime.default_compute_dtype``, reference ``_runtime.py:41-80``),
and a device out-of-memory error inside the op halves the token chunk and
retries, up to the dispatcher's limit of ``2 * max(1, BT // 512)`` chunks
(reference ``utils/dispatcher.py:218-293``; the op cannot raise back to a
caller-side loop, so the retry lives in it).  The drop-in's extensions come
along: ``TopKTeacher``, ``student_norm=StudentRMSNorm(w, eps)`` (the norm
weight is an op input with its own gradient) and ``logits_gemm="fp8"``.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from ._runtime import _autocast_dtype
from .api import (DistillationLossOutput, StudentRMSNorm, TopKTeacher, _resolve_teacher_ce_weight,
                  _teacher_mode_and_tensors, _validate_teacher)
from .divergences import Divergence, resolve_divergence

__all__ = ["distillation_loss"]

_GRAD_SLOTS = 5  # student hidden, weight, teacher hidden, teacher weight, student norm weight
_TENSOR_INPUTS = 9  # student hidden, weight, labels, teacher hidden / weight / logits, top-k ids / log-probs, norm weight


def _mode_name(mode: str, teacher_logits) -> str:
    if mode == "precomputed":
        return "precomputed_logits" if teacher_logits is not None else "precomputed_hidden"
    return mode


_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _compute_dtype(student_hidden, weight, teacher_hidden, teacher_weight, teacher_logits, use_teacher: bool,
                   autocast: str = ""):
    """The compute dtype by the reference's rule (``_runtime.py:61-80``): the
    autocast dtype when one was active at the call (``autocast``: its name,
    "" for none), else bf16 if any input is bf16, then fp16, then fp32."""
    if autocast:
        return _DTYPES[autocast]
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
    topk_indices: Optional[torch.Tensor],
    topk_logprobs: Optional[torch.Tensor],
    norm_weight: Optional[torch.Tensor],
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
    norm_eps: float,
    fp8_logits: bool,
    autocast: str,
) -> list[torch.Tensor]:
    """Loss components, gradients and the applied-factor record of one fused
    evaluation (see module doc).  ``div_alpha`` / ``div_beta`` NaN = the
    divergence's default; ``chunk_size`` 0 = the reference's auto chunk;
    ``need_grads``: student hidden, weight, teacher hidden, teacher weight,
    norm weight; ``autocast``: the autocast dtype's name at the call ("" for
    none)."""
    from .ops._engine import FusedCall, run_fused_call, token_chunk_for
    from .utils._autotune import _is_oom_error
    from .utils.resolver import resolve_chunk_size

    use_teacher = kl_weight != 0.0 or teacher_ce_weight != 0.0
    dtype = _compute_dtype(student_hidden, weight, teacher_hidden, teacher_weight, teacher_logits, use_teacher,
                           autocast)
    BT, H = student_hidden.shape
    V = weight.shape[0]
    limit = 2 * max(1, BT // 512)
    cs, n_chunks = (chunk_size, None) if chunk_size > 0 else resolve_chunk_size(BT, None, V=V, max_chunks=limit)
    nan_none = lambda x: None if math.isnan(x) else float(x)  # noqa: E731
    div = resolve_divergence(Divergence(divergence, nan_none(div_alpha), nan_none(div_beta)))
    need = _need(mode, teacher_ce_weight, need_grads, norm_weight)
    cast = lambda t: None if t is None else t.detach().contiguous().to(dtype)  # noqa: E731
    extended = mode == "topk" or norm_weight is not None or fp8_logits
    lt = None
    if teacher_logits is not None:
        lt = teacher_logits.detach()
        if extended and lt.dtype != dtype:
            lt = lt.to(dtype)  # (as the reference casts them, ops/precomputed_teacher.py:340-348)
        elif lt.dtype != dtype and lt.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            lt = lt.float()
    call = FusedCall(
        mode=mode, student_hidden=cast(student_hidden), weight=cast(weight), labels=labels.contiguous(),
        teacher_hidden=cast(teacher_hidden), teacher_weight=cast(teacher_weight), teacher_logits=lt,
        student_ce_weight=float(student_ce_weight), teacher_ce_weight=float(teacher_ce_weight),
        kl_weight=float(kl_weight), kl_temperature=float(kl_temperature), ignore_index=int(ignore_index),
        reduction=reduction, vocab_chunk=0, divergence=div, compute_teacher_ce=teacher_ce_weight != 0.0,
        need_grad_student_hidden=need[0], need_grad_weight=need[1], need_grad_teacher_hidden=need[2],
        need_grad_teacher_weight=need[3],
        # gradients inside forward (precomputed logits of another dtype are
        # cast to the compute dtype on their way into the chunk's buffer);
        # the extensions always run this schedule
        grads_in_forward=extended or any(need),
        token_chunk=token_chunk_for(cs),
        topk_indices=None if topk_indices is None else topk_indices.contiguous().to(torch.int64),
        topk_logprobs=None if topk_logprobs is None else topk_logprobs.detach().contiguous().to(torch.float32),
        student_norm_weight=cast(norm_weight), norm_eps=float(norm_eps), need_grad_student_norm_weight=need[4],
        fp8_logits=bool(fp8_logits),
    )
    while True:
        try:
            outs, grads, _ = run_fused_call(call)
            break
        except Exception as exc:  # the dispatcher's OOM retry (reference utils/dispatcher.py:244-293)
            if chunk_size > 0 or not _is_oom_error(exc) or n_chunks >= min(BT, limit):
                raise
            torch.cuda.empty_cache()
            n_chunks = min(2 * n_chunks, BT, limit)
            call.token_chunk = token_chunk_for(-(-BT // n_chunks))
    widths = (H, H, H if mode == "tied" else (teacher_hidden.shape[1] if teacher_hidden is not None else 0),
              teacher_hidden.shape[1] if teacher_hidden is not None else 0)
    res = list(outs)
    # padded columns (H not a multiple of the kernels' 16 bytes) are cut off
    # into a dense tensor: the fake gives dense (N, width) outputs, and the
    # backward scales these tensors in place
    for g, width in zip(grads[:4], widths):
        if g is None:
            res.append(student_hidden.new_empty((0,), dtype=dtype))
        else:
            res.append(g[:, :width].contiguous() if g.shape[1] != width else g)
    g_nw = grads[4]
    res.append(student_hidden.new_empty((0,), dtype=dtype) if g_nw is None else g_nw[:H].contiguous())
    res.append(torch.ones(1, dtype=torch.float32, device=student_hidden.device))
    return res


def _need(mode, teacher_ce_weight, need_grads, norm_weight):
    """Which gradients the op computes.  A tied teacher that requires grad
    gets one even with its CE off (zeros, as the reference returns,
    ``ops/tied_teacher.py:349,478-479``); a separate teacher's come only
    with its CE (the student-only Function returns none,
    ``ops/separate_teacher.py:713``)."""
    t_ce = teacher_ce_weight != 0.0
    return [bool(need_grads[0]), bool(need_grads[1]),
            bool(need_grads[2]) and (mode == "tied" or (mode == "separate" and t_ce)),
            bool(need_grads[3]) and mode == "separate" and t_ce,
            bool(need_grads[4]) and norm_weight is not None]


@fused_loss.register_fake
def _fused_loss_fake(student_hidden, weight, labels, teacher_hidden, teacher_weight, teacher_logits, topk_indices,
                     topk_logprobs, norm_weight, mode, student_ce_weight, teacher_ce_weight, kl_weight,
                     kl_temperature, ignore_index, reduction, divergence, div_alpha, div_beta, need_grads,
                     chunk_size, norm_eps, fp8_logits, autocast):
    use_teacher = kl_weight != 0.0 or teacher_ce_weight != 0.0
    dtype = _compute_dtype(student_hidden, weight, teacher_hidden, teacher_weight, teacher_logits, use_teacher,
                           autocast)
    need = _need(mode, teacher_ce_weight, need_grads, norm_weight)
    res = [student_hidden.new_empty((), dtype=torch.float32) for _ in range(4)]
    for flag, ref in zip(need, (student_hidden, weight, teacher_hidden, teacher_weight, norm_weight)):
        res.append(ref.new_empty(ref.shape, dtype=dtype) if (flag and ref is not None)
                   else student_hidden.new_empty((0,), dtype=dtype))
    res.append(student_hidden.new_empty((1,), dtype=torch.float32))
    return res


@torch.library.custom_op("orda_ce::scale_grads_", mutates_args=("grads", "applied"))
def scale_grads_(grads: list[torch.Tensor], applied: torch.Tensor, grad_output: torch.Tensor) -> None:
    """``grads *= grad_output / applied`` in place, then ``applied =
    grad_output``: the gradients ``fused_loss`` returned, scaled for this
    backward (``applied`` records the factor already in them; 1 after the
    forward, so the first backward multiplies by ``grad_output`` exactly, on
    the library's kernel, which skips a factor of 1)."""
    from . import _native

    go = grad_output.detach().to(device=applied.device, dtype=torch.float32).reshape(1)
    factor = go / applied
    for g in grads:
        if g.numel():
            _native.scale_gradient_(g, factor)
    applied.copy_(go)


@scale_grads_.register_fake
def _scale_grads_fake(grads, applied, grad_output):
    return None


def _setup_context(ctx, inputs, output):
    # The gradients and the factor record are held on ctx as plain
    # references (marked non-differentiable): they are mutated by the
    # backward, which the version check of saved tensors would reject.
    held = output[4:4 + _GRAD_SLOTS + 1]
    ctx.mark_non_differentiable(*held)
    ctx.held = tuple(held)
    ctx.op_args = tuple(inputs)
    ctx.input_dtypes = tuple(None if inputs[i] is None else inputs[i].dtype for i in (0, 1, 3, 4, 8))


def _traced(t: torch.Tensor) -> bool:
    """True while AOT autograd traces the backward (functional or fake
    tensors), False for an eager call."""
    from torch._subclasses.fake_tensor import FakeTensor
    from torch._subclasses.functional_tensor import FunctionalTensor

    return isinstance(t, (FakeTensor, FunctionalTensor))


def _backward(ctx, grads):
    g_loss = grads[0]
    held = ctx.held
    if held is None:
        # eager, a second backward through a retained graph: the first one
        # handed its buffers over, so recompute (as the drop-in does)
        held = tuple(fused_loss(*ctx.op_args)[4:4 + _GRAD_SLOTS + 1])
    *gs, applied = held
    live = [g for g, dt in zip(gs, ctx.input_dtypes) if g.numel() and dt is not None]
    if g_loss is None or not live:
        return (None,) * (_TENSOR_INPUTS + 15)
    torch.ops.orda_ce.scale_grads_(live, applied, g_loss)
    if not _traced(applied):
        ctx.held = None  # eager: drop our references so autograd takes the buffers without a copy
    res = []
    for g, dt in zip(gs, ctx.input_dtypes):
        if g.numel() == 0 or dt is None:
            res.append(None)
        else:
            res.append(g if g.dtype == dt else g.to(dt))
    d_hs, d_w, d_ht, d_wt, d_nw = res
    # one gradient per op input (None for labels, logits, top-k pairs and the
    # scalars)
    return (d_hs, d_w, None, d_ht, d_wt, None, None, None, d_nw) + (None,) * 15


fused_loss.register_autograd(_backward, setup_context=_setup_context)


def _autocast_name(device: torch.device) -> str:
    if device.type != "cuda":  # the op runs on HIP tensors; meta tensors trace without autocast
        return ""
    dt = _autocast_dtype(device)
    return "" if dt is None else str(dt).replace("torch.", "")


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
    student_norm: StudentRMSNorm | None = None,
    logits_gemm: str = "default",
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
    if logits_gemm not in ("default", "fp8"):
        raise ValueError(f"logits_gemm must be 'default' or 'fp8', got {logits_gemm!r}")
    div = resolve_divergence(divergence)
    tk_i = tk_lp = None
    if isinstance(teacher, TopKTeacher):
        from .ops.topk_teacher import check_topk_teacher

        if teacher_ce_weight not in (None, 0.0):
            raise ValueError("a TopKTeacher has no teacher CE: teacher_ce_weight must be None or 0.0")
        if logits_gemm == "fp8":
            raise ValueError("logits_gemm='fp8' does not support a TopKTeacher")
        check_topk_teacher(teacher.indices, teacher.logprobs, student_hidden.shape[0], weight.shape[0], div)
        mode, t_hidden, t_weight, t_logits, w_t = "topk", None, None, None, 0.0
        tk_i, tk_lp = teacher.indices, teacher.logprobs
    else:
        mode, t_hidden, t_weight, t_logits = _teacher_mode_and_tensors(teacher)
        _validate_teacher(mode=mode, teacher_hidden=t_hidden, teacher_weight=t_weight, teacher_logits=t_logits,
                          student_hidden=student_hidden, weight=weight)
        w_t = _resolve_teacher_ce_weight(mode, teacher_ce_weight)
        if mode == "precomputed" and w_t != 0.0:
            raise ValueError("a PrecomputedTeacher has no gradient path: teacher_ce_weight must be 0.0")
        mode = _mode_name(mode, t_logits)
    nw, eps = None, 1e-6
    if student_norm is not None:
        if not isinstance(student_norm, StudentRMSNorm):
            raise TypeError(f"student_norm must be a StudentRMSNorm, got {type(student_norm).__name__}")
        nw, eps = student_norm.weight, float(student_norm.eps)
        if nw.ndim != 1 or nw.shape[0] != student_hidden.shape[1]:
            raise ValueError(f"StudentRMSNorm.weight must have shape ({student_hidden.shape[1]},), got "
                             f"{tuple(nw.shape)}")
        if not (eps >= 0.0) or eps == float("inf"):
            raise ValueError(f"StudentRMSNorm.eps must be finite and >= 0, got {student_norm.eps}")
    need = [student_hidden.requires_grad, weight.requires_grad,
            t_hidden is not None and t_hidden.requires_grad and mode in ("tied", "separate"),
            t_weight is not None and t_weight.requires_grad and mode == "separate",
            nw is not None and nw.requires_grad]
    outs = fused_loss(
        student_hidden, weight, labels, t_hidden, t_weight, t_logits, tk_i, tk_lp, nw, mode,
        float(student_ce_weight), float(w_t), float(kl_weight), float(kl_temperature), int(ignore_index),
        reduction, div.name, float("nan") if div.alpha is None else float(div.alpha),
        float("nan") if div.beta is None else float(div.beta), need, int(chunk_size or 0), eps,
        logits_gemm == "fp8", _autocast_name(student_hidden.device),
    )
    return DistillationLossOutput(outs[0], outs[1].detach(), outs[2].detach(), outs[3].detach())
