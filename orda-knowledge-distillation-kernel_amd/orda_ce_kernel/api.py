"""Public API (reference ``api.py``): teacher descriptors, ``KernelConfig``,
``DistillationLossOutput``, ``distillation_loss`` and ``DistillationLoss``.

Backends
--------
``backend="auto"`` (default) runs the fused HIP kernels for HIP tensors and
the unfused torch formulation for CPU tensors, as the reference does
(``api.py:385-413``).  Unlike the reference, a HIP tensor never falls back
silently: if ``liborda_ce.so`` cannot be loaded, ``auto`` raises.  With a
``PrecomputedTeacher`` and ``teacher_ce_weight != 0`` the reference's
``auto`` drops to torch; here the HIP path computes that case too.
``backend="triton"`` is kept as the name of the kernel path (there is no
Triton in this build; ``"hip"`` is an alias) and ``backend="torch"`` selects
the unfused formulation explicitly.

``divergence=`` (new, default ``"forward_kl"``) selects the distillation
term; see :mod:`orda_ce_kernel.divergences`.

``TopKTeacher`` (new, no counterpart in the reference) is a precomputed
teacher kept as its k most likely ids and their log-probabilities per token;
see :mod:`orda_ce_kernel.ops.topk_teacher`.  ``student_norm=StudentRMSNorm(w,
eps)`` (new) fuses the student's final RMSNorm in front of the loss:
``student_hidden`` is then the norm's input; ``logits_gemm="fp8"`` (new) runs
the logits GEMM on gfx950's fp8 MFMA (e4m3 operands, one power-of-two scale
per row; gradient GEMMs unchanged); see
:mod:`orda_ce_kernel.ops.rmsnorm_prologue`.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Literal, NamedTuple

import torch
import torch.nn.functional as F
from torch import nn

from ._runtime import HAS_NATIVE, native_error
from .divergences import Divergence, divergence_rows_torch, resolve_divergence
from .utils.dispatcher import dynamic_chunk
from .utils.resolver import DEFAULT_MAX_FUSED_SIZE, _is_auto_chunk_size, is_power_of_two

Reduction = Literal["mean", "sum"]
Profile = Literal["balanced", "debug"]
Backend = Literal["auto", "triton", "hip", "torch"]

__all__ = [
    "DistillationLoss", "DistillationLossOutput", "KernelConfig", "PrecomputedTeacher", "SeparateTeacher",
    "StudentRMSNorm", "TiedTeacher", "TopKTeacher", "distillation_loss",
]


# ── Teacher descriptors (reference api.py:21-52) ─────────────────────────────
@dataclass(frozen=True)
class TiedTeacher:
    """Teacher hidden states that share the student's LM-head weight."""

    hidden: torch.Tensor


@dataclass(frozen=True)
class SeparateTeacher:
    """Teacher hidden states with the teacher's own LM-head weight."""

    hidden: torch.Tensor
    weight: torch.Tensor


@dataclass(frozen=True)
class PrecomputedTeacher:
    """A frozen teacher: its logits, or its (hidden, weight) pair."""

    logits: torch.Tensor | None = None
    teacher_hidden: torch.Tensor | None = None
    teacher_weight: torch.Tensor | None = None

    def __post_init__(self):
        with_logits = self.logits is not None
        with_pair = self.teacher_hidden is not None or self.teacher_weight is not None
        if with_logits and with_pair:
            raise ValueError("PrecomputedTeacher: provide logits or (teacher_hidden, teacher_weight), not both")
        if not with_logits and not with_pair:
            raise ValueError("PrecomputedTeacher: must provide logits or (teacher_hidden, teacher_weight)")
        if with_pair and (self.teacher_hidden is None or self.teacher_weight is None):
            raise ValueError("PrecomputedTeacher: teacher_hidden and teacher_weight must both be provided")


@dataclass(frozen=True)
class TopKTeacher:
    """A precomputed teacher as its top-k (id, log-probability) pairs per
    token: ``indices`` ``[BT, k]`` integer ids, distinct per row, in
    ``[0, V)``; ``logprobs`` ``[BT, k]`` the teacher's log-probabilities at
    those ids (temperature 1).  The distribution it stands for is the teacher
    renormalised over its ids: ``softmax(logprobs / T)`` there, zero
    elsewhere.  Divergences: ``forward_kl`` and ``soft_target_ce``; no
    teacher CE.  Not in the reference, whose precomputed teacher is full
    ``[BT, V]`` logits (``PrecomputedTeacher``).

    The HIP path checks the ids only with ``profile="debug"`` (a host
    synchronisation); otherwise an id outside ``[0, V)`` is clamped to 0 on
    the device and a repeated id in a row races in the dlogits scatter, so
    both give undefined (nondeterministic) gradients.  A row whose
    log-probabilities are all ``-inf`` has no teacher mass: fine on an
    ignored row (it adds nothing), NaN on a counted one."""

    indices: torch.Tensor
    logprobs: torch.Tensor


@dataclass(frozen=True)
class StudentRMSNorm:
    """The student's final RMSNorm, fused in front of the loss:
    ``y = x * rsqrt(mean(x^2, -1) + eps) * weight`` (reference producer,
    ``test/benchmark/src/core.py:7-14``), with ``x`` the ``student_hidden``
    passed to the loss and ``weight`` of shape ``[H]``.  Gradients flow to
    ``x`` and ``weight``.  Not in the reference's loss API."""

    weight: torch.Tensor
    eps: float = 1e-6


def _rmsnorm_torch(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """The reference producer's RMSNorm (``test/benchmark/src/core.py:13-14``)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * weight


def _e4m3_rows(x: torch.Tensor) -> torch.Tensor:
    """Rows scaled by the power of two that puts their amax in (224, 448],
    rounded to ``float8_e4m3fn`` and scaled back (the fp8 logits GEMM's
    operands; no gradient)."""
    x = x.detach()
    amax = x.abs().amax(dim=1)
    m, k = torch.frexp(torch.where(amax > 0, amax, torch.ones_like(amax)))
    e = torch.where(amax > 0, k - 9 + (m > 0.875).to(k.dtype), torch.zeros_like(k))
    sc = torch.ldexp(torch.ones_like(amax), e)[:, None]
    return (x / sc).to(torch.float8_e4m3fn).to(x.dtype) * sc


def _logits_fp8(h: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``h w^T`` with the value of the fp8 GEMM and the gradient of the exact
    one (the kernels form the dlogits from the fp8 logits and run the
    gradient GEMMs on the unrounded operands)."""
    exact = h @ w.t()
    return (_e4m3_rows(h) @ _e4m3_rows(w).t()).detach() + exact - exact.detach()


# ── Config and output types (reference api.py:56-76) ────────────────────────
@dataclass(frozen=True)
class KernelConfig:
    """Tuning knobs.  ``chunk_size`` / ``num_chunks`` / ``max_chunks`` set the
    backward staging chunks; ``max_fused_size`` is validated (power of two)
    and otherwise unused; ``autotune`` is accepted and ignored (the gfx950
    tile is fixed); gradients always accumulate in fp32, so
    ``fp32_grad_weight_accumulation`` has nothing left to switch."""

    fp32_grad_weight_accumulation: bool | None = None
    chunk_size: int | Literal["auto", "dynamic"] | None = None
    num_chunks: int | None = None
    max_chunks: int | None = None
    max_fused_size: int | None = None
    kl_weight: float | None = None
    kl_temperature: float | None = None
    autotune: bool | None = None

    @property
    def effective_fp32_grad_weight_accumulation(self) -> bool:
        return bool(self.fp32_grad_weight_accumulation)


class DistillationLossOutput(NamedTuple):
    loss: torch.Tensor
    student_ce: torch.Tensor
    teacher_ce: torch.Tensor
    kl: torch.Tensor


# ── Config resolution (reference api.py:80-141) ─────────────────────────────
def _resolve_profile(profile: Profile) -> KernelConfig:
    if profile not in ("balanced", "debug"):
        raise ValueError(f"profile must be 'balanced' or 'debug', got {profile!r}")
    return KernelConfig(
        fp32_grad_weight_accumulation=(profile == "debug"),
        max_fused_size=DEFAULT_MAX_FUSED_SIZE,
        autotune=False,
    )


def _resolve_config(profile: Profile, config: KernelConfig | None) -> KernelConfig:
    """Profile defaults overridden field by field by ``config``."""
    base = _resolve_profile(profile)
    if config is None:
        return base
    merged = {
        name: getattr(base, name) if getattr(config, name) is None else getattr(config, name)
        for name in KernelConfig.__dataclass_fields__
    }
    return KernelConfig(**merged)


def _resolve_kl_config(config: KernelConfig, kl_weight: float, kl_temperature: float) -> tuple[float, float]:
    weight = kl_weight if config.kl_weight is None else float(config.kl_weight)
    temperature = kl_temperature if config.kl_temperature is None else float(config.kl_temperature)
    return weight, temperature


def _teacher_mode_and_tensors(teacher):
    if isinstance(teacher, TiedTeacher):
        return "tied", teacher.hidden, None, None
    if isinstance(teacher, SeparateTeacher):
        return "separate", teacher.hidden, teacher.weight, None
    if isinstance(teacher, PrecomputedTeacher):
        return "precomputed", teacher.teacher_hidden, teacher.teacher_weight, teacher.logits
    raise TypeError("teacher must be TiedTeacher, SeparateTeacher, or PrecomputedTeacher")


def _resolve_teacher_ce_weight(mode: str, teacher_ce_weight: float | None) -> float:
    if teacher_ce_weight is not None:
        return float(teacher_ce_weight)
    return 1.0 if mode == "tied" else 0.0


# ── Validation (reference api.py:145-265) ───────────────────────────────────
def _validate_public_args(*, student_hidden, weight, labels, student_ce_weight, teacher_ce_weight, kl_weight,
                          kl_temperature, reduction, backend, config) -> None:
    if student_ce_weight < 0.0:
        raise ValueError(f"student_ce_weight must be >= 0.0, got {student_ce_weight}")
    if teacher_ce_weight is not None and teacher_ce_weight < 0.0:
        raise ValueError(f"teacher_ce_weight must be >= 0.0, got {teacher_ce_weight}")
    if kl_weight < 0.0:
        raise ValueError(f"kl_weight must be >= 0.0, got {kl_weight}")
    if kl_temperature <= 0.0:
        raise ValueError(f"kl_temperature must be > 0.0, got {kl_temperature}")
    if reduction not in ("mean", "sum"):
        raise ValueError(f"reduction must be 'mean' or 'sum', got {reduction!r}")
    if backend not in ("auto", "triton", "hip", "torch"):
        raise ValueError(f"backend must be 'auto', 'triton', 'hip', or 'torch', got {backend!r}")
    if student_hidden.ndim != 2:
        raise ValueError(f"student_hidden must be 2D, got shape={tuple(student_hidden.shape)}")
    BT, H = student_hidden.shape
    if weight.ndim != 2 or weight.shape[1] != H:
        raise ValueError(f"weight must have shape (vocab, {H}), got {tuple(weight.shape)}")
    if labels.shape != (BT,):
        raise ValueError(f"labels must have shape ({BT},), got {tuple(labels.shape)}")
    if labels.dtype != torch.long:
        raise ValueError(f"labels must have dtype torch.long, got {labels.dtype}")
    if config.max_chunks is not None and config.max_chunks < 1:
        raise ValueError(f"config.max_chunks must be >= 1, got {config.max_chunks}")
    if config.num_chunks is not None and config.num_chunks < 1:
        raise ValueError(f"config.num_chunks must be >= 1, got {config.num_chunks}")
    if config.num_chunks is not None and not _is_auto_chunk_size(config.chunk_size):
        raise ValueError("config.chunk_size and config.num_chunks are mutually exclusive")
    if config.num_chunks is not None and config.max_chunks is not None:
        if min(int(config.num_chunks), BT) > config.max_chunks:
            raise ValueError(
                f"config.num_chunks must be <= config.max_chunks, got "
                f"num_chunks={config.num_chunks}, max_chunks={config.max_chunks}"
            )
    if config.max_fused_size < 1:
        raise ValueError(f"config.max_fused_size must be >= 1, got {config.max_fused_size}")
    if not is_power_of_two(int(config.max_fused_size)):
        raise ValueError(f"config.max_fused_size must be a power of two, got {config.max_fused_size}")


def _validate_teacher(*, mode, teacher_hidden, teacher_weight, teacher_logits, student_hidden, weight) -> None:
    BT, H = student_hidden.shape
    V = weight.shape[0]
    if mode == "tied":
        if teacher_hidden.shape != (BT, H):
            raise ValueError(f"TiedTeacher.hidden must have shape {(BT, H)}, got {tuple(teacher_hidden.shape)}")
        return
    if mode == "separate":
        if teacher_hidden.ndim != 2 or teacher_hidden.shape[0] != BT:
            raise ValueError(
                f"SeparateTeacher.hidden must have shape (BT, teacher_hidden_dim), got {tuple(teacher_hidden.shape)}"
            )
        if teacher_weight.shape != (V, teacher_hidden.shape[1]):
            raise ValueError(
                f"SeparateTeacher.weight must have shape {(V, teacher_hidden.shape[1])}, "
                f"got {tuple(teacher_weight.shape)}"
            )
        return
    if teacher_logits is not None:
        if teacher_logits.shape != (BT, V):
            raise ValueError(
                f"PrecomputedTeacher.logits must have shape {(BT, V)}, got {tuple(teacher_logits.shape)}"
            )
        if teacher_logits.requires_grad:
            raise ValueError(
                "PrecomputedTeacher.logits must not require gradients; use SeparateTeacher "
                "when the teacher path needs gradients"
            )
        return
    if teacher_hidden is None or teacher_weight is None:
        raise ValueError("PrecomputedTeacher requires logits or (teacher_hidden, teacher_weight)")
    if teacher_hidden.ndim != 2 or teacher_hidden.shape[0] != BT:
        raise ValueError(
            f"PrecomputedTeacher.teacher_hidden must have shape (BT, D_t), got {tuple(teacher_hidden.shape)}"
        )
    if teacher_weight.shape != (V, teacher_hidden.shape[1]):
        raise ValueError(
            f"PrecomputedTeacher.teacher_weight must have shape {(V, teacher_hidden.shape[1])}, "
            f"got {tuple(teacher_weight.shape)}"
        )
    if teacher_hidden.requires_grad or teacher_weight.requires_grad:
        raise ValueError("PrecomputedTeacher.teacher_hidden and teacher_weight must not require gradients")


# ── Unfused torch formulation (reference api.py:274-335) ────────────────────
def _torch_reference(*, student_hidden, weight, labels, teacher, student_ce_weight, teacher_ce_weight, kl_weight,
                     kl_temperature, ignore_index, reduction, divergence: Divergence | None = None,
                     fp8_logits: bool = False):
    """Materialises full logits and lets autograd differentiate.  Used for
    ``backend="torch"`` and CPU tensors; the divergence term is computed even
    when ``kl_weight == 0`` (reported, not weighted), as in the reference.
    ``fp8_logits``: the student's (and a tied teacher's) logits take the fp8
    GEMM's values (``_logits_fp8``)."""
    div = resolve_divergence(divergence)
    mode, t_hidden, t_weight, t_logits = _teacher_mode_and_tensors(teacher)
    logits_s = _logits_fp8(student_hidden, weight) if fp8_logits else student_hidden @ weight.t()
    if mode == "tied":
        logits_t = _logits_fp8(t_hidden, weight) if fp8_logits else t_hidden @ weight.t()
    elif mode == "separate":
        logits_t = t_hidden @ t_weight.t()
    elif t_logits is not None:
        logits_t = t_logits.detach()
    else:
        logits_t = (t_hidden @ t_weight.t()).detach()

    ce_s_rows = F.cross_entropy(logits_s, labels, ignore_index=ignore_index, reduction="none")
    ce_t_rows = F.cross_entropy(logits_t, labels, ignore_index=ignore_index, reduction="none")
    keep = labels != ignore_index
    denom = keep.sum().clamp(min=1)

    T = float(kl_temperature)
    log_p_s = F.log_softmax(logits_s / T, dim=-1)
    log_p_t = F.log_softmax(logits_t.detach() / T, dim=-1)
    d_rows = (divergence_rows_torch(log_p_s, log_p_t, div) * (T * T)).masked_fill(~keep, 0.0)

    if reduction == "mean":
        student_ce, teacher_ce_all, kl = ce_s_rows.sum() / denom, ce_t_rows.sum() / denom, d_rows.sum() / denom
    else:
        student_ce, teacher_ce_all, kl = ce_s_rows.sum(), ce_t_rows.sum(), d_rows.sum()
    teacher_ce = teacher_ce_all if teacher_ce_weight != 0.0 else student_ce.new_zeros(())
    loss = student_ce_weight * student_ce + teacher_ce_weight * teacher_ce + kl_weight * kl
    return DistillationLossOutput(loss, student_ce.detach(), teacher_ce.detach(), kl.detach())


def _torch_topk_reference(*, student_hidden, weight, labels, teacher: TopKTeacher, student_ce_weight, kl_weight,
                          kl_temperature, ignore_index, reduction, divergence: Divergence):
    """The top-k teacher's loss, unfused (CPU tensors, ``backend="torch"``):
    student CE plus ``T^2 D(p_t || p_s)`` with ``p_t = softmax(logprobs / T)``
    on the ids and zero elsewhere -- forward KL ``sum p_t (log p_t - log
    p_s^T)`` or soft-target CE ``-sum p_t log p_s^T`` over the ids."""
    logits_s = student_hidden @ weight.t()
    ce_s_rows = F.cross_entropy(logits_s, labels, ignore_index=ignore_index, reduction="none")
    keep = labels != ignore_index
    denom = keep.sum().clamp(min=1)
    T = float(kl_temperature)
    log_p_s = F.log_softmax(logits_s / T, dim=-1)
    lps_k = log_p_s.gather(1, teacher.indices.long())
    # ignored rows add nothing; their teacher (padding tokens may carry only
    # -inf log-probabilities) is replaced by a finite one so that no NaN
    # reaches the gradients through the masked rows
    lp_t = teacher.logprobs.detach().to(lps_k.dtype).masked_fill(~keep[:, None], 0.0)
    p_t = F.softmax(lp_t / T, dim=-1)
    cross = -(p_t * lps_k).sum(-1)
    d = cross + torch.xlogy(p_t, p_t).sum(-1) if divergence.name == "forward_kl" else cross
    d_rows = (d * (T * T)).masked_fill(~keep, 0.0)
    if reduction == "mean":
        student_ce, kl = ce_s_rows.sum() / denom, d_rows.sum() / denom
    else:
        student_ce, kl = ce_s_rows.sum(), d_rows.sum()
    loss = student_ce_weight * student_ce + kl_weight * kl
    return DistillationLossOutput(loss, student_ce.detach(), student_ce.new_zeros(()), kl.detach())


def _topk_loss(*, student_hidden, weight, labels, teacher: TopKTeacher, teacher_ce_weight, student_ce_weight,
               kl_weight, kl_temperature, ignore_index, reduction, profile, backend, resolved: KernelConfig,
               divergence: Divergence) -> DistillationLossOutput:
    from .ops.topk_teacher import check_topk_teacher, topk_distillation_loss

    if teacher_ce_weight not in (None, 0.0):
        raise ValueError("a TopKTeacher has no teacher CE: teacher_ce_weight must be None or 0.0")
    BT, V = student_hidden.shape[0], weight.shape[0]
    check_topk_teacher(teacher.indices, teacher.logprobs, BT, V, divergence)
    if teacher.indices.device != student_hidden.device or teacher.logprobs.device != student_hidden.device:
        raise ValueError("TopKTeacher tensors must be on the student's device")
    if profile == "debug":
        idx = teacher.indices.long()
        if bool(((idx < 0) | (idx >= V)).any()):
            raise ValueError(f"TopKTeacher.indices must lie in [0, {V})")
        srt = idx.sort(dim=1).values
        if bool((srt[:, 1:] == srt[:, :-1]).any()):
            raise ValueError("TopKTeacher.indices must be distinct within each row")
    if backend == "torch" or (backend == "auto" and student_hidden.device.type != "cuda"):
        return _torch_topk_reference(
            student_hidden=student_hidden, weight=weight, labels=labels, teacher=teacher,
            student_ce_weight=student_ce_weight, kl_weight=kl_weight, kl_temperature=kl_temperature,
            ignore_index=ignore_index, reduction=reduction, divergence=divergence,
        )
    if not _supports_native(student_hidden):
        raise RuntimeError(
            f"backend={backend!r} on {student_hidden.device} tensors requires the HIP extension liborda_ce.so "
            f"({native_error() or 'loaded'}); pass backend='torch' to run the unfused PyTorch formulation"
        )
    from .utils.resolver import resolve_chunk_size

    cs, _ = resolve_chunk_size(BT, resolved.chunk_size, V=V, max_chunks=resolved.max_chunks,
                               num_chunks=resolved.num_chunks)
    out = topk_distillation_loss(
        student_hidden, weight, teacher.indices, teacher.logprobs, labels, student_ce_weight=student_ce_weight,
        ignore_index=ignore_index, reduction=reduction, chunk_size=cs, kl_weight=kl_weight,
        kl_temperature=kl_temperature, max_chunks=resolved.max_chunks, max_fused_size=resolved.max_fused_size,
        validate_labels=profile == "debug", divergence=divergence,
    )
    return DistillationLossOutput(*out)


def _extended_loss(*, x, weight, labels, teacher, norm: StudentRMSNorm | None, fp8: bool, kw: dict, profile,
                   backend, resolved: KernelConfig, divergence: Divergence) -> DistillationLossOutput:
    """``student_norm=`` and/or ``logits_gemm="fp8"``: the unfused torch
    formulation on CPU tensors (or ``backend="torch"``), else the extension
    Function on the HIP path."""
    nw, eps = None, 1e-6
    if norm is not None:
        if not isinstance(norm, StudentRMSNorm):
            raise TypeError(f"student_norm must be a StudentRMSNorm, got {type(norm).__name__}")
        nw = norm.weight
        H = x.shape[1]
        if not isinstance(nw, torch.Tensor) or nw.ndim != 1 or nw.shape[0] != H or not nw.is_floating_point():
            raise ValueError(f"StudentRMSNorm.weight must be a floating tensor of shape ({H},), got "
                             f"{getattr(nw, 'shape', None)}")
        if nw.device != x.device:
            raise ValueError("StudentRMSNorm.weight must be on the student's device")
        eps = float(norm.eps)
        if not (eps >= 0.0) or eps == float("inf"):
            raise ValueError(f"StudentRMSNorm.eps must be finite and >= 0, got {norm.eps}")
    if fp8 and isinstance(teacher, TopKTeacher):
        raise ValueError("logits_gemm='fp8' does not support a TopKTeacher")
    if backend == "torch" or (backend == "auto" and x.device.type != "cuda"):
        y = _rmsnorm_torch(x, nw, eps) if nw is not None else x
        if not fp8:
            return distillation_loss(y, weight, labels, teacher, profile=profile, backend="torch", config=resolved,
                                     divergence=divergence, **kw)
        mode = _teacher_mode_and_tensors(teacher)[0]
        return _torch_reference(
            student_hidden=y, weight=weight, labels=labels, teacher=teacher,
            student_ce_weight=kw["student_ce_weight"], teacher_ce_weight=_resolve_teacher_ce_weight(
                mode, kw["teacher_ce_weight"]), kl_weight=kw["kl_weight"], kl_temperature=kw["kl_temperature"],
            ignore_index=kw["ignore_index"], reduction=kw["reduction"], divergence=divergence, fp8_logits=True,
        )
    if not _supports_native(x):
        raise RuntimeError(
            f"backend={backend!r} on {x.device} tensors requires the HIP extension liborda_ce.so "
            f"({native_error() or 'loaded'}); pass backend='torch' to run the unfused PyTorch formulation"
        )
    from .ops.rmsnorm_prologue import NormedCall, RMSNormPrologueFunction
    from .utils.resolver import resolve_chunk_size

    w_t_arg = kw["teacher_ce_weight"]
    t_logits = tk_i = tk_lp = t_hidden = t_weight = None
    if isinstance(teacher, TopKTeacher):
        from .ops.topk_teacher import check_topk_teacher

        if w_t_arg not in (None, 0.0):
            raise ValueError("a TopKTeacher has no teacher CE: teacher_ce_weight must be None or 0.0")
        check_topk_teacher(teacher.indices, teacher.logprobs, x.shape[0], weight.shape[0], divergence)
        mode, w_t, tk_i, tk_lp = "topk", 0.0, teacher.indices, teacher.logprobs
    else:
        mode, t_hidden, t_weight, t_logits = _teacher_mode_and_tensors(teacher)
        _validate_teacher(mode=mode, teacher_hidden=t_hidden, teacher_weight=t_weight, teacher_logits=t_logits,
                          student_hidden=x, weight=weight)
        w_t = _resolve_teacher_ce_weight(mode, w_t_arg)
        if mode == "precomputed":
            mode = "precomputed_logits" if t_logits is not None else "precomputed_hidden"
    if profile == "debug":
        from .ops._checks import check_labels_in_range

        check_labels_in_range(labels, weight.shape[0], kw["ignore_index"])
    cs, _ = resolve_chunk_size(x.shape[0], resolved.chunk_size, V=weight.shape[0], max_chunks=resolved.max_chunks,
                               num_chunks=resolved.num_chunks)
    spec = NormedCall(
        mode=mode, teacher_logits=t_logits, topk_indices=tk_i, topk_logprobs=tk_lp,
        student_ce_weight=float(kw["student_ce_weight"]), teacher_ce_weight=float(w_t),
        kl_weight=float(kw["kl_weight"]), kl_temperature=float(kw["kl_temperature"]),
        ignore_index=int(kw["ignore_index"]), reduction=kw["reduction"], divergence=divergence,
        token_chunk=int(cs), eps=eps, fp8_logits=fp8,
    )
    out = RMSNormPrologueFunction.apply(x, nw, weight, t_hidden, t_weight, labels, spec)
    return DistillationLossOutput(*out)


def _supports_native(student_hidden: torch.Tensor) -> bool:
    return bool(HAS_NATIVE and student_hidden.device.type == "cuda")


# ── Functional API (reference api.py:339-437) ───────────────────────────────
@torch._dynamo.disable
def distillation_loss(
    student_hidden: torch.Tensor,
    weight: torch.Tensor,
    labels: torch.Tensor,
    teacher: TiedTeacher | SeparateTeacher | PrecomputedTeacher | TopKTeacher,
    *,
    student_ce_weight: float = 1.0,
    teacher_ce_weight: float | None = None,
    kl_weight: float = 0.0,
    kl_temperature: float = 1.0,
    ignore_index: int = -100,
    reduction: Reduction = "mean",
    profile: Profile = "balanced",
    backend: Backend = "auto",
    config: KernelConfig | None = None,
    divergence: str | Divergence = "forward_kl",
    student_norm: StudentRMSNorm | None = None,
    logits_gemm: Literal["default", "fp8"] = "default",
) -> DistillationLossOutput:
    """Fused LM-head CE + distillation loss.

    ``loss = student_ce_weight * CE(student) + teacher_ce_weight * CE(teacher)
    + kl_weight * T^2 * D(teacher || student)`` over non-ignored rows, mean or
    sum.  ``teacher_ce_weight`` defaults to 1.0 for a tied teacher and 0.0
    otherwise.  Only ``loss`` carries gradients.
    """
    resolved = _resolve_config(profile, config)
    kl_w, kl_t = _resolve_kl_config(resolved, kl_weight, kl_temperature)
    _validate_public_args(
        student_hidden=student_hidden, weight=weight, labels=labels, student_ce_weight=student_ce_weight,
        teacher_ce_weight=teacher_ce_weight, kl_weight=kl_w, kl_temperature=kl_t, reduction=reduction,
        backend=backend, config=resolved,
    )
    div = resolve_divergence(divergence)
    if logits_gemm not in ("default", "fp8"):
        raise ValueError(f"logits_gemm must be 'default' or 'fp8', got {logits_gemm!r}")
    if student_norm is not None or logits_gemm == "fp8":
        kw = dict(student_ce_weight=student_ce_weight, teacher_ce_weight=teacher_ce_weight, kl_weight=kl_w,
                  kl_temperature=kl_t, ignore_index=ignore_index, reduction=reduction)
        return _extended_loss(x=student_hidden, weight=weight, labels=labels, teacher=teacher, norm=student_norm,
                              fp8=logits_gemm == "fp8", kw=kw, profile=profile, backend=backend, resolved=resolved,
                              divergence=div)
    if isinstance(teacher, TopKTeacher):
        return _topk_loss(
            student_hidden=student_hidden, weight=weight, labels=labels, teacher=teacher,
            teacher_ce_weight=teacher_ce_weight, student_ce_weight=student_ce_weight, kl_weight=kl_w,
            kl_temperature=kl_t, ignore_index=ignore_index, reduction=reduction, profile=profile, backend=backend,
            resolved=resolved, divergence=div,
        )
    mode, t_hidden, t_weight, t_logits = _teacher_mode_and_tensors(teacher)
    _validate_teacher(
        mode=mode, teacher_hidden=t_hidden, teacher_weight=t_weight, teacher_logits=t_logits,
        student_hidden=student_hidden, weight=weight,
    )
    w_t = _resolve_teacher_ce_weight(mode, teacher_ce_weight)
    on_device = student_hidden.device.type == "cuda"

    if backend == "triton" and mode == "precomputed" and w_t != 0.0:
        raise ValueError("backend='triton' with PrecomputedTeacher requires teacher_ce_weight=0.0")
    if backend == "torch" or (backend == "auto" and not on_device):
        return _torch_reference(
            student_hidden=student_hidden, weight=weight, labels=labels, teacher=teacher,
            student_ce_weight=student_ce_weight, teacher_ce_weight=w_t, kl_weight=kl_w, kl_temperature=kl_t,
            ignore_index=ignore_index, reduction=reduction, divergence=div,
        )
    if not _supports_native(student_hidden):
        raise RuntimeError(
            f"backend={backend!r} on {student_hidden.device} tensors requires the HIP extension liborda_ce.so "
            f"({native_error() or 'loaded'}); on a HIP device this build never falls back silently, pass "
            "backend='torch' to run the unfused PyTorch formulation explicitly"
        )

    common = dict(
        student_ce_weight=student_ce_weight, ignore_index=ignore_index, reduction=reduction,
        chunk_size=resolved.chunk_size, num_chunks=resolved.num_chunks,
        use_fp32_accum=resolved.effective_fp32_grad_weight_accumulation, kl_weight=kl_w, kl_temperature=kl_t,
        max_chunks=resolved.max_chunks, max_fused_size=resolved.max_fused_size, autotune=resolved.autotune,
        teacher_ce_weight=w_t, validate_labels=profile == "debug", divergence=div,
    )
    if mode == "precomputed" and w_t != 0.0:
        from .ops.precomputed_teacher import precomputed_distillation_loss_with_teacher_ce
        from .utils.resolver import resolve_chunk_size

        cs, _ = resolve_chunk_size(
            student_hidden.shape[0], resolved.chunk_size, V=weight.shape[0], max_chunks=resolved.max_chunks,
            num_chunks=resolved.num_chunks,
        )
        common.pop("num_chunks")
        common["chunk_size"] = cs
        out = precomputed_distillation_loss_with_teacher_ce(
            student_hidden, weight, t_logits, labels, teacher_hidden=t_hidden, teacher_weight=t_weight, **common
        )
        return DistillationLossOutput(*out)
    out = dynamic_chunk(
        student_hidden, t_hidden, weight, labels, teacher_mode=mode, teacher_weight=t_weight,
        logits_teacher=t_logits, **common,
    )
    return DistillationLossOutput(*out)


# ── Module wrapper (reference api.py:441-486) ───────────────────────────────
class DistillationLoss(nn.Module):
    def __init__(
        self,
        *,
        student_ce_weight: float = 1.0,
        teacher_ce_weight: float | None = None,
        kl_weight: float = 0.0,
        kl_temperature: float = 1.0,
        ignore_index: int = -100,
        reduction: Reduction = "mean",
        profile: Profile = "balanced",
        backend: Backend = "auto",
        config: KernelConfig | None = None,
        divergence: str | Divergence = "forward_kl",
        logits_gemm: Literal["default", "fp8"] = "default",
    ) -> None:
        super().__init__()
        self.logits_gemm = logits_gemm
        self.student_ce_weight = student_ce_weight
        self.teacher_ce_weight = teacher_ce_weight
        self.kl_weight = kl_weight
        self.kl_temperature = kl_temperature
        self.ignore_index = ignore_index
        self.reduction = reduction
        self.profile = profile
        self.backend = backend
        self.config = config
        self.divergence = divergence

    def forward(self, student_hidden, weight, labels, teacher, student_norm=None) -> DistillationLossOutput:
        return distillation_loss(
            student_hidden, weight, labels, teacher,
            student_ce_weight=self.student_ce_weight, teacher_ce_weight=self.teacher_ce_weight,
            kl_weight=self.kl_weight, kl_temperature=self.kl_temperature, ignore_index=self.ignore_index,
            reduction=self.reduction, profile=self.profile, backend=self.backend, config=self.config,
            divergence=self.divergence, student_norm=student_norm, logits_gemm=self.logits_gemm,
        )
