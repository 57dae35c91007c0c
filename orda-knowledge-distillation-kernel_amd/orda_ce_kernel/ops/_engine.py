"""Host side of the fused HIP path, shared by the four autograd Functions.

Two schedules, chosen per call by :func:`grads_in_forward`:

* gradients inside forward (the reference's schedule,
  ``ops/tied_teacher.py:366-516,531-564``; default for tied and separate
  teachers when ``fp32_grad_weight_accumulation`` is off): ``orda_forward``
  walks token chunks, materialises each chunk's logits in a workspace,
  turns them into dlogits in place and multiplies them into the gradients,
  accumulating grad W across chunks in the weight dtype as the reference's
  ``addmm_`` does; backward only multiplies by ``grad_output`` (in place,
  once: a second backward through a retained graph recomputes the
  gradients rather than rescale tensors already handed out);
* two-phase (``fp32_grad_weight_accumulation=True``, precomputed logits
  in another dtype than the compute dtype, and forward-only calls):
  ``orda_forward``
  computes the losses with an online-softmax scan (no logits stored) and
  ``orda_backward`` recomputes the logits per vocabulary chunk, so every
  grad W element is one fp32-accumulated GEMM rounded once.

PyTorch allocates every buffer (outputs, the saved statistics, workspaces),
so an out-of-memory error is a ``torch.cuda.OutOfMemoryError`` that the
dispatcher's retry understands.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .. import _native
from .._runtime import HAS_NATIVE, native_error
from ..divergences import Divergence, resolve_divergence

__all__ = ["FusedCall", "cast_to", "fused_forward", "fused_backward", "run_fused_call", "vocab_chunk_for",
           "require_native",
           "grads_in_forward", "token_chunk_for"]


def require_native(entry: str) -> None:
    """Raise RuntimeError when the HIP library cannot be used."""
    if not HAS_NATIVE:
        raise RuntimeError(
            f"{entry} requires the HIP extension liborda_ce.so and HIP tensors "
            f"({native_error()}). Use distillation_loss(..., backend='auto' or 'torch') for fallback execution."
        )


def vocab_chunk_for(BT: int, V: int, chunk_size, max_chunks) -> int:
    """Vocabulary columns per backward chunk.

    The reference splits the tokens into ``num_chunks`` chunks of logits
    (``utils/resolver.py:28-62``); this build splits the vocabulary into the
    same number of chunks, so the staging memory scales the same way with the
    chunk settings and the OOM retry (which doubles ``num_chunks``) halves it.
    """
    from ..utils.resolver import resolve_chunk_size

    _, num_chunks = resolve_chunk_size(BT, chunk_size, V=V, max_chunks=max_chunks)
    return -(-int(V) // int(num_chunks))


def token_chunk_for(chunk_size) -> int:
    """Requested tokens per chunk of the gradients-in-forward schedule: the
    reference's chunk (``utils/resolver.py:28-62``, as the dispatcher passes
    it).  The library's chunk is this times the gfx950 launch table's scale
    (2, or 4 when precomputed logits are read in place): a chunk keeps only
    its 16-bit logits in HBM, and the dispatcher's OOM retry, which halves
    the chunk, still halves it.  0 lets the library choose."""
    if chunk_size is None or isinstance(chunk_size, str):
        return 0
    return int(chunk_size)


# Launch overrides for tuning sweeps (bench.py --splits): fields of
# orda_problem_t set on every call when not None.  None = the launch table.
LAUNCH_OVERRIDES: dict[str, int | None] = {"grad_hidden_splits": None}


def grads_in_forward(mode: str, use_fp32_accum, divergence, any_grad: bool) -> bool:
    """Whether a call takes the gradients-in-forward schedule.

    Every mode may (precomputed teachers get no gradient; their logits are
    stored beside the student's for the chunk's dlogits, so the precomputed
    logits caller checks that their dtype is the compute dtype).
    """
    if not any_grad or bool(use_fp32_accum):
        return False
    return mode in ("tied", "separate", "precomputed_logits", "precomputed_hidden")


def _kelems(dtype: torch.dtype) -> int:
    return 4 if dtype == torch.float32 else 8


def _pad_cols(x: torch.Tensor, mult: int) -> torch.Tensor:
    """Zero-pad the last dimension to a multiple of ``mult`` (zero columns do
    not change any dot product) and make the base 16-byte aligned."""
    pad = (-x.shape[-1]) % mult
    if pad:
        x = F.pad(x, (0, pad))
    if x.data_ptr() % 16 != 0:
        x = x.clone()
    return x


def _ptr(x: torch.Tensor | None):
    return None if x is None else x.data_ptr()


@dataclass
class FusedCall:
    """Everything one fused loss evaluation needs (built by the Functions)."""

    mode: str                         # tied / separate / precomputed_logits / precomputed_hidden / topk
    student_hidden: torch.Tensor
    weight: torch.Tensor
    labels: torch.Tensor
    teacher_hidden: torch.Tensor | None
    teacher_weight: torch.Tensor | None
    teacher_logits: torch.Tensor | None
    student_ce_weight: float
    teacher_ce_weight: float
    kl_weight: float
    kl_temperature: float
    ignore_index: int
    reduction: str
    vocab_chunk: int
    divergence: Divergence
    compute_teacher_ce: bool
    need_grad_student_hidden: bool
    need_grad_weight: bool
    need_grad_teacher_hidden: bool = False
    need_grad_teacher_weight: bool = False
    grads_in_forward: bool = False
    token_chunk: int = 0
    topk_indices: torch.Tensor | None = None   # mode "topk": [N x k] int64
    topk_logprobs: torch.Tensor | None = None  # mode "topk": [N x k] fp32
    # the student's final RMSNorm fused in front of the loss: student_hidden
    # is then its input x and this its weight [H] (compute dtype)
    student_norm_weight: torch.Tensor | None = None
    norm_eps: float = 1e-6
    need_grad_student_norm_weight: bool = False
    # the scan's logits GEMM on e4m3 operands with per-row power-of-two scales
    fp8_logits: bool = False


def _problem(call: FusedCall, H: int, Ht: int, logits_dtype: torch.dtype | None) -> _native.Problem:
    flags = 0
    if call.need_grad_student_hidden:
        flags |= _native.FLAG["need_grad_student_hidden"]
    if call.need_grad_weight:
        flags |= _native.FLAG["need_grad_weight"]
    if call.need_grad_teacher_hidden:
        flags |= _native.FLAG["need_grad_teacher_hidden"]
    if call.need_grad_teacher_weight:
        flags |= _native.FLAG["need_grad_teacher_weight"]
    if call.compute_teacher_ce:
        flags |= _native.FLAG["compute_teacher_ce"]
    if float(call.kl_weight) != 0.0:
        flags |= _native.FLAG["compute_divergence"]
    if call.reduction == "sum":
        flags |= _native.FLAG["reduction_sum"]
    if call.grads_in_forward:
        flags |= _native.FLAG["grads_in_forward"]
    if call.fp8_logits:
        flags |= _native.FLAG["fp8_logits"]
    if call.student_norm_weight is not None:
        flags |= _native.FLAG["student_rmsnorm"]
        if call.need_grad_student_norm_weight:
            flags |= _native.FLAG["need_grad_student_norm_weight"]
    div = call.divergence
    p = _native.Problem()
    p.abi_version = _native.ABI_VERSION
    p.mode = _native.MODE[call.mode]
    p.dtype = _native.DTYPE[call.student_hidden.dtype]
    p.logits_dtype = _native.DTYPE[logits_dtype] if logits_dtype is not None else 0
    p.n_rows = call.student_hidden.shape[0]
    p.vocab = call.weight.shape[0]
    p.hidden = H
    p.teacher_hidden = Ht
    p.ignore_index = int(call.ignore_index)
    p.vocab_chunk = int(call.vocab_chunk)
    p.flags = flags
    p.divergence = div.code
    p.temperature = float(call.kl_temperature)
    p.student_ce_weight = float(call.student_ce_weight)
    p.teacher_ce_weight = float(call.teacher_ce_weight) if call.compute_teacher_ce else 0.0
    p.kl_weight = float(call.kl_weight)
    p.div_alpha = float(div.alpha) if div.alpha is not None else 0.0
    p.div_beta = float(div.beta) if div.beta is not None else 0.0
    p.token_chunk = int(call.token_chunk)
    splits = LAUNCH_OVERRIDES.get("grad_hidden_splits")
    p.grad_hidden_splits = int(splits) if splits else 0
    p.topk = int(call.topk_indices.shape[1]) if call.topk_indices is not None else 0
    if call.student_norm_weight is not None:
        p.norm_dim = int(call.student_hidden.shape[1])  # the unpadded hidden size
        p.norm_eps = float(call.norm_eps)
    return p


def fused_forward(ctx, call: FusedCall):
    """Run the fused forward; stash what backward needs on ``ctx``.

    Inputs must already be contiguous and in the compute dtype (the
    Functions do that, as the reference does at ``ops/tied_teacher.py:334-344``).
    Returns ``(loss, student_ce, teacher_ce, kl)`` as fp32 0-dim tensors.
    """
    outs, grads, state = run_fused_call(call)
    problem, (H, Ht), inputs, saved = state
    ctx.orda_problem = problem
    ctx.orda_shapes = (H, Ht)
    ctx.orda_mode = call.mode
    ctx.save_for_backward(*inputs, saved)
    # Gradients computed in forward: the first backward scales them in place
    # and hands them to autograd, dropping this reference (so autograd can
    # keep the buffers as .grad without a copy); a later backward through a
    # retained graph recomputes them, so no returned tensor is ever scaled
    # twice.
    ctx.orda_grads = grads if call.grads_in_forward else None
    return tuple(outs)


def run_fused_call(call: FusedCall):
    """orda_forward for ``call`` without autograd state.  Returns ``(outs,
    grads, state)``: the four fp32 0-dim losses, the four gradients (None
    where not computed; padded columns included) and ``(problem, (H, Ht),
    padded inputs, saved)`` for a later backward."""
    require_native("the fused HIP path")
    dev = call.student_hidden.device
    if dev.type != "cuda":
        raise ValueError(f"tensors must be CUDA/HIP tensors, got device={dev}")
    call.divergence = resolve_divergence(call.divergence)
    mult = _kelems(call.student_hidden.dtype)
    H = call.student_hidden.shape[1]
    hs = _pad_cols(call.student_hidden, mult)
    w = _pad_cols(call.weight, mult)
    ht = wt = lt = None
    Ht = H
    if call.mode == "tied":
        ht = _pad_cols(call.teacher_hidden, mult)
    elif call.mode in ("separate", "precomputed_hidden"):
        Ht = call.teacher_hidden.shape[1]
        ht = _pad_cols(call.teacher_hidden, mult)
        wt = _pad_cols(call.teacher_weight, mult)
    elif call.mode == "precomputed_logits":
        lt = call.teacher_logits.contiguous()
        if lt.dtype not in _native.DTYPE:
            lt = lt.float()
        if lt.data_ptr() % 16 != 0:  # the kernels read 16-byte rows in place
            lt = lt.clone()
    labels = call.labels.contiguous()
    tk_i = tk_lp = None
    if call.mode == "topk":
        # the kernels read N x k int64 ids and fp32 log-probs on this device
        tk_i = call.topk_indices.contiguous()
        tk_lp = call.topk_logprobs.contiguous()
        n = call.student_hidden.shape[0]
        if (tk_i.dtype != torch.int64 or tk_lp.dtype != torch.float32 or tk_i.ndim != 2 or tk_i.shape[0] != n
                or tk_lp.shape != tk_i.shape or tk_i.device != dev or tk_lp.device != dev):
            raise ValueError("top-k teacher: indices must be int64 and logprobs float32, both [N, k] on "
                             f"{dev}; got {tk_i.dtype} {tuple(tk_i.shape)} on {tk_i.device}, "
                             f"{tk_lp.dtype} {tuple(tk_lp.shape)} on {tk_lp.device}")
    nw = None
    if call.student_norm_weight is not None:
        # padded like the hidden rows: zero weight on zero columns
        nw = _pad_cols(call.student_norm_weight.reshape(1, -1), mult).reshape(-1)
        if nw.dtype != hs.dtype or nw.device != dev:
            raise ValueError(f"student_norm_weight must be {hs.dtype} on {dev}, got {nw.dtype} on {nw.device}")
    Hp = hs.shape[1]
    Htp = ht.shape[1] if (ht is not None and call.mode != "tied") else Hp
    problem = _problem(call, Hp, Htp, lt.dtype if lt is not None else None)

    saved = torch.empty(_native.saved_bytes(problem), dtype=torch.uint8, device=dev)
    outs = [torch.empty((), dtype=torch.float32, device=dev) for _ in range(4)]
    grads = _alloc_grads(problem.flags, hs, w, ht, wt, nw) if call.grads_in_forward else (None,) * 5
    inputs = (hs, w, ht, wt, lt, labels, tk_i, tk_lp, nw)
    _run_forward(problem, inputs, saved, outs, grads)
    return outs, grads, (problem, (H, Ht), inputs, saved)


def _run_forward(problem, inputs, saved, outs, grads) -> None:
    """One orda_forward call with a fresh workspace (freed on return)."""
    hs, w, ht, wt, lt, labels, tk_i, tk_lp, nw = inputs
    ws = torch.empty(_native.forward_workspace_bytes(problem), dtype=torch.uint8, device=hs.device)
    t = _native.Tensors()
    t.student_hidden, t.weight, t.labels = _ptr(hs), _ptr(w), _ptr(labels)
    t.teacher_hidden, t.teacher_weight, t.teacher_logits = _ptr(ht), _ptr(wt), _ptr(lt)
    t.teacher_topk_indices, t.teacher_topk_logprobs = _ptr(tk_i), _ptr(tk_lp)
    t.student_norm_weight = _ptr(nw)
    t.out_loss, t.out_student_ce, t.out_teacher_ce, t.out_kl = (o.data_ptr() for o in outs)
    t.saved = saved.data_ptr()
    t.grad_student_hidden, t.grad_weight, t.grad_teacher_hidden, t.grad_teacher_weight = (_ptr(g) for g in grads[:4])
    t.grad_student_norm_weight = _ptr(grads[4])
    _native.forward(problem, t, ws)
    del ws


def _alloc_grads(flags: int, hs, w, ht, wt, nw=None):
    need = lambda name: bool(flags & _native.FLAG[name])  # noqa: E731
    g_hs = torch.empty_like(hs) if need("need_grad_student_hidden") else None
    g_w = torch.empty_like(w) if need("need_grad_weight") else None
    g_ht = torch.empty_like(ht) if (need("need_grad_teacher_hidden") and ht is not None) else None
    g_wt = torch.empty_like(wt) if (need("need_grad_teacher_weight") and wt is not None) else None
    g_nw = torch.empty_like(nw) if (need("need_grad_student_norm_weight") and nw is not None) else None
    return g_hs, g_w, g_ht, g_wt, g_nw


def fused_backward(ctx, grad_output: torch.Tensor, with_norm: bool = False):
    """Gradients ``(d_student_hidden, d_weight, d_teacher_hidden,
    d_teacher_weight)`` in the compute dtype, unpadded; None where not needed.
    ``with_norm``: also ``d_student_norm_weight`` (the fused RMSNorm's
    weight), as a fifth entry."""
    hs, w, ht, wt, lt, labels, tk_i, tk_lp, nw, saved = ctx.saved_tensors
    problem = ctx.orda_problem
    H, Ht = ctx.orda_shapes
    flags = problem.flags
    dev = hs.device
    inputs = (hs, w, ht, wt, lt, labels, tk_i, tk_lp, nw)
    if flags & _native.FLAG["grads_in_forward"]:
        grads, ctx.orda_grads = ctx.orda_grads, None
        if grads is None:  # a second backward through a retained graph
            grads = _alloc_grads(flags, hs, w, ht, wt, nw)
            outs = [torch.empty((), dtype=torch.float32, device=dev) for _ in range(4)]
            _run_forward(problem, inputs, torch.empty_like(saved), outs, grads)
        g_hs, g_w, g_ht, g_wt, g_nw = grads
    else:
        g_hs, g_w, g_ht, g_wt, g_nw = _alloc_grads(flags, hs, w, ht, wt, nw)
    go = grad_output.detach().to(device=dev, dtype=torch.float32).reshape(()).contiguous()
    ws_bytes = 0 if flags & _native.FLAG["grads_in_forward"] else _native.backward_workspace_bytes(problem)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
    t = _native.Tensors()
    t.student_hidden, t.weight, t.labels = _ptr(hs), _ptr(w), _ptr(labels)
    t.teacher_hidden, t.teacher_weight, t.teacher_logits = _ptr(ht), _ptr(wt), _ptr(lt)
    t.teacher_topk_indices, t.teacher_topk_logprobs = _ptr(tk_i), _ptr(tk_lp)
    t.student_norm_weight = _ptr(nw)
    t.saved = saved.data_ptr()
    t.grad_output = go.data_ptr()
    t.grad_student_hidden, t.grad_weight = _ptr(g_hs), _ptr(g_w)
    t.grad_teacher_hidden, t.grad_teacher_weight = _ptr(g_ht), _ptr(g_wt)
    t.grad_student_norm_weight = _ptr(g_nw)
    _native.backward(problem, t, ws, dev)
    del ws
    if g_hs is not None and g_hs.shape[1] != H:
        g_hs = g_hs[:, :H]
    if g_w is not None and g_w.shape[1] != H:
        g_w = g_w[:, :H]
    ht_cols = H if ctx.orda_mode == "tied" else Ht
    if g_ht is not None and g_ht.shape[1] != ht_cols:
        g_ht = g_ht[:, :ht_cols]
    if g_wt is not None and g_wt.shape[1] != Ht:
        g_wt = g_wt[:, :Ht]
    if g_nw is not None and g_nw.shape[0] != H:
        g_nw = g_nw[:H]
    if with_norm:
        return g_hs, g_w, g_ht, g_wt, g_nw
    return g_hs, g_w, g_ht, g_wt


def cast_to(grad: torch.Tensor | None, dtype: torch.dtype) -> torch.Tensor | None:
    """Gradient in the dtype of the original input (the reference casts
    grad_W to the weight dtype, ``ops/tied_teacher.py:545``)."""
    if grad is None:
        return None
    return grad if grad.dtype == dtype else grad.to(dtype)


def finite_or_raise(value: float, name: str) -> float:
    value = float(value)
    if math.isnan(value):
        raise ValueError(f"{name} must not be NaN")
    return value
