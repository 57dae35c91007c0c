"""Plain PyTorch float32 reference of the fused loss, chunked over tokens so
it runs at the full benchmark shapes on a GPU -- TEST INFRASTRUCTURE ONLY.

It restates the reference's unfused torch path (``api.py:274-335`` of
``src/orda_ce_kernel``: logits, ``logsumexp`` cross-entropies, the
distillation term times ``T^2`` masked on ignored rows, masked mean with
``clamp(count, 1)``) with autograd over each chunk's logits for the dlogits,
then the gradient GEMMs in float32.  The distillation term never sends a
gradient to the teacher (``ops/tied_teacher.py:153-186``).  Every divergence
of the package is written here from its published definition (the reference
has forward KL only); a label outside ``[0, V)`` counts as class 0, as in the
Triton kernels (``ops/tied_teacher.py:42-44``).

``tests/test_fp32_reference.py`` pins this restatement against the float64
oracle on small shapes (CPU), so the full-size GPU tests compare the HIP path
with a checked reference.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

# every divergence of the package, with the registry's default parameters
# (renyi / amari alpha 0.5, ab alpha = beta = 0.5, jsd beta 0.5, skew alpha
# 0.1), written from the published definitions
DEFAULT_PARAMS = {"renyi": (0.5, None), "amari_alpha": (0.5, None), "ab": (0.5, 0.5), "jsd": (None, 0.5),
                  "skew_forward_kl": (0.1, None), "skew_reverse_kl": (0.1, None)}
DIVERGENCES = ("forward_kl", "reverse_kl", "symmetric_kl", "soft_target_ce", "hellinger", "bhattacharyya", "renyi",
               "amari_alpha", "chi_squared", "squared_l2", "ab", "jsd", "skew_forward_kl", "skew_reverse_kl", "tvd")


def _divergence_rows(ls: torch.Tensor, lt: torch.Tensor, name: str, alpha: float | None = None,
                     beta: float | None = None) -> torch.Tensor:
    """Per-row D(p_t || p_s) from log-probabilities (teacher ``lt`` detached);
    ``alpha`` / ``beta`` default to the registry's (``DEFAULT_PARAMS``)."""
    da, db = DEFAULT_PARAMS.get(name, (None, None))
    a = da if alpha is None else float(alpha)
    b = db if beta is None else float(beta)
    pt, ps = lt.exp(), ls.exp()
    if name == "forward_kl":
        return (pt * (lt - ls)).sum(1)
    if name == "reverse_kl":
        return (ps * (ls - lt)).sum(1)
    if name == "symmetric_kl":
        return (pt * (lt - ls)).sum(1) + (ps * (ls - lt)).sum(1)
    if name == "soft_target_ce":
        return -(pt * ls).sum(1)
    if name == "hellinger":
        return 1.0 - (0.5 * (lt + ls)).exp().sum(1)
    if name == "bhattacharyya":
        return -torch.logsumexp(0.5 * (lt + ls), 1)
    if name == "renyi":
        return torch.logsumexp(a * lt + (1.0 - a) * ls, 1) / (a - 1.0)
    if name == "amari_alpha":
        return (1.0 - (a * lt + (1.0 - a) * ls).exp().sum(1)) / (a * (1.0 - a))
    if name == "chi_squared":
        return ((pt - ps) ** 2 * (-ls).exp()).sum(1)
    if name == "squared_l2":
        return ((pt - ps) ** 2).sum(1)
    if name == "ab":
        q1 = (a * lt + b * ls).exp()
        q2 = ((a + b) * lt).exp()
        q3 = ((a + b) * ls).exp()
        return -(q1 - a / (a + b) * q2 - b / (a + b) * q3).sum(1) / (a * b)
    if name == "jsd":
        lm = torch.logaddexp(math.log(b) + lt, math.log(1.0 - b) + ls)
        return b * (pt * (lt - lm)).sum(1) + (1.0 - b) * (ps * (ls - lm)).sum(1)
    if name == "skew_forward_kl":
        lm = torch.logaddexp(math.log(a) + lt, math.log(1.0 - a) + ls)
        return (pt * (lt - lm)).sum(1)
    if name == "skew_reverse_kl":
        lm = torch.logaddexp(math.log(a) + ls, math.log(1.0 - a) + lt)
        return (ps * (ls - lm)).sum(1)
    if name == "tvd":
        return 0.5 * (pt - ps).abs().sum(1)
    raise ValueError(f"divergence {name!r} is not in the float32 reference")


@torch.no_grad()
def _teacher_logits(mode, s, e, ht, Wt_f, lt):
    if mode == "precomputed":
        return lt[s:e].float()
    return ht[s:e].float() @ Wt_f.t()


def fp32_reference(mode, hs, W, y, *, ht=None, Wt=None, lt=None, student_ce_weight=1.0, teacher_ce_weight=None,
                   kl_weight=0.0, kl_temperature=1.0, divergence="forward_kl", ignore_index=-100, chunk=1024):
    """Loss components (python floats) and float32 gradients.

    ``mode``: ``tied`` (teacher logits ``ht W^T``), ``separate``
    (``ht Wt^T``) or ``precomputed`` (``lt``).  Returns a dict with
    ``loss``, ``student_ce``, ``teacher_ce``, ``kl``, ``count``,
    ``grad_student_hidden`` [N x H] and ``grad_weight`` [V x H] (float32,
    on the inputs' device) and ``teacher_entropy`` (min, max) in nats.
    """
    N, V, H = hs.shape[0], W.shape[0], W.shape[1]
    w_s = float(student_ce_weight)
    w_t = (1.0 if mode == "tied" else 0.0) if teacher_ce_weight is None else float(teacher_ce_weight)
    kl_w = float(kl_weight)
    T = float(kl_temperature)
    dev = hs.device
    W_f = W.float()
    Wt_f = W_f if mode == "tied" else (Wt.float() if Wt is not None else None)
    keep_all = y != ignore_index
    count = int(keep_all.sum())
    scale = 1.0 / max(count, 1)
    y_eff = torch.where((y >= 0) & (y < V), y, torch.zeros_like(y))
    sums = torch.zeros(3, dtype=torch.float64, device=dev)
    grad_h = torch.empty(N, H, dtype=torch.float32, device=dev)
    grad_W = torch.zeros(V, H, dtype=torch.float32, device=dev)
    ent_min, ent_max = math.inf, -math.inf
    for s in range(0, N, chunk):
        e = min(N, s + chunk)
        keep = keep_all[s:e].float()
        yc = y_eff[s:e, None]
        with torch.no_grad():
            xs0 = hs[s:e].float() @ W_f.t()
            xt0 = _teacher_logits(mode, s, e, ht, Wt_f, lt)
        x_s = xs0.requires_grad_(True)
        x_t = xt0.requires_grad_(True)
        with torch.enable_grad():
            ce_s = (torch.logsumexp(x_s, 1) - x_s.gather(1, yc)[:, 0]) * keep
            ce_t = (torch.logsumexp(x_t, 1) - x_t.gather(1, yc)[:, 0]) * keep
            ls = F.log_softmax(x_s / T, 1)
            lt_T = F.log_softmax(x_t.detach() / T, 1)
            d = _divergence_rows(ls, lt_T, divergence) * keep * (T * T)
            if kl_w == 0.0:
                d = d * 0.0
            total = w_s * ce_s.sum() + w_t * ce_t.sum() + kl_w * d.sum()
            total.backward()
        with torch.no_grad():
            lp = F.log_softmax(xt0, 1)
            ent = -(lp.exp() * lp).sum(1)
            ent_min = min(ent_min, float(ent.min()))
            ent_max = max(ent_max, float(ent.max()))
            sums += torch.stack([ce_s.sum(), ce_t.sum(), d.sum()]).double()
            ds = x_s.grad * scale
            grad_h[s:e] = ds @ W_f
            grad_W.addmm_(ds.t(), hs[s:e].float())
            if mode == "tied" and w_t != 0.0:
                grad_W.addmm_((x_t.grad * scale).t(), ht[s:e].float())
        del x_s, x_t, xs0, xt0, ce_s, ce_t, ls, lt_T, d, total
    ce_s_v, ce_t_v, kl_v = (float(v) * scale for v in sums.cpu())
    if w_t == 0.0:
        ce_t_v = 0.0
    return {
        "loss": w_s * ce_s_v + w_t * ce_t_v + kl_w * kl_v, "student_ce": ce_s_v, "teacher_ce": ce_t_v,
        "kl": kl_v, "count": count, "grad_student_hidden": grad_h, "grad_weight": grad_W,
        "teacher_entropy": (ent_min, ent_max),
    }
