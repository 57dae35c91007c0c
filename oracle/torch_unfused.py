"""Unfused PyTorch restatement of the reference loss -- TEST INFRASTRUCTURE
and the timed CPU baseline of ``bench.py``; never imported by the product.

Follows the reference's torch path ``_torch_reference`` (``api.py:274-335``):
full ``[N x V]`` logits, ``F.cross_entropy(reduction="none")`` for student
and teacher, ``log_softmax(x / T)`` twice, ``T^2 sum p_t (log p_t - log
p_s)`` masked on ignored rows, mean over non-ignored rows, weighted sum, and
autograd for the backward.  Forward KL only (the reference's divergence).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["tied_forward_kl_loss"]


def tied_forward_kl_loss(hs, ht, W, labels, *, student_ce_weight=1.0, teacher_ce_weight=1.0, kl_weight=1.0,
                         kl_temperature=1.0, ignore_index=-100):
    """Tied teacher, mean reduction; returns (loss, student_ce, teacher_ce, kl)."""
    logits_s = hs @ W.t()
    logits_t = ht @ W.t()
    ce_s = F.cross_entropy(logits_s, labels, ignore_index=ignore_index, reduction="none")
    ce_t = F.cross_entropy(logits_t, labels, ignore_index=ignore_index, reduction="none")
    keep = labels != ignore_index
    denom = keep.sum().clamp(min=1)
    T = float(kl_temperature)
    log_p_s = F.log_softmax(logits_s / T, dim=-1)
    log_p_t = F.log_softmax(logits_t.detach() / T, dim=-1)
    kl_rows = (log_p_t.exp() * (log_p_t - log_p_s)).sum(-1) * (T * T)
    kl_rows = kl_rows.masked_fill(~keep, 0.0)
    student_ce, teacher_ce, kl = ce_s.sum() / denom, ce_t.sum() / denom, kl_rows.sum() / denom
    loss = student_ce_weight * student_ce + teacher_ce_weight * teacher_ce + kl_weight * kl
    return loss, student_ce.detach(), teacher_ce.detach(), kl.detach()
