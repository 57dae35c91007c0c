"""The package's unfused torch backend (backend="torch", CPU) against the
float64 oracle: the reference's test/correctness/test_torch_backend_cpu.py
cases (tolerance atol 1e-6 / rtol 1e-5) plus every divergence."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle
from orda_ce_kernel import PrecomputedTeacher, SeparateTeacher, TiedTeacher, distillation_loss

ATOL, RTOL = 1e-6, 1e-5


def _t(seed, *shape, scale=0.1):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def _labels(seed, BT, V):
    g = torch.Generator().manual_seed(seed)
    y = torch.randint(0, V, (BT,), generator=g)
    y[:: max(1, BT // 4)] = -100
    return y


def _np(x):
    return x.detach().double().numpy()


def _check(out, ref, grads):
    for name in ("loss", "student_ce", "teacher_ce", "kl"):
        assert np.isclose(float(getattr(out, name)), ref[name], atol=ATOL, rtol=RTOL), name
    for tensor, key in grads:
        np.testing.assert_allclose(_np(tensor.grad), ref[key], atol=ATOL, rtol=RTOL, err_msg=key)


@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_tied(reduction):
    hs = _t(1, 9, 7).requires_grad_(True)
    ht = _t(2, 9, 7).requires_grad_(True)
    w = _t(3, 17, 7).requires_grad_(True)
    y = _labels(101, 9, 17)
    out = distillation_loss(hs, w, y, TiedTeacher(ht), student_ce_weight=0.8, teacher_ce_weight=0.25, kl_weight=0.35,
                            kl_temperature=1.4, reduction=reduction, backend="torch")
    out.loss.backward()
    ref = distillation_loss_oracle("tied", _np(hs), _np(w), y.numpy(), teacher_hidden=_np(ht), student_ce_weight=0.8,
                                   teacher_ce_weight=0.25, kl_weight=0.35, kl_temperature=1.4, reduction=reduction,
                                   kernel_semantics=False)
    _check(out, ref, [(hs, "grad_student_hidden"), (ht, "grad_teacher_hidden"), (w, "grad_weight")])


@pytest.mark.parametrize("full", [False, True])
def test_separate(full):
    hs = _t(4, 10, 6).requires_grad_(True)
    ht = _t(5, 10, 8).requires_grad_(True)
    w = _t(6, 19, 6).requires_grad_(True)
    wt = _t(7, 19, 8).requires_grad_(True)
    y = _labels(102, 10, 19)
    out = distillation_loss(hs, w, y, SeparateTeacher(ht, wt), teacher_ce_weight=1.0 if full else None,
                            kl_weight=0.4, kl_temperature=1.6, backend="torch")
    out.loss.backward()
    ref = distillation_loss_oracle("separate", _np(hs), _np(w), y.numpy(), teacher_hidden=_np(ht),
                                   teacher_weight=_np(wt), teacher_ce_weight=1.0 if full else None, kl_weight=0.4,
                                   kl_temperature=1.6, kernel_semantics=False, teacher_grads=full)
    grads = [(hs, "grad_student_hidden"), (w, "grad_weight")]
    if full:
        grads += [(ht, "grad_teacher_hidden"), (wt, "grad_teacher_weight")]
    else:
        assert float(out.teacher_ce) == 0.0
        assert ht.grad is None and wt.grad is None
    _check(out, ref, grads)


def test_precomputed_logits_and_hidden():
    hs = _t(8, 11, 7).requires_grad_(True)
    w = _t(9, 23, 7).requires_grad_(True)
    th, tw = _t(10, 11, 9), _t(11, 23, 9)
    y = _labels(104, 11, 23)
    for teacher in (PrecomputedTeacher(logits=th @ tw.t()), PrecomputedTeacher(teacher_hidden=th, teacher_weight=tw)):
        hs.grad = None
        w.grad = None
        out = distillation_loss(hs, w, y, teacher, kl_weight=0.3, kl_temperature=1.5, backend="torch")
        out.loss.backward()
        ref = distillation_loss_oracle("precomputed", _np(hs), _np(w), y.numpy(), teacher_logits=_np(th @ tw.t()),
                                       kl_weight=0.3, kl_temperature=1.5, kernel_semantics=False)
        assert float(out.teacher_ce) == 0.0
        _check(out, ref, [(hs, "grad_student_hidden"), (w, "grad_weight")])


def test_all_ignored_gives_exact_zeros():
    hs = _t(12, 8, 6).requires_grad_(True)
    ht = _t(13, 8, 6).requires_grad_(True)
    w = _t(14, 13, 6).requires_grad_(True)
    y = torch.full((8,), -100, dtype=torch.long)
    out = distillation_loss(hs, w, y, TiedTeacher(ht), kl_weight=0.5, kl_temperature=1.7, backend="torch")
    out.loss.backward()
    for t in out:
        assert torch.equal(t, torch.zeros_like(t))
    for t in (hs.grad, ht.grad, w.grad):
        assert torch.all(t == 0)


DIVS = ["forward_kl", "reverse_kl", "symmetric_kl", "soft_target_ce", "hellinger", "bhattacharyya", "renyi",
        "amari_alpha", "chi_squared", "squared_l2", "ab", "jsd", "skew_forward_kl", "skew_reverse_kl", "tvd"]


@pytest.mark.parametrize("div", DIVS)
def test_every_divergence(div):
    hs = _t(20, 12, 8, scale=0.5).requires_grad_(True)
    ht = _t(21, 12, 8, scale=0.5).requires_grad_(True)
    w = _t(22, 31, 8, scale=0.5).requires_grad_(True)
    y = _labels(23, 12, 31)
    out = distillation_loss(hs, w, y, TiedTeacher(ht), kl_weight=0.6, kl_temperature=2.0, backend="torch",
                            divergence=div)
    out.loss.backward()
    ref = distillation_loss_oracle("tied", _np(hs), _np(w), y.numpy(), teacher_hidden=_np(ht), kl_weight=0.6,
                                   kl_temperature=2.0, divergence=div, kernel_semantics=False)
    _check(out, ref, [(hs, "grad_student_hidden"), (ht, "grad_teacher_hidden"), (w, "grad_weight")])
