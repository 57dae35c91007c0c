"""CPU: the top-k teacher -- the oracle's reading of it, the unfused torch
formulation, and the API's argument checks.

A top-k teacher has no counterpart in the reference, so there are no golden
vectors for it; the oracle (``topk_dense_logits`` fed to the precomputed-
logits path, itself pinned by the reference's vectors) is pinned here by what
the mathematics fixes:

* k = V: the teacher's full log-probabilities as (id, log-prob) pairs in any
  order are the precomputed teacher with those logits;
* the distribution stands for the teacher renormalised over its ids at T
  (``scipy.special.softmax`` of ``logprobs / T`` on the ids, 0 elsewhere);
* forward KL minus soft-target CE is minus the teacher's entropy
  (``scipy.stats.entropy``), whatever the student;
* the oracle's gradients are the loss's derivatives (central differences of
  the oracle's own loss).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
from scipy.special import log_softmax as sp_log_softmax
from scipy.special import softmax as sp_softmax
from scipy.stats import entropy

from oracle.orda_oracle import distillation_loss_oracle, topk_dense_logits

import orda_ce_kernel as o


def _problem(seed, n=9, h=6, v=23, k=5):
    rng = np.random.default_rng(seed)
    hs = rng.standard_normal((n, h))
    W = rng.standard_normal((v, h)) * 0.7
    y = rng.integers(0, v, n)
    y[2] = -100
    lt = rng.standard_normal((n, v)) * 2.0
    lp = sp_log_softmax(lt, axis=1)
    idx = np.argsort(-lp, axis=1)[:, :k]
    return hs, W, y, lt, lp, idx, np.take_along_axis(lp, idx, 1)


def _oracle(hs, W, y, idx, vals, **kw):
    return distillation_loss_oracle("precomputed", hs, W, y, teacher_logits=topk_dense_logits(idx, vals, W.shape[0]),
                                    teacher_ce_weight=0.0, **kw)


@pytest.mark.parametrize("T", [1.0, 2.5])
@pytest.mark.parametrize("div", ["forward_kl", "soft_target_ce"])
def test_k_equal_to_vocab_is_the_precomputed_teacher(T, div):
    hs, W, y, lt, lp, _, _ = _problem(1)
    rng = np.random.default_rng(2)
    idx = np.stack([rng.permutation(W.shape[0]) for _ in range(hs.shape[0])])
    vals = np.take_along_axis(lp, idx, 1)
    assert np.array_equal(topk_dense_logits(idx, vals, W.shape[0]), lp)
    kw = dict(kl_weight=0.8, kl_temperature=T, divergence=div)
    a = _oracle(hs, W, y, idx, vals, **kw)
    b = distillation_loss_oracle("precomputed", hs, W, y, teacher_logits=lt, teacher_ce_weight=0.0, **kw)
    for key in ("loss", "student_ce", "kl"):
        assert a[key] == pytest.approx(b[key], rel=1e-12, abs=1e-12), key
    for key in ("grad_student_hidden", "grad_weight"):
        np.testing.assert_allclose(a[key], b[key], rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("T", [1.0, 0.5, 3.0])
def test_dense_logits_stand_for_the_renormalised_teacher(T):
    _, W, _, _, lp, idx, vals = _problem(3)
    dense = topk_dense_logits(idx, vals, W.shape[0])
    with np.errstate(invalid="ignore"):
        p = sp_softmax(dense / T, axis=1)
    expect = np.zeros_like(p)
    np.put_along_axis(expect, idx, sp_softmax(vals / T, axis=1), axis=1)
    np.testing.assert_allclose(p, expect, rtol=1e-13, atol=0)
    assert np.all(np.isneginf(np.delete(dense[0], idx[0])))


@pytest.mark.parametrize("k", [1, 4, 23])
@pytest.mark.parametrize("T", [1.0, 2.0])
def test_forward_kl_minus_soft_ce_is_minus_the_teacher_entropy(k, T):
    hs, W, y, _, _, idx, vals = _problem(5, k=k)
    fkl = _oracle(hs, W, y, idx, vals, kl_weight=1.0, kl_temperature=T, divergence="forward_kl", reduction="sum")
    soft = _oracle(hs, W, y, idx, vals, kl_weight=1.0, kl_temperature=T, divergence="soft_target_ce",
                   reduction="sum")
    keep = y != -100
    h = entropy(sp_softmax(vals / T, axis=1), axis=1)
    assert fkl["kl"] - soft["kl"] == pytest.approx(-T * T * h[keep].sum(), rel=1e-10, abs=1e-12)
    # and their student gradients are the same (they differ by a constant)
    np.testing.assert_allclose(fkl["grad_student_hidden"], soft["grad_student_hidden"], rtol=1e-10, atol=1e-13)


@pytest.mark.parametrize("div", ["forward_kl", "soft_target_ce"])
def test_oracle_gradients_are_the_loss_derivatives(div):
    hs, W, y, _, _, idx, vals = _problem(7, n=4, h=3, v=9, k=3)
    kw = dict(student_ce_weight=0.6, kl_weight=1.3, kl_temperature=1.7, divergence=div)
    ref = _oracle(hs, W, y, idx, vals, **kw)
    eps = 1e-6
    for name, x in (("grad_student_hidden", hs), ("grad_weight", W)):
        fd = np.zeros_like(x)
        for i in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[i] += eps
            xm[i] -= eps
            args = (xp, W) if name == "grad_student_hidden" else (hs, xp)
            argm = (xm, W) if name == "grad_student_hidden" else (hs, xm)
            fd[i] = (_oracle(*args, y, idx, vals, **kw)["loss"] - _oracle(*argm, y, idx, vals, **kw)["loss"]) / (2 * eps)
        np.testing.assert_allclose(ref[name], fd, rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("reduction", ["mean", "sum"])
@pytest.mark.parametrize("T", [1.0, 2.0])
@pytest.mark.parametrize("div", ["forward_kl", "soft_target_ce"])
def test_torch_formulation_matches_the_oracle(div, T, reduction):
    hs, W, y, _, _, idx, vals = _problem(11, n=12, h=8, v=40, k=7)
    hs_t = torch.tensor(hs, requires_grad=True)
    W_t = torch.tensor(W, requires_grad=True)
    teacher = o.TopKTeacher(torch.tensor(idx), torch.tensor(vals))
    out = o.distillation_loss(hs_t, W_t, torch.tensor(y), teacher, student_ce_weight=0.7, kl_weight=0.9,
                              kl_temperature=T, reduction=reduction, divergence=div)
    out.loss.backward()
    ref = _oracle(hs, W, y, idx, vals, student_ce_weight=0.7, kl_weight=0.9, kl_temperature=T,
                  reduction=reduction, divergence=div)
    for key in ("loss", "student_ce", "kl"):
        assert float(getattr(out, key).detach()) == pytest.approx(ref[key], rel=1e-10), key
    assert float(out.teacher_ce) == 0.0
    np.testing.assert_allclose(hs_t.grad.numpy(), ref["grad_student_hidden"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(W_t.grad.numpy(), ref["grad_weight"], rtol=1e-9, atol=1e-12)


def test_a_teacher_probability_that_underflows_contributes_nothing():
    """An id whose renormalised probability is 0 in float64 adds 0 (not NaN)."""
    hs, W, y, _, _, idx, vals = _problem(13, k=4)
    vals = vals.copy()
    vals[:, -1] = -1e4
    teacher = o.TopKTeacher(torch.tensor(idx), torch.tensor(vals))
    out = o.distillation_loss(torch.tensor(hs), torch.tensor(W), torch.tensor(y), teacher, kl_weight=1.0)
    ref = _oracle(hs, W, y, idx, vals, kl_weight=1.0)
    assert np.isfinite(float(out.kl)) and float(out.kl) == pytest.approx(ref["kl"], rel=1e-10)


def _cpu_args(k=5, v=23):
    hs, W, y, _, _, idx, vals = _problem(17, v=v, k=k)
    return torch.tensor(hs), torch.tensor(W), torch.tensor(y), torch.tensor(idx), torch.tensor(vals)


@pytest.mark.parametrize(
    "change, kw, message",
    [
        ("k0", {}, "1 <= k <= vocab"),
        ("shape", {}, "must have the shape of indices"),
        ("rows", {}, r"shape \(BT, k\)"),
        ("float_ids", {}, "integer dtype"),
        (None, dict(divergence="reverse_kl"), "supports the divergences"),
        (None, dict(teacher_ce_weight=1.0), "no teacher CE"),
        ("grad", {}, "must not require gradients"),
        ("dup", dict(profile="debug"), "distinct"),
        ("range", dict(profile="debug"), r"in \[0, 23\)"),
    ],
)
def test_topk_arguments_are_checked(change, kw, message):
    hs, W, y, idx, vals = _cpu_args()
    if change == "k0":
        idx, vals = idx[:, :0], vals[:, :0]
    elif change == "shape":
        vals = vals[:, :3]
    elif change == "rows":
        idx, vals = idx[:3], vals[:3]
    elif change == "float_ids":
        idx = idx.double()
    elif change == "grad":
        vals = vals.clone().requires_grad_(True)
    elif change == "dup":
        idx = idx.clone()
        idx[4, 1] = idx[4, 0]
    elif change == "range":
        idx = idx.clone()
        idx[0, 0] = 23
    with pytest.raises(ValueError, match=message):
        o.distillation_loss(hs, W, y, o.TopKTeacher(idx, vals), kl_weight=1.0, **kw)


def test_topk_module_wrapper_and_kl_off():
    """``DistillationLoss`` takes a TopKTeacher; with kl_weight = 0 the loss
    is the student CE alone."""
    hs, W, y, idx, vals = _cpu_args()
    mod = o.DistillationLoss(kl_weight=0.0)
    out = mod(hs, W, y, o.TopKTeacher(idx, vals))
    ce = torch.nn.functional.cross_entropy(hs @ W.t(), y, ignore_index=-100)
    assert float(out.loss.detach()) == pytest.approx(float(ce), rel=1e-12)


def test_ignored_rows_with_no_teacher_mass_stay_finite_on_the_torch_path():
    """Padding tokens whose top-k log-probabilities are all -inf (label
    -100): the torch formulation gives the oracle's result for the same
    rows with any finite teacher (ignored rows add nothing), with finite
    gradients; the HIP kernels' counterpart is in tests/test_gpu_topk.py."""
    hs, W, y, _, _, idx, vals = _problem(17, n=12, h=8, v=40, k=7)
    ign = np.flatnonzero(y == -100)
    assert ign.size > 0
    pad = vals.copy()
    pad[ign] = -np.inf
    hs_t = torch.tensor(hs, requires_grad=True)
    W_t = torch.tensor(W, requires_grad=True)
    out = o.distillation_loss(hs_t, W_t, torch.tensor(y), o.TopKTeacher(torch.tensor(idx), torch.tensor(pad)),
                              kl_weight=0.9, kl_temperature=2.0)
    out.loss.backward()
    ref = _oracle(hs, W, y, idx, vals, kl_weight=0.9, kl_temperature=2.0)
    assert float(out.loss.detach()) == pytest.approx(ref["loss"], rel=1e-10)
    assert np.isfinite(hs_t.grad.numpy()).all() and np.isfinite(W_t.grad.numpy()).all()
    np.testing.assert_allclose(hs_t.grad.numpy(), ref["grad_student_hidden"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(W_t.grad.numpy(), ref["grad_weight"], rtol=1e-9, atol=1e-12)
