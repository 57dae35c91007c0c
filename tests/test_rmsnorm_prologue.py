"""CPU: the student's RMSNorm fused in front of the loss -- the oracle's chain
rule, the unfused torch formulation (``student_norm=`` on CPU tensors), the
argument checks and the C-ABI's validation of the prologue flags.

The reference's loss API has no norm (its producer applies
``x * rsqrt(mean(x^2) + eps) * w`` before the loss,
``test/benchmark/src/core.py:13-14``), so there are no golden vectors; the
oracle's prologue is pinned by:

* central differences of the oracle's own loss in ``x`` and ``w``;
* torch float64 autograd through the reference producer's formula composed
  with the (separately pinned) torch formulation of the loss;
* an identity: with ``w = 1``, ``eps = 0`` and rows of unit RMS, the normed
  loss is the plain loss.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle, topk_dense_logits
from orda_ce_kernel import _native

import orda_ce_kernel as o


def _problem(seed, n=7, h=6, v=19, ht_dim=5):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, h)) * 1.7
    g = 1.0 + 0.3 * rng.standard_normal(h)
    W = rng.standard_normal((v, h)) * 0.8
    ht = rng.standard_normal((n, h))
    hts = rng.standard_normal((n, ht_dim))
    Wt = rng.standard_normal((v, ht_dim))
    y = rng.integers(0, v, n)
    y[1] = -100
    return x, g, W, ht, hts, Wt, y


MODES = ["tied", "separate", "precomputed_logits", "precomputed_hidden"]


def _oracle_kw(mode, ht, hts, Wt):
    if mode == "tied":
        return "tied", dict(teacher_hidden=ht)
    if mode == "separate":
        return "separate", dict(teacher_hidden=hts, teacher_weight=Wt)
    if mode == "precomputed_logits":
        return "precomputed", dict(teacher_logits=hts @ Wt.T)
    return "precomputed", dict(teacher_hidden=hts, teacher_weight=Wt)


@pytest.mark.parametrize("div", ["forward_kl", "jsd"])
@pytest.mark.parametrize("mode", MODES)
def test_oracle_norm_gradients_are_the_loss_derivatives(mode, div):
    x, g, W, ht, hts, Wt, y = _problem(3)
    omode, kw = _oracle_kw(mode, ht, hts, Wt)
    args = dict(student_ce_weight=0.8, kl_weight=1.1, kl_temperature=1.5, divergence=div, norm_eps=1e-3, **kw)
    ref = distillation_loss_oracle(omode, x, W, y, student_norm_weight=g, **args)
    eps = 1e-6

    def loss(xx, gg):
        return distillation_loss_oracle(omode, xx, W, y, student_norm_weight=gg, **args)["loss"]

    fd_x = np.zeros_like(x)
    for i in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[i] += eps
        xm[i] -= eps
        fd_x[i] = (loss(xp, g) - loss(xm, g)) / (2 * eps)
    fd_g = np.zeros_like(g)
    for i in range(g.shape[0]):
        gp, gm = g.copy(), g.copy()
        gp[i] += eps
        gm[i] -= eps
        fd_g[i] = (loss(x, gp) - loss(x, gm)) / (2 * eps)
    np.testing.assert_allclose(ref["grad_student_hidden"], fd_x, rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(ref["grad_student_norm_weight"], fd_g, rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("reduction", ["mean", "sum"])
@pytest.mark.parametrize("mode", MODES + ["topk"])
def test_torch_formulation_matches_the_oracle(mode, reduction):
    x, g, W, ht, hts, Wt, y = _problem(5)
    xt, gt, Wt_ = (torch.tensor(a, requires_grad=True) for a in (x, g, W))
    if mode == "tied":
        teacher = o.TiedTeacher(torch.tensor(ht))
    elif mode == "separate":
        teacher = o.SeparateTeacher(torch.tensor(hts), torch.tensor(Wt))
    elif mode == "precomputed_logits":
        teacher = o.PrecomputedTeacher(logits=torch.tensor(hts @ Wt.T))
    elif mode == "precomputed_hidden":
        teacher = o.PrecomputedTeacher(teacher_hidden=torch.tensor(hts), teacher_weight=torch.tensor(Wt))
    else:
        lp = torch.log_softmax(torch.tensor(hts @ Wt.T), dim=1)
        vals, idx = lp.topk(4, dim=1)
        teacher = o.TopKTeacher(idx, vals)
    w_t = 0.0 if mode in ("precomputed_logits", "precomputed_hidden", "topk") else 0.6
    out = o.distillation_loss(xt, Wt_, torch.tensor(y), teacher, student_ce_weight=0.9, teacher_ce_weight=w_t,
                              kl_weight=0.7, kl_temperature=2.0, reduction=reduction,
                              student_norm=o.StudentRMSNorm(gt, eps=1e-5))
    out.loss.backward()
    if mode == "topk":
        omode, kw = "precomputed", dict(teacher_logits=topk_dense_logits(idx.numpy(), vals.numpy(), W.shape[0]))
    else:
        omode, kw = _oracle_kw(mode, ht, hts, Wt)
    ref = distillation_loss_oracle(omode, x, W, y, student_ce_weight=0.9, teacher_ce_weight=w_t, kl_weight=0.7,
                                   kl_temperature=2.0, reduction=reduction, student_norm_weight=g, norm_eps=1e-5,
                                   **kw)
    for key in ("loss", "student_ce", "teacher_ce", "kl"):
        assert float(getattr(out, key).detach()) == pytest.approx(ref[key], rel=1e-10, abs=1e-12), key
    np.testing.assert_allclose(xt.grad.numpy(), ref["grad_student_hidden"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(gt.grad.numpy(), ref["grad_student_norm_weight"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(Wt_.grad.numpy(), ref["grad_weight"], rtol=1e-9, atol=1e-12)


def test_unit_rms_rows_with_unit_weight_are_the_plain_loss():
    x, _, W, ht, _, _, y = _problem(7)
    x = x / np.sqrt((x * x).mean(axis=1, keepdims=True))
    kw = dict(teacher_hidden=ht, kl_weight=0.5, kl_temperature=1.3)
    a = distillation_loss_oracle("tied", x, W, y, student_norm_weight=np.ones(x.shape[1]), norm_eps=0.0, **kw)
    b = distillation_loss_oracle("tied", x, W, y, **kw)
    assert a["loss"] == pytest.approx(b["loss"], rel=1e-13)
    np.testing.assert_allclose(a["grad_weight"], b["grad_weight"], rtol=1e-11, atol=1e-14)
    # (dx differs from dy by the projection that keeps the RMS fixed)
    dy, xs = b["grad_student_hidden"], x
    proj = dy - xs * ((dy * xs).sum(axis=1) / xs.shape[1])[:, None]
    np.testing.assert_allclose(a["grad_student_hidden"], proj, rtol=1e-10, atol=1e-14)


@pytest.mark.parametrize(
    "norm, message",
    [
        (lambda h: o.StudentRMSNorm(torch.ones(h + 1)), "shape"),
        (lambda h: o.StudentRMSNorm(torch.ones(h), eps=-1.0), "eps"),
        (lambda h: o.StudentRMSNorm(torch.ones(h, dtype=torch.long)), "floating"),
        (lambda h: (torch.ones(h), 1e-6), "StudentRMSNorm"),
    ],
)
def test_norm_arguments_are_checked(norm, message):
    x, _, W, ht, _, _, y = _problem(9)
    exc = TypeError if message == "StudentRMSNorm" else ValueError
    with pytest.raises(exc, match=message):
        o.distillation_loss(torch.tensor(x), torch.tensor(W), torch.tensor(y), o.TiedTeacher(torch.tensor(ht)),
                            student_norm=norm(x.shape[1]))


def _abi_problem(**kw):
    p = _native.Problem()
    p.abi_version = _native.ABI_VERSION
    p.mode, p.dtype = 0, 0
    p.n_rows, p.vocab, p.hidden, p.teacher_hidden = 4096, 32000, 2048, 2048
    p.ignore_index = -100
    p.flags = 0x3 | 0x10 | 0x20 | 0x80 | 0x100 | 0x200
    p.temperature = 1.0
    p.student_ce_weight = p.teacher_ce_weight = p.kl_weight = 1.0
    p.norm_eps = 1e-6
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize(
    "kw, message",
    [
        (dict(flags=0x3 | 0x100), "ORDA_GRADS_IN_FORWARD"),
        (dict(flags=0x3 | 0x80 | 0x200), "needs ORDA_STUDENT_RMSNORM"),
        (dict(norm_dim=2049), "norm_dim"),
        (dict(norm_dim=-1), "norm_dim"),
        (dict(norm_eps=-1e-3), "norm_eps"),
        (dict(norm_eps=float("inf")), "norm_eps"),
    ],
)
def test_invalid_norm_problems_are_rejected(kw, message):
    with pytest.raises(ValueError, match=message):
        _native.forward_workspace_bytes(_abi_problem(**kw))


def test_norm_workspace_holds_the_normalised_chunk():
    """The prologue's workspace: the chunk's normalised rows and their
    rsqrt, and with the weight's gradient its token-group partials."""
    p = _abi_problem(token_chunk=512)
    with_norm = _native.forward_workspace_bytes(p)
    p.flags &= ~(0x100 | 0x200)
    plain = _native.forward_workspace_bytes(p)
    chunk = _native.plan_info(p)["token_chunk"]
    assert with_norm - plain >= chunk * 2048 * 2 + chunk * 4
