"""CPU: the distillation-gradient bounds of the GPU tests can fail.

For every divergence case and temperature of ``tests/test_gpu_divergence_grads.py``,
at its shapes and inputs, a mistake planted in the oracle's divergence
gradient (never in the product) must break the bound that the GPU result is
held to, for ``grad_student_hidden`` or ``grad_weight``:

* ``zero``: the divergence gradient dropped;
* ``sign``: its sign flipped;
* ``drop_T``: the ``T`` factor of ``kl_weight * T * dD/dz`` dropped (T != 1);
* ``at_T1``: the probabilities taken at T = 1 instead of T (T != 1);
* ``no_centre``: ``p_s * g`` instead of ``p_s * (g - <p_s, g>)``;
* ``forward_kl``: forward KL's gradient in place of the divergence's (not
  for soft-target CE, whose gradient in z_s *is* forward KL's).

And an emulation of the 16-bit path (logits rounded as stored, normaliser
from the unrounded logits with the largest element's rounding corrected,
dlogits and gradients rounded) stays inside the 16-bit bound, so the GPU
tests check something the kernels can meet.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.orda_oracle as O
from tests import _divgrad as D

SLIPS = ("zero", "sign", "drop_T", "at_T1", "no_centre", "forward_kl")


def _inputs(mode, dtype):
    hs, W, ht, hts, Wt, y = D.make_inputs(7, dtype)
    f = lambda t: t.double().numpy()  # noqa: E731
    if mode == "tied":
        kw = dict(teacher_hidden=f(ht))
    elif mode == "separate":
        kw = dict(teacher_hidden=f(hts), teacher_weight=f(Wt))
    else:
        kw = dict(teacher_logits=f((hts.float() @ Wt.float().t()).to(dtype)))
    return f(hs), f(W), y.numpy(), kw


def _oracle(mode, hs, W, y, kw, name, a, b, T, dtype):
    return O.distillation_loss_oracle(
        "precomputed" if mode == "precomputed" else mode, hs, W, y, student_ce_weight=0.0, teacher_ce_weight=0.0,
        kl_weight=1.0, kl_temperature=T, divergence=name, alpha=a, beta=b, teacher_grads=False,
        grad_logits_dtype=D.grad_logits_dtype(dtype), **kw)


def _planted(slip, T, orig):
    def value_and_grad(z_t, z_s, name, alpha=None, beta=None):
        v, g = orig(z_t, z_s, name, alpha, beta)
        if slip == "zero":
            return v, 0.0 * g
        if slip == "sign":
            return v, -g
        if slip == "drop_T":
            return v, g / T
        if slip == "at_T1":
            return orig(z_t * T, z_s * T, name, alpha, beta)
        if slip == "forward_kl":
            return orig(z_t, z_s, "forward_kl")
        fn, da, db = O.DIVERGENCE_DEFS[name]  # no_centre
        a = da if alpha is None else alpha
        b = db if beta is None else beta
        lt, ls = O.log_softmax(z_t), O.log_softmax(z_s)
        pt, ps = np.exp(lt), np.exp(ls)
        out = np.empty_like(z_s)
        for i in range(z_s.shape[0]):
            out[i] = ps[i] * fn(pt[i], ps[i], lt[i], ls[i], a, b)[1]
        return v, out
    return value_and_grad


def _applies(slip, name, T):
    if slip in ("drop_T", "at_T1") and T == 1.0:
        return False
    return not (slip == "forward_kl" and name in ("forward_kl", "soft_target_ce"))


@pytest.mark.parametrize("case", D.DIV_CASES, ids=D.DIV_IDS)
def test_bounds_reject_planted_slips(case, monkeypatch):
    _, name, a, b = case
    for dtype in (torch.bfloat16, torch.float32):
        for mode in ("tied", "separate"):
            hs, W, y, kw = _inputs(mode, dtype)
            for T in D.TEMPERATURES:
                ref = _oracle(mode, hs, W, y, kw, name, a, b, T, dtype)
                for slip in SLIPS:
                    if not _applies(slip, name, T):
                        continue
                    monkeypatch.setattr(O, "divergence_value_and_grad", _planted(slip, T, O.divergence_value_and_grad))
                    got = _oracle(mode, hs, W, y, kw, name, a, b, T, dtype)
                    monkeypatch.undo()
                    ok_h, msg_h = D.grad_ok(got["grad_student_hidden"], ref["grad_student_hidden"], dtype, name)
                    ok_w, msg_w = D.grad_ok(got["grad_weight"], ref["grad_weight"], dtype, name)
                    assert not (ok_h and ok_w), (name, a, b, str(dtype), mode, T, slip, msg_h, msg_w)


def _bf16(x):
    return O.round_to(x, "bfloat16")


def _emulated_16bit(mode, hs, W, y, kw, name, a, b, T):
    """The 16-bit gradients-in-forward path's roundings, in float64."""
    xs_e = hs @ W.T
    if mode == "tied":
        xt_e = kw["teacher_hidden"] @ W.T
    elif mode == "separate":
        xt_e = kw["teacher_hidden"] @ kw["teacher_weight"].T
    else:
        xt_e = kw["teacher_logits"]
    rows = np.arange(len(y))

    def log_p(x_r, x_e):
        z = x_e / T
        zmax = z.max(1)
        lse = np.log(np.exp(z - zmax[:, None]).sum(1)) + zmax
        i = x_e.argmax(1)
        d = (x_r[rows, i] - x_e[rows, i]) / T
        return x_r / T - (lse + d * np.exp(zmax - lse))[:, None]

    xs_r, xt_r = _bf16(xs_e), _bf16(xt_e)
    ls, lt = log_p(xs_r, xs_e), log_p(xt_r, xt_e)
    ps, pt = np.exp(ls), np.exp(lt)
    fn, da, db = O.DIVERGENCE_DEFS[name]
    aa = da if a is None else a
    bb = db if b is None else b
    dz = np.empty_like(xs_e)
    for i in rows:
        g = fn(pt[i], ps[i], lt[i], ls[i], aa, bb)[1]
        dz[i] = ps[i] * (g - (ps[i] * g).sum())
    keep = (y != -100)[:, None]
    dl = _bf16(keep * T * dz / keep.sum())
    return _bf16(dl @ W), _bf16(dl.T @ hs)


@pytest.mark.parametrize("case", D.DIV_CASES, ids=D.DIV_IDS)
def test_16bit_emulation_meets_the_bounds(case):
    _, name, a, b = case
    for mode in ("tied", "separate", "precomputed"):
        hs, W, y, kw = _inputs(mode, torch.bfloat16)
        for T in D.TEMPERATURES:
            ref = _oracle(mode, hs, W, y, kw, name, a, b, T, torch.bfloat16)
            gh, gw = _emulated_16bit(mode, hs, W, y, kw, name, a, b, T)
            for got, key in ((gh, "grad_student_hidden"), (gw, "grad_weight")):
                ok, msg = D.grad_ok(got, ref[key], torch.bfloat16, name)
                assert ok, (name, a, b, mode, T, key, msg)
