"""Pins of the CPU oracle (oracle/orda_oracle.py) -- CPU only.

Each check reaches the oracle's numbers by an independent route, chosen so
that a plausible mistake (a dropped term, a wrong sign or index, a swapped
operand) fails:

* torch float64 autograd through F.cross_entropy / F.log_softmax / F.kl_div,
  the formulation of the reference's own test oracle
  (test/utils/reference.py:60-93), on the reference's CPU test cases
  (test/correctness/test_torch_backend_cpu.py, seeds 101-106);
* scipy.stats.entropy and scipy.spatial.distance.jensenshannon for the
  divergence values;
* closed-form identities between divergences;
* central finite differences of the oracle's own loss for every gradient;
* invariants: all-ignored rows give exact zeros, D(p || p) = 0, a per-row
  logit shift changes nothing, sum = mean * count.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy.spatial.distance import jensenshannon
from scipy.stats import entropy

from oracle.orda_oracle import DIVERGENCE_DEFS, distillation_loss_oracle, divergence_value_and_grad, round_to

DIVS = sorted(DIVERGENCE_DEFS)


def _rng(seed):
    return np.random.default_rng(seed)


def _inputs(seed, N=9, H=7, V=17, Ht=None, ignore_every=4):
    r = _rng(seed)
    hs = r.standard_normal((N, H)) * 0.5
    ht = r.standard_normal((N, Ht or H)) * 0.5
    W = r.standard_normal((V, H)) * 0.5
    Wt = r.standard_normal((V, Ht or H)) * 0.5
    y = r.integers(0, V, N)
    if ignore_every:
        y[::ignore_every] = -100
    return hs, ht, W, Wt, y


def _torch_ref(mode, hs, W, y, *, ht=None, Wt=None, lt=None, w_s, w_t, kl_w, T, reduction):
    """float64 autograd of the reference test oracle's formulation."""
    hs_t = torch.tensor(hs, requires_grad=True)
    W_t = torch.tensor(W, requires_grad=True)
    y_t = torch.tensor(y)
    logits_s = hs_t @ W_t.t()
    extra = {}
    if mode == "tied":
        ht_t = torch.tensor(ht, requires_grad=True)
        logits_t = ht_t @ W_t.t()
        extra["ht"] = ht_t
    elif mode == "separate":
        ht_t = torch.tensor(ht, requires_grad=True)
        wt_t = torch.tensor(Wt, requires_grad=True)
        logits_t = ht_t @ wt_t.t()
        extra["ht"], extra["wt"] = ht_t, wt_t
    else:
        logits_t = torch.tensor(lt)
    ce_s = F.cross_entropy(logits_s, y_t, ignore_index=-100, reduction="none")
    ce_t = F.cross_entropy(logits_t, y_t, ignore_index=-100, reduction="none")
    mask = y_t != -100
    denom = max(int(mask.sum()), 1)
    kl = F.kl_div(F.log_softmax(logits_s / T, -1), F.softmax(logits_t.detach() / T, -1), reduction="none").sum(-1)
    kl = (kl * T * T).masked_fill(~mask, 0.0)
    if reduction == "mean":
        s, t, k = ce_s.sum() / denom, ce_t.sum() / denom, kl.sum() / denom
    else:
        s, t, k = ce_s.sum(), ce_t.sum(), kl.sum()
    t = t if w_t != 0.0 else t.new_zeros(())
    loss = w_s * s + w_t * t + kl_w * k
    loss.backward()
    out = {"loss": loss.item(), "student_ce": s.item(), "teacher_ce": t.item(), "kl": k.item(),
           "grad_student_hidden": hs_t.grad.numpy(), "grad_weight": W_t.grad.numpy()}
    if "ht" in extra and extra["ht"].grad is not None:
        out["grad_teacher_hidden"] = extra["ht"].grad.numpy()
    if "wt" in extra and extra["wt"].grad is not None:
        out["grad_teacher_weight"] = extra["wt"].grad.numpy()
    return out


def _assert_match(a, b, keys, tol=1e-9):
    for k in keys:
        np.testing.assert_allclose(a[k], b[k], rtol=tol, atol=tol, err_msg=k)


@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_tied_matches_torch_float64_reference(reduction):
    hs, ht, W, _, y = _inputs(101)
    kw = dict(w_s=0.8, w_t=0.25, kl_w=0.35, T=1.4, reduction=reduction)
    ref = _torch_ref("tied", hs, W, y, ht=ht, **kw)
    got = distillation_loss_oracle("tied", hs, W, y, teacher_hidden=ht, student_ce_weight=0.8, teacher_ce_weight=0.25,
                                   kl_weight=0.35, kl_temperature=1.4, reduction=reduction)
    _assert_match(got, ref, ["loss", "student_ce", "teacher_ce", "kl", "grad_student_hidden", "grad_weight",
                             "grad_teacher_hidden"])


def test_separate_full_matches_torch_float64_reference():
    hs, ht, W, Wt, y = _inputs(103, N=10, H=6, V=19, Ht=8)
    ref = _torch_ref("separate", hs, W, y, ht=ht, Wt=Wt, w_s=1.0, w_t=1.0, kl_w=0.4, T=1.6, reduction="mean")
    got = distillation_loss_oracle("separate", hs, W, y, teacher_hidden=ht, teacher_weight=Wt, teacher_ce_weight=1.0,
                                   kl_weight=0.4, kl_temperature=1.6)
    _assert_match(got, ref, ["loss", "student_ce", "teacher_ce", "kl", "grad_student_hidden", "grad_weight",
                             "grad_teacher_hidden", "grad_teacher_weight"])


def test_separate_student_only_matches_torch_float64_reference():
    hs, ht, W, Wt, y = _inputs(102, N=10, H=6, V=19, Ht=8)
    ref = _torch_ref("separate", hs, W, y, ht=ht, Wt=Wt, w_s=1.0, w_t=0.0, kl_w=0.4, T=1.6, reduction="mean")
    got = distillation_loss_oracle("separate", hs, W, y, teacher_hidden=ht, teacher_weight=Wt, kl_weight=0.4,
                                   kl_temperature=1.6, teacher_grads=False)
    assert got["teacher_ce"] == 0.0
    _assert_match(got, ref, ["loss", "student_ce", "kl", "grad_student_hidden", "grad_weight"])


def test_precomputed_logits_matches_torch_float64_reference():
    hs, _, W, _, y = _inputs(104, N=11, H=7, V=23)
    lt = _rng(5).standard_normal((11, 23)) * 0.3
    ref = _torch_ref("precomputed", hs, W, y, lt=lt, w_s=1.0, w_t=0.0, kl_w=0.3, T=1.5, reduction="mean")
    got = distillation_loss_oracle("precomputed", hs, W, y, teacher_logits=lt, kl_weight=0.3, kl_temperature=1.5)
    _assert_match(got, ref, ["loss", "student_ce", "kl", "grad_student_hidden", "grad_weight"])


def test_precomputed_hidden_equals_precomputed_logits():
    hs, ht, W, Wt, y = _inputs(105, N=11, H=7, V=23, Ht=9)
    a = distillation_loss_oracle("precomputed", hs, W, y, teacher_hidden=ht, teacher_weight=Wt, kl_weight=0.3,
                                 kl_temperature=1.5)
    b = distillation_loss_oracle("precomputed", hs, W, y, teacher_logits=ht @ Wt.T, kl_weight=0.3,
                                 kl_temperature=1.5)
    _assert_match(a, b, ["loss", "kl", "grad_student_hidden", "grad_weight"], tol=1e-12)


def test_all_ignored_rows_give_exact_zeros():
    hs, ht, W, _, _ = _inputs(106, N=8, H=6, V=13)
    y = np.full(8, -100)
    out = distillation_loss_oracle("tied", hs, W, y, teacher_hidden=ht, kl_weight=0.5, kl_temperature=1.7)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        assert out[k] == 0.0
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden"):
        assert not np.any(out[k])


def test_sum_equals_mean_times_count():
    hs, ht, W, _, y = _inputs(7, N=12, V=30)
    kw = dict(teacher_hidden=ht, kl_weight=0.6, kl_temperature=2.0, divergence="jsd")
    m = distillation_loss_oracle("tied", hs, W, y, reduction="mean", **kw)
    s = distillation_loss_oracle("tied", hs, W, y, reduction="sum", **kw)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        assert np.isclose(s[k], m[k] * m["count"], rtol=1e-12)


def test_kernel_semantics_zero_kl_when_weight_zero():
    hs, ht, W, _, y = _inputs(8)
    k = distillation_loss_oracle("tied", hs, W, y, teacher_hidden=ht, kl_weight=0.0)
    t = distillation_loss_oracle("tied", hs, W, y, teacher_hidden=ht, kl_weight=0.0, kernel_semantics=False)
    assert k["kl"] == 0.0 and t["kl"] > 0.0
    assert k["loss"] == t["loss"]


def test_out_of_range_label_is_class_zero():
    hs, ht, W, _, y = _inputs(9, ignore_every=0)
    y2 = y.copy()
    y2[3] = 10_000
    y3 = y.copy()
    y3[3] = 0
    a = distillation_loss_oracle("tied", hs, W, y2, teacher_hidden=ht, kl_weight=0.2)
    b = distillation_loss_oracle("tied", hs, W, y3, teacher_hidden=ht, kl_weight=0.2)
    _assert_match(a, b, ["loss", "grad_student_hidden", "grad_weight"], tol=0)


# ---------------------------------------------------------------- divergences
def _probs(seed, rows=5, V=12, scale=1.5):
    r = _rng(seed)
    return r.standard_normal((rows, V)) * scale, r.standard_normal((rows, V)) * scale


def _softmax(z):
    e = np.exp(z - z.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def test_kl_values_match_scipy_entropy():
    zt, zs = _probs(1)
    pt, ps = _softmax(zt), _softmax(zs)
    f, _ = divergence_value_and_grad(zt, zs, "forward_kl")
    r, _ = divergence_value_and_grad(zt, zs, "reverse_kl")
    s, _ = divergence_value_and_grad(zt, zs, "symmetric_kl")
    c, _ = divergence_value_and_grad(zt, zs, "soft_target_ce")
    for i in range(zt.shape[0]):
        assert np.isclose(f[i], entropy(pt[i], ps[i]), rtol=1e-12)
        assert np.isclose(r[i], entropy(ps[i], pt[i]), rtol=1e-12)
        assert np.isclose(s[i], entropy(pt[i], ps[i]) + entropy(ps[i], pt[i]), rtol=1e-12)
        assert np.isclose(c[i], entropy(pt[i], ps[i]) + entropy(pt[i]), rtol=1e-12)


def test_jsd_matches_scipy_jensenshannon():
    zt, zs = _probs(2)
    pt, ps = _softmax(zt), _softmax(zs)
    v, _ = divergence_value_and_grad(zt, zs, "jsd", beta=0.5)
    for i in range(zt.shape[0]):
        assert np.isclose(v[i], jensenshannon(pt[i], ps[i]) ** 2, rtol=1e-10)


def test_tvd_matches_l1_definition_and_pinsker():
    zt, zs = _probs(3)
    pt, ps = _softmax(zt), _softmax(zs)
    v, _ = divergence_value_and_grad(zt, zs, "tvd")
    f, _ = divergence_value_and_grad(zt, zs, "forward_kl")
    for i in range(zt.shape[0]):
        assert np.isclose(v[i], np.max([np.sum(np.maximum(pt[i] - ps[i], 0)), 0.0]), rtol=1e-12)  # TV = sum (p-q)_+
        assert v[i] <= np.sqrt(f[i] / 2) + 1e-12  # Pinsker


def test_power_family_identities():
    zt, zs = _probs(4)
    pt, ps = _softmax(zt), _softmax(zs)
    hel, _ = divergence_value_and_grad(zt, zs, "hellinger")
    bha, _ = divergence_value_and_grad(zt, zs, "bhattacharyya")
    ren, _ = divergence_value_and_grad(zt, zs, "renyi", alpha=0.5)
    ama, _ = divergence_value_and_grad(zt, zs, "amari_alpha", alpha=0.5)
    ab, _ = divergence_value_and_grad(zt, zs, "ab", alpha=0.5, beta=0.5)
    ab2, _ = divergence_value_and_grad(zt, zs, "ab", alpha=0.3, beta=0.7)
    am3, _ = divergence_value_and_grad(zt, zs, "amari_alpha", alpha=0.3)
    chi, _ = divergence_value_and_grad(zt, zs, "chi_squared")
    l2, _ = divergence_value_and_grad(zt, zs, "squared_l2")
    fkl, _ = divergence_value_and_grad(zt, zs, "forward_kl")
    ren1, _ = divergence_value_and_grad(zt, zs, "renyi", alpha=1.0 - 1e-6)
    bc = np.sum(np.sqrt(pt * ps), -1)
    np.testing.assert_allclose(hel, 1 - bc, rtol=1e-12)
    np.testing.assert_allclose(bha, -np.log(bc), rtol=1e-12)
    np.testing.assert_allclose(ren, 2 * bha, rtol=1e-12)          # Renyi(1/2) = 2 Bhattacharyya
    np.testing.assert_allclose(ama, 4 * hel, rtol=1e-12)          # Amari(1/2) = 4 H^2
    np.testing.assert_allclose(ab, 4 * hel, rtol=1e-12)           # AB(1/2,1/2) = 4 H^2
    np.testing.assert_allclose(ab2, am3, rtol=1e-10)              # AB(a, 1-a) = Amari(a)
    np.testing.assert_allclose(ren1, fkl, rtol=1e-4)              # Renyi -> KL as alpha -> 1
    np.testing.assert_allclose(chi, np.sum((pt - ps) ** 2 / ps, -1), rtol=1e-12)
    np.testing.assert_allclose(l2, np.sum((pt - ps) ** 2, -1), rtol=1e-12)


def test_skew_divergences_reduce_to_kl_at_alpha_zero():
    zt, zs = _probs(5)
    f, gf = divergence_value_and_grad(zt, zs, "forward_kl")
    r, gr = divergence_value_and_grad(zt, zs, "reverse_kl")
    sf, gsf = divergence_value_and_grad(zt, zs, "skew_forward_kl", alpha=0.0)
    sr, gsr = divergence_value_and_grad(zt, zs, "skew_reverse_kl", alpha=0.0)
    np.testing.assert_allclose(sf, f, rtol=1e-12)
    np.testing.assert_allclose(sr, r, rtol=1e-12)
    np.testing.assert_allclose(gsf, gf, rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(gsr, gr, rtol=1e-10, atol=1e-14)


# ------------------------------------------- pins off the symmetric points
# The checks above leave five formulas where a plausible slip would not
# show: chi-squared and squared L2 were compared with restatements of
# themselves, AB only at alpha + beta = 1 (where swapping its a/(a+b) and
# b/(a+b) coefficients changes nothing), JSD only at beta = 1/2 (where
# swapping p_t and p_s changes nothing) and the skew KLs only at alpha = 0.
# Each pin below reaches the value by another route: a library routine
# (scipy.stats.entropy), an identity with a divergence pinned elsewhere, or a
# limit of the published definition.  Each pin is a function of the
# divergence evaluator, so the planted-slip tests further down can show that
# it rejects the slip it is meant to catch.
def _div(zt, zs, name, **kw):
    return divergence_value_and_grad(zt, zs, name, **kw)[0]


def _pin_chi_squared(zt, zs):
    """Pearson chi^2 (Renyi 1961; van Erven and Harremoes 2014, eq. (7)):
    the Renyi divergence of order 2 is log(1 + chi^2(P || Q)), and Renyi
    orders increase, so KL = D_1 <= D_2 = log(1 + chi^2).  Renyi itself is
    pinned at alpha = 1/2 (2 Bhattacharyya) and alpha -> 1 (KL) above."""
    chi = _div(zt, zs, "chi_squared")
    np.testing.assert_allclose(_div(zt, zs, "renyi", alpha=2.0), np.log1p(chi), rtol=1e-10)
    assert np.all(_div(zt, zs, "forward_kl") <= np.log1p(chi) + 1e-12)


def _pin_squared_l2(zt, zs):
    """AB(1, 1) = -sum(p q - p^2/2 - q^2/2) = ||p - q||^2 / 2 (Cichocki,
    Cruces and Amari 2011, the alpha = beta = 1 case), with ||p - q|| taken
    from numpy's 2-norm."""
    pt, ps = _softmax(zt), _softmax(zs)
    l2 = _div(zt, zs, "squared_l2")
    np.testing.assert_allclose(l2, np.linalg.norm(pt - ps, axis=-1) ** 2, rtol=1e-10)
    np.testing.assert_allclose(_div(zt, zs, "ab", alpha=1.0, beta=1.0), 0.5 * l2, rtol=1e-10)


def _pin_ab_off_the_line(zt, zs):
    """AB(alpha, beta) away from alpha + beta = 1, by its limits (Cichocki
    et al. 2011, eq. (22)-(23)): as beta -> 0 it tends to the generalised KL
    of the powered measures, (1/alpha^2) sum(p^a log(p^a / q^a) - p^a + q^a),
    and at alpha = 1 that is KL(p_t || p_s) (pinned by scipy above); as
    alpha -> 0 it tends to (1/beta^2) sum(q^b log(q^b / p^b) - q^b + p^b)."""
    lt, ls = np.log(_softmax(zt)), np.log(_softmax(zs))
    eps = 1e-6
    for a in (0.6, 1.0, 1.7):
        pa, qa = np.exp(a * lt), np.exp(a * ls)
        want = (pa * (a * lt - a * ls) - pa + qa).sum(-1) / a ** 2
        np.testing.assert_allclose(_div(zt, zs, "ab", alpha=a, beta=eps), want, rtol=1e-4)
    np.testing.assert_allclose(_div(zt, zs, "ab", alpha=1.0, beta=eps),
                               [entropy(p, q) for p, q in zip(_softmax(zt), _softmax(zs))], rtol=1e-4)
    for b in (0.3, 0.9):
        pb, qb = np.exp(b * lt), np.exp(b * ls)
        want = (qb * (b * ls - b * lt) - qb + pb).sum(-1) / b ** 2
        np.testing.assert_allclose(_div(zt, zs, "ab", alpha=eps, beta=b), want, rtol=1e-4)


def _pin_jsd(zt, zs):
    """Generalised JSD with mixture m = beta p_t + (1 - beta) p_s:
    beta KL(p_t || m) + (1 - beta) KL(p_s || m) = H(m) - beta H(p_t) -
    (1 - beta) H(p_s), entropies from scipy."""
    pt, ps = _softmax(zt), _softmax(zs)
    for b in (0.25, 0.5, 0.75):
        v = _div(zt, zs, "jsd", beta=b)
        for i in range(zt.shape[0]):
            m = b * pt[i] + (1 - b) * ps[i]
            want = entropy(m) - b * entropy(pt[i]) - (1 - b) * entropy(ps[i])
            np.testing.assert_allclose(v[i], want, rtol=1e-9, atol=1e-15)


def _pin_skew(zt, zs):
    """DistiLLM's skew KLs (Ko et al. 2024, eq. (3)-(4)) with scipy's
    relative entropy: skew forward KL(p_t || a p_t + (1 - a) p_s), skew
    reverse KL(p_s || a p_s + (1 - a) p_t)."""
    pt, ps = _softmax(zt), _softmax(zs)
    for a in (0.1, 0.3):
        f = _div(zt, zs, "skew_forward_kl", alpha=a)
        r = _div(zt, zs, "skew_reverse_kl", alpha=a)
        for i in range(zt.shape[0]):
            np.testing.assert_allclose(f[i], entropy(pt[i], a * pt[i] + (1 - a) * ps[i]), rtol=1e-10)
            np.testing.assert_allclose(r[i], entropy(ps[i], a * ps[i] + (1 - a) * pt[i]), rtol=1e-10)


_PINS = {"chi_squared": _pin_chi_squared, "squared_l2": _pin_squared_l2, "ab": _pin_ab_off_the_line,
         "jsd": _pin_jsd, "skew": _pin_skew}


@pytest.mark.parametrize("pin", sorted(_PINS))
def test_divergence_pins_off_the_symmetric_points(pin):
    for seed, scale in ((11, 1.5), (12, 4.0)):
        zt, zs = _probs(seed, rows=6, V=20, scale=scale)
        _PINS[pin](zt, zs)


# Planted slips: each replaces one oracle formula with a plausible mistake
# (on the CPU, in the oracle's table) and shows that its pin fails.
def _neyman_chi2(pt, ps, lt, ls, a, b):
    return ((pt - ps) ** 2 / pt).sum(), 2.0 * (ps - pt) / pt


def _half_l2(pt, ps, lt, ls, a, b):
    return 0.5 * ((pt - ps) ** 2).sum(), ps - pt


def _ab_swapped_coefficients(pt, ps, lt, ls, a, b):
    s = a + b
    v = -(np.exp(a * lt + b * ls) - b / s * np.exp(s * lt) - a / s * np.exp(s * ls)).sum() / (a * b)
    return v, np.zeros_like(ps)


def _jsd_swapped_arguments(pt, ps, lt, ls, a, b):
    m = (1 - b) * pt + b * ps
    return b * entropy(pt, m) + (1 - b) * entropy(ps, m), np.zeros_like(ps)


def _skew_forward_swapped_weights(pt, ps, lt, ls, a, b):
    return entropy(pt, (1 - a) * pt + a * ps), np.zeros_like(ps)


_SLIPS = [("chi_squared", "chi_squared", _neyman_chi2, None, None),
          ("squared_l2", "squared_l2", _half_l2, None, None),
          ("ab", "ab", _ab_swapped_coefficients, 0.5, 0.5),
          ("jsd", "jsd", _jsd_swapped_arguments, None, 0.5),
          ("skew", "skew_forward_kl", _skew_forward_swapped_weights, 0.1, None)]


@pytest.mark.parametrize("pin,name,slip,da,db", _SLIPS, ids=[s[0] for s in _SLIPS])
def test_divergence_pins_reject_planted_slips(monkeypatch, pin, name, slip, da, db):
    import oracle.orda_oracle as orc

    zt, zs = _probs(11, rows=6, V=20)
    monkeypatch.setitem(orc.DIVERGENCE_DEFS, name, (slip, da, db))
    with pytest.raises(AssertionError):
        _PINS[pin](zt, zs)


@pytest.mark.parametrize("name", DIVS)
def test_divergence_is_zero_at_equal_distributions(name):
    zt, _ = _probs(6)
    v, g = divergence_value_and_grad(zt, zt + 0.7, name)  # shifted logits: same distribution
    if name == "soft_target_ce":
        np.testing.assert_allclose(v, [entropy(p) for p in _softmax(zt)], rtol=1e-12)
    else:
        np.testing.assert_allclose(v, 0.0, atol=1e-12)
        if name != "tvd":  # |.| has no gradient at 0
            np.testing.assert_allclose(g, 0.0, atol=1e-12)


@pytest.mark.parametrize("name", DIVS)
def test_divergence_gradient_matches_finite_differences(name):
    zt, zs = _probs(7, rows=2, V=7)
    _, g = divergence_value_and_grad(zt, zs, name)
    eps = 1e-6
    num = np.zeros_like(zs)
    for i in range(zs.shape[0]):
        for j in range(zs.shape[1]):
            zp, zm = zs.copy(), zs.copy()
            zp[i, j] += eps
            zm[i, j] -= eps
            vp, _ = divergence_value_and_grad(zt, zp, name)
            vm, _ = divergence_value_and_grad(zt, zm, name)
            num[i, j] = (vp[i] - vm[i]) / (2 * eps)
    np.testing.assert_allclose(g, num, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("name", DIVS)
def test_divergence_gradient_matches_torch_autograd(name):
    from orda_ce_kernel.divergences import divergence_rows_torch, resolve_divergence

    zt, zs = _probs(8, rows=3, V=9)
    _, g = divergence_value_and_grad(zt, zs, name)
    zs_t = torch.tensor(zs, requires_grad=True)
    v = divergence_rows_torch(torch.log_softmax(zs_t, -1), torch.log_softmax(torch.tensor(zt), -1),
                              resolve_divergence(name))
    v.sum().backward()
    np.testing.assert_allclose(zs_t.grad.numpy(), g, rtol=1e-9, atol=1e-12)


def _fd(fn, arr, eps=1e-6):
    num = np.zeros_like(arr)
    for idx in np.ndindex(arr.shape):
        orig = arr[idx]
        arr[idx] = orig + eps
        lp = fn()
        arr[idx] = orig - eps
        lm = fn()
        arr[idx] = orig
        num[idx] = (lp - lm) / (2 * eps)
    return num


def test_loss_gradient_matches_finite_differences_with_temperature():
    """The teacher distribution is detached in the divergence (reference
    api.py:319), so finite differences through the teacher path are taken
    with the divergence off, and the divergence's W gradient is checked with
    the teacher logits held fixed (precomputed mode)."""
    hs, ht, W, _, y = _inputs(11, N=4, H=3, V=6)
    kw = dict(teacher_hidden=ht, kl_weight=0.7, kl_temperature=2.5, divergence="jsd", teacher_ce_weight=0.3)
    out = distillation_loss_oracle("tied", hs, W, y, **kw)
    num = _fd(lambda: distillation_loss_oracle("tied", hs, W, y, **kw)["loss"], hs)
    np.testing.assert_allclose(out["grad_student_hidden"], num, rtol=1e-5, atol=1e-8)

    kw_ce = dict(kw, kl_weight=0.0)
    out_ce = distillation_loss_oracle("tied", hs, W, y, **kw_ce)
    for arr, key in ((ht, "grad_teacher_hidden"), (W, "grad_weight")):
        num = _fd(lambda: distillation_loss_oracle("tied", hs, W, y, **kw_ce)["loss"], arr)
        np.testing.assert_allclose(out_ce[key], num, rtol=1e-5, atol=1e-8, err_msg=key)
    assert np.allclose(out["grad_teacher_hidden"], out_ce["grad_teacher_hidden"])

    lt = ht @ W.T
    kw_p = dict(teacher_logits=lt, kl_weight=0.7, kl_temperature=2.5, divergence="jsd")
    out_p = distillation_loss_oracle("precomputed", hs, W, y, **kw_p)
    num = _fd(lambda: distillation_loss_oracle("precomputed", hs, W, y, **kw_p)["loss"], W)
    np.testing.assert_allclose(out_p["grad_weight"], num, rtol=1e-5, atol=1e-8)


# ------------------------------------------------ dlogits from rounded logits
def test_round_to_matches_torch_conversions():
    """round_to's bfloat16 / float16 rounding is torch's (round to nearest
    even), exact ties and the fp32 step included."""
    r = _rng(5)
    x = np.concatenate([r.standard_normal(20000) * 10.0 ** r.integers(-6, 6, 20000),
                        [0.0, -0.0, 1.0, -3.5, 65504.0, 1e-30]])
    # exact bf16 ties: fp32 patterns whose low 16 bits are 0x8000
    ties = (r.integers(0x3F000000, 0x43000000, 2000, dtype=np.uint32) & 0xFFFF0000) | 0x8000
    x = np.concatenate([x, ties.view(np.float32).astype(np.float64)])
    xt = torch.tensor(x, dtype=torch.float64).float()
    np.testing.assert_array_equal(round_to(x, "bfloat16"), xt.bfloat16().double().numpy())
    small = x[np.abs(x) < 60000]
    np.testing.assert_array_equal(round_to(small, "float16"),
                                  torch.tensor(small).float().half().double().numpy())
    np.testing.assert_array_equal(round_to(x, None), x)


def test_rounded_logits_option_is_a_no_op_on_representable_logits():
    """With one-hot student and teacher hidden rows the logits are columns of
    a bf16 W, which bfloat16 holds exactly: the option must change nothing."""
    r = _rng(6)
    N, H, V = 12, 12, 40
    W = round_to(r.standard_normal((V, H)) * 2.0, "bfloat16")
    hs = np.eye(N, H)
    ht = np.roll(np.eye(N, H), 3, axis=1)
    y = r.integers(0, V, N)
    y[::5] = -100
    for div in ("forward_kl", "jsd", "hellinger"):
        kw = dict(teacher_hidden=ht, kl_weight=0.6, kl_temperature=2.0, teacher_ce_weight=0.4, divergence=div)
        a = distillation_loss_oracle("tied", hs, W, y, **kw)
        b = distillation_loss_oracle("tied", hs, W, y, grad_logits_dtype="bfloat16", **kw)
        for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden"):
            np.testing.assert_array_equal(a[k], b[k], err_msg=k)


def test_rounded_logits_option_rounds_the_logits_the_dlogits_see():
    """Against a direct restatement: softmax dlogits of the rounded student
    logits (the student CE part only: w_t = kl = 0), and the row-sum
    invariant (softmax dlogits sum to zero per row) still holds."""
    hs, ht, W, _, y = _inputs(7, N=6, H=5, V=30)
    hs, W = hs * 3.0, W * 3.0
    out = distillation_loss_oracle("tied", hs, W, y, teacher_hidden=ht, teacher_ce_weight=0.0,
                                   grad_logits_dtype="bfloat16")
    x = round_to(hs @ W.T, "bfloat16")
    p = np.exp(x - x.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    keep = y != -100
    p[np.arange(len(y))[keep], y[keep]] -= 1.0
    p[~keep] = 0.0
    want = p / keep.sum()
    np.testing.assert_allclose(out["dlogits_student"], want, rtol=1e-12, atol=1e-15)
    assert np.abs(out["dlogits_student"].sum(1)).max() < 1e-15
    plain = distillation_loss_oracle("tied", hs, W, y, teacher_hidden=ht, teacher_ce_weight=0.0)
    assert np.abs(plain["dlogits_student"] - want).max() > 1e-6  # the rounding is visible at this scale
