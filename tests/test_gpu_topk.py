"""GPU: the top-k teacher (``TopKTeacher``) against the oracle.

The oracle reads a top-k teacher as precomputed teacher logits equal to its
log-probabilities on its ids and -inf elsewhere (``topk_dense_logits``; the
reading is pinned on the CPU in ``tests/test_topk_teacher.py``).  The HIP
path never forms those logits: the student-only ring scan, a per-token pass
over the k ids (fp32 dot products for the student's logits there), the dense
dlogits pass with a zero teacher and a scatter of the ids' share.

Cases: k = 1, 16, 64 (one wave's worth of ids), 100 (two passes of 64, the
second partial) and V (every id, in descending order); T = 1 and 2; forward
KL and soft-target CE; bf16 and fp32; multi-chunk (96 + 64 tokens) and
single-chunk schedules; ignored rows.  Losses within 1e-3 relative; gradients
within the scale-relative bounds of the other divergence tests
(``tests/_divgrad.py``) with the distillation term isolated, and the
combined loss (student CE + distillation) likewise.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle, topk_dense_logits
from tests import _divgrad as D

pytestmark = pytest.mark.gpu


def _orda():
    import orda_ce_kernel

    assert orda_ce_kernel.is_available(), "liborda_ce.so must load on a HIP device"
    return orda_ce_kernel


def _np(x):
    return x.detach().double().cpu().numpy()


def _teacher(seed: int, hts, Wt, k: int):
    """Top-k (ids, log-probs) of an independent teacher, ids descending."""
    lt = hts.double() @ Wt.double().t()
    lp = torch.log_softmax(lt, dim=1)
    vals, idx = lp.topk(k, dim=1)
    return idx, vals.float()


def _check(o, dtype, k, T, div, chunk, w_s, kl_w, reduction="mean", seed=31):
    hs, W, _, hts, Wt, y = D.make_inputs(seed, dtype)
    idx, lp = _teacher(seed, hts, Wt, k)
    hs_d = hs.cuda().requires_grad_(True)
    W_d = W.cuda().requires_grad_(True)
    cfg = o.KernelConfig(chunk_size=chunk) if chunk else None
    out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TopKTeacher(idx.cuda(), lp.cuda()), student_ce_weight=w_s,
                              kl_weight=kl_w, kl_temperature=T, reduction=reduction, backend="triton", config=cfg,
                              divergence=div)
    out.loss.backward()
    torch.cuda.synchronize()
    ref = distillation_loss_oracle("precomputed", _np(hs), _np(W), y.numpy(),
                                   teacher_logits=topk_dense_logits(idx.numpy(), lp.double().numpy(), D.V),
                                   student_ce_weight=w_s, teacher_ce_weight=0.0, kl_weight=kl_w, kl_temperature=T,
                                   reduction=reduction, divergence=div, grad_logits_dtype=D.grad_logits_dtype(dtype))
    tag = f"{dtype} k={k} T={T} {div} chunk={chunk} w_s={w_s} kl={kl_w} {reduction}"
    for key in ("loss", "student_ce", "kl"):
        got = float(getattr(out, key).detach())
        assert abs(got - ref[key]) <= 1e-3 * abs(ref[key]) + 1e-5, (tag, key, got, ref[key])
    assert float(out.teacher_ce) == 0.0
    for got, key in ((hs_d.grad, "grad_student_hidden"), (W_d.grad, "grad_weight")):
        ok, msg = D.grad_ok(_np(got), ref[key], dtype, div)
        assert ok, f"{tag} {key}: {msg}"


@pytest.mark.parametrize("div", ["forward_kl", "soft_target_ce"])
@pytest.mark.parametrize("k", [1, 16, 64, 100, D.V])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_topk_distillation_gradient_matches_oracle(dtype, k, div):
    o = _orda()
    for T in (1.0, 2.0):
        _check(o, dtype, k, T, div, chunk=48 if dtype == torch.bfloat16 else None, w_s=0.0, kl_w=1.0)


@pytest.mark.parametrize("reduction", ["mean", "sum"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_topk_with_student_ce_matches_oracle(dtype, reduction):
    o = _orda()
    _check(o, dtype, 64, 2.0, "forward_kl", chunk=None, w_s=1.0, kl_w=0.5, reduction=reduction)
    _check(o, dtype, 16, 1.0, "soft_target_ce", chunk=48, w_s=0.7, kl_w=1.3, reduction=reduction)


def test_topk_without_divergence_is_the_student_ce():
    """kl_weight = 0: the student-only ring scan alone; the student CE and its
    gradients as the oracle's, and as a TiedTeacher call with every teacher
    term off."""
    o = _orda()
    hs, W, ht, hts, Wt, y = D.make_inputs(37, torch.bfloat16)
    idx, lp = _teacher(37, hts, Wt, 8)
    res = []
    for teacher in (o.TopKTeacher(idx.cuda(), lp.cuda()), o.TiedTeacher(ht.cuda())):
        hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
        out = o.distillation_loss(hs_d, W_d, y.cuda(), teacher, teacher_ce_weight=0.0, kl_weight=0.0,
                                  backend="triton")
        out.loss.backward()
        res.append((float(out.loss), _np(hs_d.grad), _np(W_d.grad)))
    ref = distillation_loss_oracle("tied", _np(hs), _np(W), y.numpy(), teacher_hidden=_np(ht), teacher_ce_weight=0.0,
                                   grad_logits_dtype="bfloat16")
    for loss, g_hs, g_w in res:
        assert abs(loss - ref["loss"]) <= 1e-3 * abs(ref["loss"])
        for got, key in ((g_hs, "grad_student_hidden"), (g_w, "grad_weight")):
            ok, msg = D.grad_ok(got, ref[key], torch.bfloat16)
            assert ok, f"{key}: {msg}"


def test_topk_is_bit_stable():
    """Two identical calls: bit-identical losses and gradients (the ids of a
    row are distinct, so the scatter has one writer per element)."""
    o = _orda()
    hs, W, _, hts, Wt, y = D.make_inputs(41, torch.bfloat16, n=300, v=2000)
    idx, lp = _teacher(41, hts, Wt, 64)
    res = []
    for _ in range(2):
        hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
        out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TopKTeacher(idx.cuda(), lp.cuda()), kl_weight=0.7,
                                  kl_temperature=2.0, backend="triton", config=o.KernelConfig(chunk_size=64))
        out.loss.backward()
        res.append([t.detach() for t in out] + [hs_d.grad, W_d.grad])
    for i, (a, b) in enumerate(zip(*res)):
        assert torch.equal(a, b), i


def test_topk_int32_ids_and_shuffled_order():
    """int32 ids, and ids in any order within a row, give the int64 /
    descending-order result (the loss does not depend on the order)."""
    o = _orda()
    hs, W, _, hts, Wt, y = D.make_inputs(43, torch.bfloat16)
    idx, lp = _teacher(43, hts, Wt, 32)
    perm = torch.stack([torch.randperm(32, generator=torch.Generator().manual_seed(i)) for i in range(idx.shape[0])])
    outs = []
    for ids, vals in ((idx, lp), (idx.gather(1, perm).int(), lp.gather(1, perm))):
        hs_d = hs.cuda().requires_grad_(True)
        out = o.distillation_loss(hs_d, W.cuda(), y.cuda(), o.TopKTeacher(ids.cuda(), vals.cuda()), kl_weight=1.0,
                                  backend="triton")
        out.loss.backward()
        outs.append((float(out.kl), _np(hs_d.grad)))
    assert outs[0][0] == pytest.approx(outs[1][0], rel=1e-5)
    np.testing.assert_allclose(outs[0][1], outs[1][1], rtol=0, atol=1e-2 * np.abs(outs[0][1]).max())


def test_topk_ignored_rows_with_no_teacher_mass_give_finite_gradients():
    """Padding tokens (label -100) whose top-k log-probabilities are all
    -inf: they add nothing (exact zeros in their dlogits, no NaN carried
    into grad W by the scatter), so the result equals the oracle's with any
    finite teacher on those rows."""
    o = _orda()
    hs, W, _, hts, Wt, y = D.make_inputs(61, torch.bfloat16)
    idx, lp = _teacher(61, hts, Wt, 16)
    ign = torch.nonzero(y == -100).flatten()
    assert ign.numel() > 0
    lp_pad = lp.clone()
    lp_pad[ign] = -float("inf")
    hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
    out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TopKTeacher(idx.cuda(), lp_pad.cuda()), kl_weight=1.0,
                              kl_temperature=2.0, backend="triton", config=o.KernelConfig(chunk_size=48))
    out.loss.backward()
    torch.cuda.synchronize()
    assert torch.isfinite(hs_d.grad).all() and torch.isfinite(W_d.grad).all()
    assert not torch.any(hs_d.grad[ign.cuda()])
    ref = distillation_loss_oracle("precomputed", _np(hs), _np(W), y.numpy(),
                                   teacher_logits=topk_dense_logits(idx.numpy(), lp.double().numpy(), D.V),
                                   teacher_ce_weight=0.0, kl_weight=1.0, kl_temperature=2.0,
                                   grad_logits_dtype="bfloat16")
    for key in ("loss", "student_ce", "kl"):
        got = float(getattr(out, key).detach())
        assert abs(got - ref[key]) <= 1e-3 * abs(ref[key]) + 1e-5, (key, got, ref[key])
    for got, key in ((hs_d.grad, "grad_student_hidden"), (W_d.grad, "grad_weight")):
        ok, msg = D.grad_ok(_np(got), ref[key], torch.bfloat16)
        assert ok, f"{key}: {msg}"
