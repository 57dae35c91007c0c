"""GPU: the student's RMSNorm fused in front of the loss
(``student_norm=StudentRMSNorm(w, eps)``) against the oracle.

The oracle applies the reference producer's norm (``x * rsqrt(mean(x^2) +
eps) * w``, ``test/benchmark/src/core.py:13-14``) in float64, rounds ``y`` to
the compute dtype as the kernels store it, and differentiates through it by
the chain rule (pinned on the CPU in ``tests/test_rmsnorm_prologue.py``).
Checked: the four loss values (1e-3 relative), ``dloss/dx``, ``dloss/dW`` and
``dloss/dw`` (the norm weight) within the scale-relative bounds of
``tests/_divgrad.py``; every teacher mode; a two-pass divergence (JSD); a
hidden size that is not a multiple of 8 (the library pads x and w with zero
columns and takes the mean over the true size); multi-chunk schedules (the
norm weight's gradient summed over chunks); the norm weight with and without
``requires_grad``; bit-stable repeats.
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


def _inputs(seed, dtype, h=D.H):
    hs, W, ht, hts, Wt, y = D.make_inputs(seed, dtype, h=h)
    g = torch.Generator().manual_seed(seed + 1)
    # pre-norm rows of uneven scale, and a norm weight away from 1
    x = (hs.float() * (0.5 + 2.0 * torch.rand(hs.shape[0], 1, generator=g))).to(dtype)
    nw = (1.0 + 0.4 * torch.randn(h, generator=g)).to(dtype)
    return x, nw, W, ht, hts, Wt, y


CASES = {
    # id: (mode, dtype, divergence, T, chunk, w_s, w_t, kl_w, h)
    "tied_bf16_fkl": ("tied", torch.bfloat16, "forward_kl", 1.0, 48, 1.0, 1.0, 0.5, D.H),
    "tied_bf16_kl_only_T2": ("tied", torch.bfloat16, "forward_kl", 2.0, None, 0.0, 0.0, 1.0, D.H),
    "tied_f32": ("tied", torch.float32, "forward_kl", 2.0, 48, 1.0, 1.0, 0.5, D.H),
    "separate_bf16_jsd": ("separate", torch.bfloat16, "jsd", 2.0, 48, 0.7, 0.0, 1.0, D.H),
    "pre_logits_bf16": ("precomputed_logits", torch.bfloat16, "reverse_kl", 1.0, None, 1.0, 0.0, 1.0, D.H),
    "pre_hidden_bf16": ("precomputed_hidden", torch.bfloat16, "forward_kl", 4.0, 48, 1.0, 0.0, 1.0, D.H),
    "topk_bf16": ("topk", torch.bfloat16, "forward_kl", 2.0, 48, 1.0, 0.0, 1.0, D.H),
    "tied_bf16_h122": ("tied", torch.bfloat16, "forward_kl", 1.0, 48, 1.0, 1.0, 0.5, 122),
    "student_ce_only_bf16": ("tied", torch.bfloat16, "forward_kl", 1.0, 48, 1.0, 0.0, 0.0, D.H),
}


@pytest.mark.parametrize("norm_grad", [True, False], ids=["dw", "no_dw"])
@pytest.mark.parametrize("case", list(CASES))
def test_rmsnorm_prologue_matches_oracle(case, norm_grad):
    o = _orda()
    mode, dtype, div, T, chunk, w_s, w_t, kl_w, h = CASES[case]
    x, nw, W, ht, hts, Wt, y = _inputs(53, dtype, h=h)
    x_d = x.cuda().requires_grad_(True)
    nw_d = nw.cuda().requires_grad_(norm_grad)
    W_d = W.cuda().requires_grad_(True)
    okw = {}
    if mode == "tied":
        teacher, omode, okw = o.TiedTeacher(ht.cuda()), "tied", dict(teacher_hidden=_np(ht))
    elif mode == "separate":
        teacher, omode = o.SeparateTeacher(hts.cuda(), Wt.cuda()), "separate"
        okw = dict(teacher_hidden=_np(hts), teacher_weight=_np(Wt), teacher_grads=False)
    elif mode == "precomputed_logits":
        lt = (hts.float() @ Wt.float().t()).to(dtype)
        teacher, omode, okw = o.PrecomputedTeacher(logits=lt.cuda()), "precomputed", dict(teacher_logits=_np(lt))
    elif mode == "precomputed_hidden":
        teacher = o.PrecomputedTeacher(teacher_hidden=hts.cuda(), teacher_weight=Wt.cuda())
        omode, okw = "precomputed", dict(teacher_hidden=_np(hts), teacher_weight=_np(Wt))
    else:
        lp = torch.log_softmax(hts.double() @ Wt.double().t(), dim=1)
        vals, idx = lp.topk(32, dim=1)
        teacher = o.TopKTeacher(idx.cuda(), vals.float().cuda())
        omode, okw = "precomputed", dict(teacher_logits=topk_dense_logits(idx.numpy(), vals.float().double().numpy(),
                                                                          D.V))
    cfg = o.KernelConfig(chunk_size=chunk) if chunk else None
    out = o.distillation_loss(x_d, W_d, y.cuda(), teacher, student_ce_weight=w_s, teacher_ce_weight=w_t,
                              kl_weight=kl_w, kl_temperature=T, backend="triton", config=cfg, divergence=div,
                              student_norm=o.StudentRMSNorm(nw_d, eps=1e-5))
    out.loss.backward()
    torch.cuda.synchronize()
    gld = D.grad_logits_dtype(dtype)
    ref = distillation_loss_oracle(omode, _np(x), _np(W), y.numpy(), student_ce_weight=w_s, teacher_ce_weight=w_t,
                                   kl_weight=kl_w, kl_temperature=T, divergence=div, grad_logits_dtype=gld,
                                   student_norm_weight=_np(nw), norm_eps=1e-5, normed_dtype=gld, **okw)
    for key in ("loss", "student_ce", "teacher_ce", "kl"):
        got = float(getattr(out, key).detach())
        assert abs(got - ref[key]) <= 1e-3 * abs(ref[key]) + 1e-5, (case, key, got, ref[key])
    checks = [(x_d.grad, "grad_student_hidden"), (W_d.grad, "grad_weight")]
    if norm_grad:
        checks.append((nw_d.grad, "grad_student_norm_weight"))
    else:
        assert nw_d.grad is None
    for got, key in checks:
        assert got is not None and got.shape == ({"grad_student_hidden": x.shape, "grad_weight": W.shape,
                                                  "grad_student_norm_weight": nw.shape}[key])
        ok, msg = D.grad_ok(_np(got), ref[key], dtype, div)
        assert ok, f"{case} {key}: {msg}"


def test_rmsnorm_prologue_is_bit_stable():
    o = _orda()
    x, nw, W, ht, _, _, y = _inputs(59, torch.bfloat16)
    res = []
    for _ in range(2):
        x_d, nw_d, W_d = (t.cuda().requires_grad_(True) for t in (x, nw, W))
        out = o.distillation_loss(x_d, W_d, y.cuda(), o.TiedTeacher(ht.cuda()), kl_weight=0.7, backend="triton",
                                  config=o.KernelConfig(chunk_size=48), student_norm=o.StudentRMSNorm(nw_d))
        out.loss.backward()
        res.append([t.detach() for t in out] + [x_d.grad, nw_d.grad, W_d.grad])
    for i, (a, b) in enumerate(zip(*res)):
        assert torch.equal(a, b), i


def test_rmsnorm_prologue_matches_the_unfused_producer_in_fp32():
    """Against the reference producer's formula in torch float32 on the GPU
    followed by this package's own kernels without the prologue: the same
    loss, and the same gradients once autograd takes the norm's backward."""
    o = _orda()
    x, nw, W, ht, _, _, y = _inputs(61, torch.float32)
    res = []
    for fused in (True, False):
        x_d, nw_d, W_d = (t.cuda().requires_grad_(True) for t in (x, nw, W))
        if fused:
            out = o.distillation_loss(x_d, W_d, y.cuda(), o.TiedTeacher(ht.cuda()), kl_weight=0.7, backend="triton",
                                      student_norm=o.StudentRMSNorm(nw_d, eps=1e-6))
        else:
            yv = x_d * torch.rsqrt(x_d.pow(2).mean(-1, keepdim=True) + 1e-6) * nw_d
            out = o.distillation_loss(yv, W_d, y.cuda(), o.TiedTeacher(ht.cuda()), kl_weight=0.7, backend="triton")
        out.loss.backward()
        res.append((float(out.loss), _np(x_d.grad), _np(nw_d.grad), _np(W_d.grad)))
    (la, *ga), (lb, *gb) = res
    assert la == pytest.approx(lb, rel=1e-5)
    for a, b in zip(ga, gb):
        ok, msg = D.grad_ok(a, b, torch.float32)
        assert ok, msg
