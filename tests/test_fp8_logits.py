"""CPU: the fp8 logits GEMM (``logits_gemm="fp8"``, ``ORDA_FP8_LOGITS``) --
the oracle's E4M3 rounding, the per-row power-of-two scaling, the torch
formulation of the flag, the flag's accuracy against exact logits, and the
C-ABI's validation.

The reference has no fp8 path (its logits GEMM is a bf16 ``torch.mm``,
``ops/tied_teacher.py:444-445``), so the operand rounding is pinned against
torch's own ``float8_e4m3fn`` conversion and the rest of the loss against the
pinned oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle, quantize_rows_e4m3, round_e4m3
from orda_ce_kernel import _native
from tests import _divgrad as D

import orda_ce_kernel as o


def test_e4m3_rounding_matches_torch_float8():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000) * np.exp2(rng.uniform(-14, 8.5, 100000))
    x = np.clip(x, -448, 448)
    # exact ties between neighbours (normal and subnormal), and the extremes
    grid = torch.arange(0, 256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    grid = np.unique(grid[np.isfinite(grid) & (np.abs(grid) <= 448)])
    ties = (grid[1:] + grid[:-1]) / 2
    x = np.concatenate([x, ties, -ties, grid, [0.0, 448.0, -448.0, 2.0 ** -9, 2.0 ** -10]])
    want = torch.tensor(x).to(torch.float8_e4m3fn).double().numpy()
    np.testing.assert_array_equal(round_e4m3(x), want)


def test_row_scaling_puts_each_row_amax_in_range():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 96)) * np.exp2(rng.uniform(-20, 20, (64, 1)))
    x[3] = 0.0
    q = quantize_rows_e4m3(x)
    amax = np.abs(x).max(axis=1)
    m, k = np.frexp(np.where(amax > 0, amax, 1.0))
    e = np.where(amax > 0, k - 9 + (m > 0.875), 0)
    scaled = amax / np.exp2(e)
    assert np.all((scaled[amax > 0] > 224) & (scaled[amax > 0] <= 448))
    assert np.all(q[3] == 0.0)
    np.testing.assert_array_equal(quantize_rows_e4m3(q), q)  # idempotent
    # relative error of the normal-range values: at most half a step, 2^-4
    big = np.abs(x) >= np.exp2(e - 6)[:, None]
    rel = np.abs(q - x)[big] / np.abs(x)[big]
    assert rel.max() <= 2.0 ** -4 + 1e-12


@pytest.mark.parametrize("mode", ["tied", "precomputed_logits", "student_only"])
def test_torch_formulation_matches_the_fp8_oracle(mode):
    hs, W, ht, hts, Wt, y = D.make_inputs(5, torch.float64, n=24, h=32, v=60)
    hs_t, W_t = hs.clone().requires_grad_(True), W.clone().requires_grad_(True)
    n = lambda x: x.double().numpy()  # noqa: E731
    if mode == "tied":
        teacher, omode, kw, w_t, kl = o.TiedTeacher(ht), "tied", dict(teacher_hidden=n(ht)), 0.6, 0.8
    elif mode == "precomputed_logits":
        lt = hts @ Wt.t()
        teacher, omode, kw, w_t, kl = o.PrecomputedTeacher(logits=lt), "precomputed", dict(teacher_logits=n(lt)), 0.0, 0.8
    else:
        teacher, omode, kw, w_t, kl = o.TiedTeacher(ht), "tied", dict(teacher_hidden=n(ht)), 0.0, 0.0
    out = o.distillation_loss(hs_t, W_t, y, teacher, teacher_ce_weight=w_t, kl_weight=kl, kl_temperature=1.5,
                              logits_gemm="fp8")
    out.loss.backward()
    # (the torch formulation reports the divergence with kl_weight = 0 too)
    ref = distillation_loss_oracle(omode, n(hs), n(W), y.numpy(), teacher_ce_weight=w_t, kl_weight=kl,
                                   kl_temperature=1.5, fp8_operands=True, kernel_semantics=False, **kw)
    for key in ("loss", "student_ce", "teacher_ce", "kl"):
        assert float(getattr(out, key).detach()) == pytest.approx(ref[key], rel=1e-10, abs=1e-12), key
    np.testing.assert_allclose(hs_t.grad.numpy(), ref["grad_student_hidden"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(W_t.grad.numpy(), ref["grad_weight"], rtol=1e-9, atol=1e-12)


# The flag's accuracy against exact logits, as documented with it: loss
# components within FP8_LOSS_REL, gradients within (FP8_GRAD_MAX, FP8_GRAD_FRO)
# of the scale-relative bounds (worst |err| / max|ref|, Frobenius).  The
# gradient bound is set by the distillation term alone (student and teacher
# CE weights 0), which differences two distributions whose logits both carry
# the e4m3 rounding (~3.6% RMS per operand element): up to 7% (Frobenius) on
# the CPU oracle over forward/reverse/symmetric KL, JSD, soft CE and Hellinger
# at T = 1, 2, 4; with the CE terms present about 2%.  TVD's gradient is a sign
# function of p_s - p_t and has no such bound.
FP8_LOSS_REL = 1e-2
FP8_GRAD_MAX, FP8_GRAD_FRO = 0.15, 0.1


@pytest.mark.parametrize("div", ["forward_kl", "reverse_kl", "jsd"])
@pytest.mark.parametrize("T", [1.0, 2.0])
def test_fp8_oracle_stays_within_the_stated_tolerance_of_exact(div, T):
    hs, W, ht, _, _, y = D.make_inputs(71, torch.bfloat16, h=256)
    n = lambda x: x.double().numpy()  # noqa: E731
    kw = dict(teacher_hidden=n(ht), teacher_ce_weight=1.0, kl_weight=1.0, kl_temperature=T, divergence=div,
              grad_logits_dtype="bfloat16")
    exact = distillation_loss_oracle("tied", n(hs), n(W), y.numpy(), **kw)
    f8 = distillation_loss_oracle("tied", n(hs), n(W), y.numpy(), fp8_operands=True, **kw)
    for key in ("loss", "student_ce", "teacher_ce", "kl"):
        assert abs(f8[key] - exact[key]) <= FP8_LOSS_REL * abs(exact[key]), key
    for key in ("grad_student_hidden", "grad_weight"):
        worst, fro = D.grad_errors(f8[key], exact[key])
        assert worst <= FP8_GRAD_MAX and fro <= FP8_GRAD_FRO, (key, worst, fro)
        # and the rounding is visible: these bounds are not vacuous
        assert fro > 1e-3


def test_fp8_arguments_are_checked():
    hs, W, ht, hts, Wt, y = D.make_inputs(7, torch.float64, n=8, h=32, v=40)
    with pytest.raises(ValueError, match="logits_gemm"):
        o.distillation_loss(hs, W, y, o.TiedTeacher(ht), logits_gemm="fp4")
    lp = torch.log_softmax(hts @ Wt.t(), dim=1)
    vals, idx = lp.topk(4, dim=1)
    with pytest.raises(ValueError, match="TopKTeacher"):
        o.distillation_loss(hs, W, y, o.TopKTeacher(idx, vals), kl_weight=1.0, logits_gemm="fp8")


def _abi_problem(**kw):
    p = _native.Problem()
    p.abi_version = _native.ABI_VERSION
    p.mode, p.dtype = 0, 0
    p.n_rows, p.vocab, p.hidden, p.teacher_hidden = 4096, 32000, 2048, 2048
    p.ignore_index = -100
    p.flags = 0x3 | 0x10 | 0x20 | 0x80 | 0x400
    p.temperature = 1.0
    p.student_ce_weight = p.teacher_ce_weight = p.kl_weight = 1.0
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize(
    "kw, message",
    [
        (dict(flags=0x3 | 0x400), "ORDA_GRADS_IN_FORWARD"),
        (dict(dtype=2), "16-bit"),
        (dict(hidden=2056, teacher_hidden=2056), "multiple of 16"),
        (dict(hidden=128, teacher_hidden=128), "> 128"),
        (dict(mode=1, teacher_hidden=1024), "tied teacher"),          # separate: staged teacher logits
        (dict(mode=2, logits_dtype=0, divergence=4), "tied teacher"),  # precomputed, power family
        (dict(mode=4, topk=16, flags=0x3 | 0x20 | 0x80 | 0x400, teacher_ce_weight=0.0), "top-k"),
    ],
)
def test_invalid_fp8_problems_are_rejected(kw, message):
    with pytest.raises(ValueError, match=message):
        _native.forward_workspace_bytes(_abi_problem(**kw))


def test_fp8_workspace_holds_the_e4m3_operands():
    p = _abi_problem(token_chunk=512)
    with_f8 = _native.forward_workspace_bytes(p)
    p.flags &= ~0x400
    plain = _native.forward_workspace_bytes(p)
    chunk = _native.plan_info(p)["token_chunk"]
    # W in e4m3 plus the chunk's student and teacher rows
    assert with_f8 - plain >= 32000 * 2048 + 2 * chunk * 2048
