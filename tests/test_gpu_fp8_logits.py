"""GPU: the fp8 logits GEMM (``logits_gemm="fp8"``, ``ORDA_FP8_LOGITS``).

Two checks per case:

* faithfulness -- against the oracle with the same operand rounding
  (``fp8_operands=True``: W and the hidden rows rounded per row to E4M3 with
  a power-of-two scale, pinned against torch's ``float8_e4m3fn`` on the CPU in
  ``tests/test_fp8_logits.py``): the products of e4m3 values are exact in
  fp32, so only the summation order differs -- losses within 1e-4 relative,
  gradients within the bf16 bounds of ``tests/_divgrad.py``;
* accuracy -- against exact logits (the plain oracle): losses within
  ``FP8_LOSS_REL`` and gradients within ``(FP8_GRAD_MAX, FP8_GRAD_FRO)``, the
  tolerance stated with the flag.

Cases: tied teacher (student CE + teacher CE + divergence, T = 1 and 2, a
two-pass divergence), precomputed logits read in place, no teacher term,
multi-chunk, and the flag together with the fused RMSNorm.
"""
from __future__ import annotations

import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle
from tests import _divgrad as D
from tests.test_fp8_logits import FP8_GRAD_FRO, FP8_GRAD_MAX, FP8_LOSS_REL

pytestmark = pytest.mark.gpu

H8 = 256  # fp8 needs hidden > 128 and a multiple of 16


def _orda():
    import orda_ce_kernel

    assert orda_ce_kernel.is_available(), "liborda_ce.so must load on a HIP device"
    return orda_ce_kernel


def _np(x):
    return x.detach().double().cpu().numpy()


CASES = {
    # id: (mode, divergence, T, chunk, w_s, w_t, kl_w)
    "tied_fkl_T1": ("tied", "forward_kl", 1.0, 48, 1.0, 1.0, 1.0),
    "tied_fkl_T2": ("tied", "forward_kl", 2.0, None, 1.0, 1.0, 1.0),
    "tied_jsd_T2": ("tied", "jsd", 2.0, 48, 0.5, 0.0, 1.0),
    "tied_rkl_kl_only": ("tied", "reverse_kl", 1.0, None, 0.0, 0.0, 1.0),
    "pre_logits_fkl": ("precomputed_logits", "forward_kl", 1.0, 48, 1.0, 0.0, 1.0),
    "pre_logits_soft_T2": ("precomputed_logits", "soft_target_ce", 2.0, None, 1.0, 0.0, 0.7),
    "student_ce_only": ("tied", "forward_kl", 1.0, 48, 1.0, 0.0, 0.0),
}


def _run(o, case, seed=83, norm=False):
    mode, div, T, chunk, w_s, w_t, kl_w = CASES[case]
    hs, W, ht, hts, Wt, y = D.make_inputs(seed, torch.bfloat16, h=H8)
    hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
    if mode == "tied":
        teacher, omode, okw = o.TiedTeacher(ht.cuda()), "tied", dict(teacher_hidden=_np(ht))
    else:
        lt = (hts.float() @ Wt.float().t()).to(torch.bfloat16)
        teacher, omode, okw = o.PrecomputedTeacher(logits=lt.cuda()), "precomputed", dict(teacher_logits=_np(lt))
    kw = {}
    nw = None
    if norm:
        nw = (1.0 + 0.3 * torch.randn(H8, generator=torch.Generator().manual_seed(seed))).to(torch.bfloat16)
        nw_d = nw.cuda().requires_grad_(True)
        kw = dict(student_norm=o.StudentRMSNorm(nw_d, eps=1e-5))
    cfg = o.KernelConfig(chunk_size=chunk) if chunk else None
    out = o.distillation_loss(hs_d, W_d, y.cuda(), teacher, student_ce_weight=w_s, teacher_ce_weight=w_t,
                              kl_weight=kl_w, kl_temperature=T, divergence=div, backend="triton", config=cfg,
                              logits_gemm="fp8", **kw)
    out.loss.backward()
    torch.cuda.synchronize()
    got = {k: float(getattr(out, k).detach()) for k in ("loss", "student_ce", "teacher_ce", "kl")}
    got["grad_student_hidden"] = _np(hs_d.grad)
    got["grad_weight"] = _np(W_d.grad)
    if norm:
        got["grad_student_norm_weight"] = _np(nw_d.grad)
    refkw = dict(student_ce_weight=w_s, teacher_ce_weight=w_t, kl_weight=kl_w, kl_temperature=T, divergence=div,
                 grad_logits_dtype="bfloat16", **okw)
    if norm:
        refkw.update(student_norm_weight=_np(nw), norm_eps=1e-5, normed_dtype="bfloat16")
    ref8 = distillation_loss_oracle(omode, _np(hs), _np(W), y.numpy(), fp8_operands=True, **refkw)
    exact = distillation_loss_oracle(omode, _np(hs), _np(W), y.numpy(), **refkw)
    return got, ref8, exact, div


@pytest.mark.parametrize("case", list(CASES))
def test_fp8_logits_match_the_fp8_oracle(case):
    o = _orda()
    got, ref8, _, div = _run(o, case)
    for key in ("loss", "student_ce", "teacher_ce", "kl"):
        assert abs(got[key] - ref8[key]) <= 1e-4 * abs(ref8[key]) + 1e-6, (case, key, got[key], ref8[key])
    for key in ("grad_student_hidden", "grad_weight"):
        ok, msg = D.grad_ok(got[key], ref8[key], torch.bfloat16, div)
        assert ok, f"{case} {key}: {msg}"


@pytest.mark.parametrize("case", list(CASES))
def test_fp8_logits_within_the_stated_tolerance_of_exact(case):
    o = _orda()
    got, _, exact, _ = _run(o, case)
    for key in ("loss", "student_ce", "teacher_ce", "kl"):
        assert abs(got[key] - exact[key]) <= FP8_LOSS_REL * abs(exact[key]) + 1e-6, (case, key, got[key], exact[key])
    for key in ("grad_student_hidden", "grad_weight"):
        worst, fro = D.grad_errors(got[key], exact[key])
        assert worst <= FP8_GRAD_MAX and fro <= FP8_GRAD_FRO, (case, key, worst, fro)


def test_fp8_logits_with_the_fused_rmsnorm():
    o = _orda()
    got, ref8, _, div = _run(o, "tied_fkl_T2", seed=89, norm=True)
    for key in ("loss", "student_ce", "teacher_ce", "kl"):
        assert abs(got[key] - ref8[key]) <= 1e-4 * abs(ref8[key]) + 1e-6, (key, got[key], ref8[key])
    for key in ("grad_student_hidden", "grad_weight", "grad_student_norm_weight"):
        ok, msg = D.grad_ok(got[key], ref8[key], torch.bfloat16, div)
        assert ok, f"{key}: {msg}"


def test_fp8_logits_are_bit_stable():
    o = _orda()
    hs, W, ht, _, _, y = D.make_inputs(97, torch.bfloat16, n=300, v=2000, h=H8)
    res = []
    for _ in range(2):
        hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
        out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TiedTeacher(ht.cuda()), kl_weight=0.7, backend="triton",
                                  config=o.KernelConfig(chunk_size=64), logits_gemm="fp8")
        out.loss.backward()
        res.append([t.detach() for t in out] + [hs_d.grad, W_d.grad])
    for i, (a, b) in enumerate(zip(*res)):
        assert torch.equal(a, b), i
