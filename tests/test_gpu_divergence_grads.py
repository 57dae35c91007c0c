"""GPU: the distillation term's gradients, isolated, against the oracle.

``student_ce_weight = teacher_ce_weight = 0`` and ``kl_weight = 1``, so
``grad_student_hidden`` and ``grad_weight`` are ``T dD/dz_s`` through the
LM-head GEMMs alone; every divergence (non-default parameters too) at
T = 1, 2, 4, in every schedule and teacher source the kernels have:

* ``tied_f32``: float32 (two-stage engine), balanced schedule;
* ``tied_bf16``: ring scan, two tokens per lane, 96-token chunks (96 + 64,
  grad W accumulated across chunks in bf16);
* ``tied_bf16_debug``: the two-phase schedule (scan, then recompute);
* ``separate_bf16``: the student-only Function, teacher logits from their
  own GEMM staged in the chunk buffer;
* ``pre_hidden_bf16``: a frozen (hidden, weight) teacher, as above;
* ``pre_logits_bf16``: logits read in place (V a multiple of 8);
* ``pre_logits_bf16_ring``: V = 1004 (a multiple of 4, not 8): read by the
  ring scan and written to the chunk buffer;
* ``pre_logits_bf16_staged``: V = 998: transposed into the chunk buffer.

Bounds and their power to fail are in ``tests/_divgrad.py`` and
``tests/test_divergence_grad_bounds.py``.  Also here: bit-stable losses and
gradients for every divergence in both schedules.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle
from tests import _divgrad as D

pytestmark = pytest.mark.gpu

VARIANTS = {
    # id: (mode, dtype, profile, chunk_size, V)
    "tied_f32": ("tied", torch.float32, "balanced", None, D.V),
    "tied_bf16": ("tied", torch.bfloat16, "balanced", 48, D.V),
    "tied_bf16_debug": ("tied", torch.bfloat16, "debug", None, D.V),
    "separate_bf16": ("separate", torch.bfloat16, "balanced", None, D.V),
    "pre_hidden_bf16": ("precomputed_hidden", torch.bfloat16, "balanced", None, D.V),
    "pre_logits_bf16": ("precomputed_logits", torch.bfloat16, "balanced", None, D.V),
    "pre_logits_bf16_ring": ("precomputed_logits", torch.bfloat16, "balanced", None, 1004),
    "pre_logits_bf16_staged": ("precomputed_logits", torch.bfloat16, "balanced", None, 998),
}


def _orda():
    import orda_ce_kernel

    assert orda_ce_kernel.is_available(), "liborda_ce.so must load on a HIP device"
    return orda_ce_kernel


def _np(x):
    return x.detach().double().cpu().numpy()


@pytest.mark.parametrize("case", D.DIV_CASES, ids=D.DIV_IDS)
@pytest.mark.parametrize("variant", list(VARIANTS))
def test_divergence_gradient_matches_oracle(variant, case):
    from orda_ce_kernel.divergences import Divergence

    o = _orda()
    mode, dtype, profile, chunk, V = VARIANTS[variant]
    _, name, a, b = case
    div = Divergence(name, a, b)
    hs, W, ht, hts, Wt, y = D.make_inputs(17, dtype, v=V)
    cfg = o.KernelConfig(chunk_size=chunk) if chunk else None
    for T in D.TEMPERATURES:
        hs_d = hs.cuda().requires_grad_(True)
        W_d = W.cuda().requires_grad_(True)
        if mode == "tied":
            teacher, kw, omode = o.TiedTeacher(ht.cuda()), dict(teacher_hidden=_np(ht)), "tied"
        elif mode == "separate":
            teacher = o.SeparateTeacher(hts.cuda(), Wt.cuda())
            kw, omode = dict(teacher_hidden=_np(hts), teacher_weight=_np(Wt)), "separate"
        elif mode == "precomputed_hidden":
            teacher = o.PrecomputedTeacher(teacher_hidden=hts.cuda(), teacher_weight=Wt.cuda())
            kw, omode = dict(teacher_hidden=_np(hts), teacher_weight=_np(Wt)), "precomputed"
        else:
            lt = (hts.float() @ Wt.float().t()).to(dtype)
            teacher, kw, omode = o.PrecomputedTeacher(logits=lt.cuda()), dict(teacher_logits=_np(lt)), "precomputed"
        out = o.distillation_loss(hs_d, W_d, y.cuda(), teacher, student_ce_weight=0.0, teacher_ce_weight=0.0,
                                  kl_weight=1.0, kl_temperature=T, backend="triton", profile=profile, config=cfg,
                                  divergence=div)
        out.loss.backward()
        torch.cuda.synchronize()
        ref = distillation_loss_oracle(omode, _np(hs), _np(W), y.numpy(), student_ce_weight=0.0,
                                       teacher_ce_weight=0.0, kl_weight=1.0, kl_temperature=T, divergence=name,
                                       alpha=a, beta=b, teacher_grads=False,
                                       grad_logits_dtype=D.grad_logits_dtype(dtype), **kw)
        got_kl = float(out.kl)
        assert abs(got_kl - ref["kl"]) <= 1e-3 * abs(ref["kl"]) + 1e-5, (variant, name, T, got_kl, ref["kl"])
        for got, key in ((hs_d.grad, "grad_student_hidden"), (W_d.grad, "grad_weight")):
            ok, msg = D.grad_ok(_np(got), ref[key], dtype, name)
            assert ok, f"{variant} {name} a={a} b={b} T={T} {key}: {msg}"


@pytest.mark.parametrize("name", sorted({c[1] for c in D.DIV_CASES}))
@pytest.mark.parametrize("profile", ["balanced", "debug"])
def test_every_divergence_is_bit_stable(name, profile):
    """Two identical calls give bit-identical losses and gradients (fixed
    reduction orders, no float atomics), for every divergence in both
    schedules; 300 tokens in 128-token chunks, V = 2000."""
    o = _orda()
    hs, W, ht, _, _, y = D.make_inputs(23, torch.bfloat16, n=300, v=2000)
    res = []
    for _ in range(2):
        hs_d, W_d, ht_d = (x.cuda().requires_grad_(True) for x in (hs, W, ht))
        out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TiedTeacher(ht_d), kl_weight=0.7, kl_temperature=2.0,
                                  backend="triton", profile=profile, config=o.KernelConfig(chunk_size=64),
                                  divergence=name)
        out.loss.backward()
        res.append([t.detach() for t in out] + [hs_d.grad, W_d.grad, ht_d.grad])
    for i, (a, b) in enumerate(zip(*res)):
        assert torch.equal(a, b), (name, profile, i)
