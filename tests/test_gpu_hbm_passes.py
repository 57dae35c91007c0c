"""GPU: the HBM-bound passes at shapes where one launch holds both full
blocks (the paths without per-row guards) and ragged ones, against the
oracle.

``k_dlm_tm`` and ``k_two_rows_tm`` (precomputed logits read in place) take
256-token x 64-row blocks, and ``k_two_rows`` 256-token blocks over
64-row-multiple vocabulary ranges; blocks wholly inside the chunk take an
unguarded path.  With N = 600 tokens in 512-token chunks (in place) or
256-token chunks (separate teacher) and V = 1032 (16 full 64-row tiles and
8 rows), every launch has full blocks, a ragged token block and a ragged
vocabulary tile.  Checked: the four loss values (1e-3 relative) and the
gradients within the scale-relative bounds of ``tests/_divgrad.py``, for the
one-pass, two-pass and one-term power divergences (the latter on the ring
scan with staged or in-place teacher logits; chi-squared over a computed
teacher on the two-stage scan).  The tied and no-teacher cases run the ring
scans' staged logits stores on full token tiles (and the per-block stores on
the ragged one) beside the 8-row vocabulary tail.
"""
from __future__ import annotations

import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle
from tests import _divgrad as D

pytestmark = pytest.mark.gpu

N, V = 600, 1032


def _orda():
    import orda_ce_kernel

    assert orda_ce_kernel.is_available(), "liborda_ce.so must load on a HIP device"
    return orda_ce_kernel


def _np(x):
    return x.detach().double().cpu().numpy()


CASES = [
    # (mode, divergence, T, w_s)
    ("in_place", "forward_kl", 1.0, 1.0),
    ("in_place", "reverse_kl", 2.0, 0.0),
    ("in_place", "jsd", 2.0, 1.0),
    ("in_place", "tvd", 1.0, 0.0),
    ("in_place", "skew_forward_kl", 4.0, 0.0),
    ("in_place", "hellinger", 1.0, 0.0),
    ("in_place", "chi_squared", 1.0, 0.0),
    ("separate", "jsd", 2.0, 1.0),
    ("separate", "skew_reverse_kl", 1.0, 0.0),
    ("separate", "hellinger", 2.0, 0.0),
    ("separate", "chi_squared", 1.0, 0.0),
    # the ring scans' staged logits stores at full token tiles beside a
    # vocabulary tail: tied tiles (128 tokens, both halves) and student-only
    # tiles (256 tokens, no teacher term)
    ("tied", "forward_kl", 1.0, 1.0),
    ("no_teacher", "forward_kl", 1.0, 1.0),
]


@pytest.mark.parametrize("mode, div, T, w_s", CASES, ids=[f"{c[0]}-{c[1]}-T{c[2]:g}" for c in CASES])
def test_hbm_passes_with_full_and_ragged_blocks(mode, div, T, w_s):
    o = _orda()
    hs, W, ht, hts, Wt, y = D.make_inputs(29, torch.bfloat16, n=N, v=V)
    hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
    kl_w = 0.0 if mode == "no_teacher" else 1.0
    if mode in ("tied", "no_teacher"):
        teacher, omode, okw = o.TiedTeacher(ht.cuda()), "tied", dict(teacher_hidden=_np(ht))
    elif mode == "in_place":
        lt = (hts.float() @ Wt.float().t()).to(torch.bfloat16)
        teacher, omode, okw = o.PrecomputedTeacher(logits=lt.cuda()), "precomputed", dict(teacher_logits=_np(lt))
    else:
        teacher, omode = o.SeparateTeacher(hts.cuda(), Wt.cuda()), "separate"
        okw = dict(teacher_hidden=_np(hts), teacher_weight=_np(Wt), teacher_grads=False)
    out = o.distillation_loss(hs_d, W_d, y.cuda(), teacher, student_ce_weight=w_s, teacher_ce_weight=0.0,
                              kl_weight=kl_w, kl_temperature=T, divergence=div, backend="triton",
                              config=o.KernelConfig(chunk_size=128))
    out.loss.backward()
    torch.cuda.synchronize()
    ref = distillation_loss_oracle(omode, _np(hs), _np(W), y.numpy(), student_ce_weight=w_s, teacher_ce_weight=0.0,
                                   kl_weight=kl_w, kl_temperature=T, divergence=div, grad_logits_dtype="bfloat16",
                                   **okw)
    for key in ("loss", "student_ce", "teacher_ce", "kl"):
        got = float(getattr(out, key).detach())
        assert abs(got - ref[key]) <= 1e-3 * abs(ref[key]) + 1e-5, (mode, div, key, got, ref[key])
    for got, key in ((hs_d.grad, "grad_student_hidden"), (W_d.grad, "grad_weight")):
        ok, msg = D.grad_ok(_np(got), ref[key], torch.bfloat16, div)
        assert ok, f"{mode} {div} T={T} {key}: {msg}"
