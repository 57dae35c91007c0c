"""Pins the chunked float32 torch reference used by the full-size GPU tests
against the float64 oracle on small shapes (CPU only)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle
from tests._fp32_reference import DIVERGENCES, fp32_reference


def _case(mode, div, *, N=70, H=24, Ht=40, V=300, seed=7, T=2.0, w_t=None, kl_w=0.6, chunk=32):
    g = torch.Generator().manual_seed(seed)
    hs = torch.randn(N, H, generator=g)
    W = 0.3 * torch.randn(V, H, generator=g)
    ht_dim = H if mode == "tied" else Ht
    ht = torch.randn(N, ht_dim, generator=g)
    Wt = 0.3 * torch.randn(V, ht_dim, generator=g)
    lt = torch.log_softmax(3.0 * torch.randn(N, V, generator=g), 1)
    y = torch.randint(0, V, (N,), generator=g)
    y[::9] = -100
    y[5] = V + 3  # out of range: class 0
    got = fp32_reference(mode, hs, W, y, ht=ht, Wt=None if mode == "tied" else Wt, lt=lt, student_ce_weight=0.7,
                         teacher_ce_weight=w_t, kl_weight=kl_w, kl_temperature=T, divergence=div, chunk=chunk)
    kw = {"tied": dict(teacher_hidden=ht.double().numpy()),
          "separate": dict(teacher_hidden=ht.double().numpy(), teacher_weight=Wt.double().numpy()),
          "precomputed": dict(teacher_logits=lt.double().numpy())}[mode]
    want = distillation_loss_oracle(mode, hs.double().numpy(), W.double().numpy(), y.numpy(), student_ce_weight=0.7,
                                    teacher_ce_weight=w_t, kl_weight=kl_w, kl_temperature=T, divergence=div,
                                    teacher_grads=False, **kw)
    return got, want


@pytest.mark.parametrize("mode", ["tied", "separate", "precomputed"])
@pytest.mark.parametrize("div", DIVERGENCES)
def test_fp32_reference_matches_oracle(mode, div):
    got, want = _case(mode, div)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        assert abs(got[k] - want[k]) <= 1e-5 * abs(want[k]) + 1e-6, (k, got[k], want[k])
    for k in ("grad_student_hidden", "grad_weight"):
        np.testing.assert_allclose(got[k].double().numpy(), want[k], rtol=1e-4, atol=1e-7, err_msg=k)


def test_fp32_reference_teacher_ce_and_kl_weight_zero():
    got, want = _case("tied", "forward_kl", w_t=0.0, kl_w=0.0)
    assert got["teacher_ce"] == 0.0 and got["kl"] == 0.0 and want["kl"] == 0.0
    assert abs(got["loss"] - want["loss"]) <= 1e-5 * abs(want["loss"])
    np.testing.assert_allclose(got["grad_weight"].double().numpy(), want["grad_weight"], rtol=1e-4, atol=1e-7)


def test_fp32_reference_is_chunk_independent():
    a, _ = _case("tied", "jsd", chunk=13)
    b, _ = _case("tied", "jsd", chunk=70)
    assert abs(a["loss"] - b["loss"]) <= 1e-6 * abs(b["loss"])
    assert torch.allclose(a["grad_weight"], b["grad_weight"], rtol=1e-5, atol=1e-8)


def test_fp32_reference_catches_a_dropped_temperature_factor():
    """A plausible slip (the T^2 factor left out) moves the loss well outside
    the tolerance the GPU tests use, so the comparison can see it."""
    got, want = _case("tied", "forward_kl", T=2.0)
    wrong = got["loss"] - 0.6 * got["kl"] * (1 - 1 / 4.0)
    assert abs(wrong - want["loss"]) > 1e-3 * abs(want["loss"])
