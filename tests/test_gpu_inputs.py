"""GPU: input forms the hot path accepts, against the float64 oracle.

* non-contiguous (transposed) inputs in all five teacher modes, as the
  reference tests them (``test/correctness/test_public_api_cuda.py:397-504``:
  BT=16, Hs=32, Ht=48, V=257, fp16, every 4th label ignored, T=1.4,
  chunk_size=7); here with the divergence term isolated as well;
* precomputed teacher logits in float32 with a bf16 student, in both
  schedules: taken as the compute dtype holds them, as the reference casts
  them to the compute dtype first (``ops/precomputed_teacher.py:340-348``);
* precomputed teacher log-probs with part of the vocabulary masked to a
  large finite negative value, for every divergence and each way the
  teacher's logits reach the kernels;
* autocast to bf16 / fp16 around float32 inputs (compute dtype from the
  autocast, ``_runtime.py:41-80``; gradients come back in float32);
* a second backward through a retained graph (and ``autograd.grad`` then
  ``backward``), with ``grad_output`` != 1: each gradient is scaled once.

Gradient bounds: ``tests/_divgrad.py``.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle
from tests import _divgrad as D

pytestmark = pytest.mark.gpu


def _orda():
    import orda_ce_kernel

    assert orda_ce_kernel.is_available(), "liborda_ce.so must load on a HIP device"
    return orda_ce_kernel


def _np(x):
    return x.detach().double().cpu().numpy()


def _noncontig(x: torch.Tensor) -> torch.Tensor:
    """The same values as a transposed (non-contiguous) view on the GPU."""
    v = x.t().contiguous().cuda().t()
    assert v.shape == x.shape and not v.is_contiguous()
    return v


def _check_scalars(out, ref, what):
    for name in ("loss", "student_ce", "teacher_ce", "kl"):
        got, want = float(getattr(out, name)), ref[name]
        assert abs(got - want) <= 1e-3 * abs(want) + 1e-5, (what, name, got, want)


def _check_grad(got, want, dtype, what, div="forward_kl"):
    assert got is not None, what
    ok, msg = D.grad_ok(_np(got), want, dtype, div)
    assert ok, f"{what}: {msg}"


MODES = ["tied", "separate", "separate-full", "precomputed-logits", "precomputed-hidden"]


@pytest.mark.parametrize("isolated", [False, True], ids=["all_terms", "divergence_only"])
@pytest.mark.parametrize("mode", MODES)
def test_noncontiguous_inputs(mode, isolated):
    o = _orda()
    dtype = torch.float16
    BT, Hs, Ht, V = 16, 32, 48, 257
    g = torch.Generator().manual_seed(301)
    hs = torch.randn(BT, Hs, generator=g).to(dtype)
    W = (torch.randn(V, Hs, generator=g) * (1.5 / Hs ** 0.5)).to(dtype)
    ht_t = torch.randn(BT, Hs, generator=g).to(dtype)
    ht_s = torch.randn(BT, Ht, generator=g).to(dtype)
    Wt = (torch.randn(V, Ht, generator=g) * (1.5 / Ht ** 0.5)).to(dtype)
    y = torch.randint(0, V, (BT,), generator=g)
    y[::4] = -100
    full = mode in ("tied", "separate-full")
    w_s, w_t = (0.0, 0.0) if isolated else (1.0, (1.0 if full else None))
    hs_d, W_d = _noncontig(hs).requires_grad_(True), _noncontig(W).requires_grad_(True)
    extra = {}
    if mode == "tied":
        ht_d = _noncontig(ht_t).requires_grad_(True)
        teacher, kw, omode = o.TiedTeacher(ht_d), dict(teacher_hidden=_np(ht_t)), "tied"
        extra["grad_teacher_hidden"] = ht_d
    elif mode.startswith("separate"):
        ht_d = _noncontig(ht_s).requires_grad_(full)
        Wt_d = _noncontig(Wt).requires_grad_(full)
        teacher = o.SeparateTeacher(ht_d, Wt_d)
        kw, omode = dict(teacher_hidden=_np(ht_s), teacher_weight=_np(Wt)), "separate"
        if full:
            extra["grad_teacher_hidden"], extra["grad_teacher_weight"] = ht_d, Wt_d
    elif mode == "precomputed-logits":
        lt = (ht_s.float() @ Wt.float().t()).to(dtype)
        teacher, kw, omode = o.PrecomputedTeacher(logits=_noncontig(lt)), dict(teacher_logits=_np(lt)), "precomputed"
    else:
        teacher = o.PrecomputedTeacher(teacher_hidden=_noncontig(ht_s), teacher_weight=_noncontig(Wt))
        kw, omode = dict(teacher_hidden=_np(ht_s), teacher_weight=_np(Wt)), "precomputed"
    out = o.distillation_loss(hs_d, W_d, y.cuda(), teacher, student_ce_weight=1.0 if not isolated else 0.0,
                              teacher_ce_weight=w_t, kl_weight=0.35 if not isolated else 1.0, kl_temperature=1.4,
                              backend="triton", config=o.KernelConfig(chunk_size=7))
    out.loss.backward()
    torch.cuda.synchronize()
    ref = distillation_loss_oracle(omode, _np(hs), _np(W), y.numpy(), student_ce_weight=1.0 if not isolated else 0.0,
                                   teacher_ce_weight=w_t, kl_weight=0.35 if not isolated else 1.0, kl_temperature=1.4,
                                   teacher_grads=full, grad_logits_dtype="float16", **kw)
    _check_scalars(out, ref, mode)
    assert hs_d.grad.shape == hs_d.shape and W_d.grad.shape == W_d.shape
    _check_grad(hs_d.grad, ref["grad_student_hidden"], dtype, f"{mode} grad_student_hidden")
    _check_grad(W_d.grad, ref["grad_weight"], dtype, f"{mode} grad_weight")
    for key, t in extra.items():
        if isolated:  # no teacher CE: a zero gradient, or none (separate: student-only Function)
            assert t.grad is None or torch.count_nonzero(t.grad) == 0, (mode, key)
            continue
        assert t.grad.shape == t.shape
        _check_grad(t.grad, ref[key], dtype, f"{mode} {key}")


@pytest.mark.parametrize("profile", ["balanced", "debug"], ids=["grads_in_forward", "two_phase"])
@pytest.mark.parametrize("div, T", [("forward_kl", 1.0), ("reverse_kl", 2.0), ("jsd", 2.0), ("hellinger", 4.0),
                                    ("tvd", 1.0)])
def test_float32_teacher_logits_with_bf16_student(div, T, profile):
    """fp32 logits and a bf16 student: the teacher's logits are taken as the
    compute dtype holds them -- the reference casts each chunk into a bf16
    buffer (ops/precomputed_teacher.py:343-348) -- in both schedules (the
    default one stages them through a cast-transpose), the student runs in
    bf16.  Against the oracle on the bf16-rounded logits, and within the loss
    tolerance of the unrounded ones (the reference's unfused torch path keeps
    them in fp32).  Divergence term isolated, and all terms."""
    o = _orda()
    hs, W, _, hts, Wt, y = D.make_inputs(29, torch.bfloat16, n=200)
    lt = hts.float() @ Wt.float().t()  # float32, not representable in bf16
    lt16 = lt.to(torch.bfloat16)
    for w_s, kl_w in ((0.0, 1.0), (0.7, 0.5)):
        hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
        out = o.distillation_loss(hs_d, W_d, y.cuda(), o.PrecomputedTeacher(logits=lt.cuda()), student_ce_weight=w_s,
                                  kl_weight=kl_w, kl_temperature=T, backend="triton", divergence=div,
                                  profile=profile)
        out.loss.backward()
        torch.cuda.synchronize()
        kw = dict(student_ce_weight=w_s, kl_weight=kl_w, kl_temperature=T, divergence=div)
        exact = distillation_loss_oracle("precomputed", _np(hs), _np(W), y.numpy(), teacher_logits=_np(lt), **kw)
        for key in ("loss", "kl"):
            got = float(getattr(out, key).detach())
            assert abs(got - exact[key]) <= 1e-3 * abs(exact[key]) + 1e-5, (key, got, exact[key])
        ref = distillation_loss_oracle("precomputed", _np(hs), _np(W), y.numpy(), teacher_logits=_np(lt16), **kw)
        _check_scalars(out, ref, div)
        _check_grad(hs_d.grad, ref["grad_student_hidden"], torch.bfloat16, f"{div} grad_student_hidden", div)
        _check_grad(W_d.grad, ref["grad_weight"], torch.bfloat16, f"{div} grad_weight", div)


@pytest.mark.parametrize("logits_dtype", [torch.bfloat16, torch.float32], ids=["bf16_logits", "f32_logits"])
@pytest.mark.parametrize("profile", ["balanced", "debug"], ids=["grads_in_forward", "two_phase"])
def test_teacher_logits_cast_to_an_f16_student(logits_dtype, profile):
    """An fp16 student with bf16 or fp32 teacher logits: the logits are
    rounded to fp16 (the compute dtype), as the reference's per-chunk cast
    does, on the element path of the cast-transpose (bf16 into fp16) and its
    16-byte path (fp32 into fp16)."""
    o = _orda()
    hs, W, _, hts, Wt, y = D.make_inputs(37, torch.float16, n=300, v=1032)
    lt = (hts.float() @ Wt.float().t()).to(logits_dtype)
    lt16 = lt.to(torch.float16)
    hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
    out = o.distillation_loss(hs_d, W_d, y.cuda(), o.PrecomputedTeacher(logits=lt.cuda()), student_ce_weight=0.5,
                              kl_weight=1.0, kl_temperature=2.0, backend="triton", divergence="forward_kl",
                              profile=profile)
    out.loss.backward()
    torch.cuda.synchronize()
    ref = distillation_loss_oracle("precomputed", _np(hs), _np(W), y.numpy(), teacher_logits=_np(lt16),
                                   student_ce_weight=0.5, kl_weight=1.0, kl_temperature=2.0, divergence="forward_kl")
    _check_scalars(out, ref, f"{logits_dtype} {profile}")
    _check_grad(hs_d.grad, ref["grad_student_hidden"], torch.float16, "grad_student_hidden")
    _check_grad(W_d.grad, ref["grad_weight"], torch.float16, "grad_weight")


DIVS = [
    "forward_kl", "reverse_kl", "symmetric_kl", "soft_target_ce", "hellinger", "bhattacharyya", "renyi",
    "amari_alpha", "chi_squared", "squared_l2", "ab", "jsd", "skew_forward_kl", "skew_reverse_kl", "tvd",
]


@pytest.mark.parametrize("profile, V", [("balanced", 1032), ("balanced", 1028), ("balanced", 1030), ("debug", 1032)],
                         ids=["in_place", "staged_ring", "staged_transposed", "two_phase"])
@pytest.mark.parametrize("T", [1.0, 4.0])
@pytest.mark.parametrize("div", DIVS)
def test_masked_teacher_vocabulary(div, T, profile, V):
    """Precomputed teacher log-probs with 30% of each row masked to a finite
    -1e4 (how a teacher that rules tokens out stores them in a 16-bit
    tensor): those entries carry no teacher mass (their exponentials
    underflow to 0 inside the kernels' sums), every divergence stays finite
    and matches the oracle on the same bf16 values; divergence term isolated
    (no student CE).  V picks how the teacher's logits reach the passes
    after the scan: read in place (V % 8 == 0), copied into the chunk buffer
    by the scan that reads them token-major (V % 4 == 0), or transposed into
    the chunk buffer ahead of the scan."""
    o = _orda()
    hs, W, _, hts, Wt, y = D.make_inputs(43, torch.bfloat16, n=200, v=V)
    lt = torch.log_softmax(hts.float() @ Wt.float().t(), dim=-1)
    mask = torch.rand(lt.shape, generator=torch.Generator().manual_seed(7)) < 0.3
    lt16 = lt.masked_fill(mask, -1e4).to(torch.bfloat16)
    hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
    out = o.distillation_loss(hs_d, W_d, y.cuda(), o.PrecomputedTeacher(logits=lt16.cuda()), student_ce_weight=0.0,
                              kl_weight=1.0, kl_temperature=T, backend="triton", divergence=div, profile=profile)
    out.loss.backward()
    torch.cuda.synchronize()
    ref = distillation_loss_oracle("precomputed", _np(hs), _np(W), y.numpy(), teacher_logits=_np(lt16),
                                   student_ce_weight=0.0, kl_weight=1.0, kl_temperature=T, divergence=div)
    assert np.isfinite(ref["loss"])
    _check_scalars(out, ref, f"{div} T={T}")
    _check_grad(hs_d.grad, ref["grad_student_hidden"], torch.bfloat16, f"{div} grad_student_hidden", div)
    _check_grad(W_d.grad, ref["grad_weight"], torch.bfloat16, f"{div} grad_weight", div)


@pytest.mark.parametrize("ac_dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("mode", ["tied", "separate", "precomputed-logits"])
def test_autocast_sets_the_compute_dtype(mode, ac_dtype):
    o = _orda()
    hs32, W32, ht32, hts32, Wt32, y = D.make_inputs(31, torch.float32)
    rounded = lambda x: x.to(ac_dtype).float()  # noqa: E731  (the values the kernels see)
    hs_d, W_d = hs32.cuda().requires_grad_(True), W32.cuda().requires_grad_(True)
    if mode == "tied":
        teacher, kw, omode = o.TiedTeacher(ht32.cuda()), dict(teacher_hidden=_np(rounded(ht32))), "tied"
    elif mode == "separate":
        teacher = o.SeparateTeacher(hts32.cuda(), Wt32.cuda())
        kw, omode = dict(teacher_hidden=_np(rounded(hts32)), teacher_weight=_np(rounded(Wt32))), "separate"
    else:
        lt = rounded(hts32) @ rounded(Wt32).t()
        lt_in = lt.to(ac_dtype)  # logits in the autocast dtype
        teacher, kw, omode = o.PrecomputedTeacher(logits=lt_in.cuda()), dict(teacher_logits=_np(lt_in)), "precomputed"
    with torch.autocast("cuda", dtype=ac_dtype):
        out = o.distillation_loss(hs_d, W_d, y.cuda(), teacher, student_ce_weight=0.5, teacher_ce_weight=0.0,
                                  kl_weight=1.0, kl_temperature=2.0, backend="triton", divergence="reverse_kl")
    out.loss.backward()
    torch.cuda.synchronize()
    assert out.loss.dtype == torch.float32
    assert hs_d.grad.dtype == torch.float32 and W_d.grad.dtype == torch.float32
    ref = distillation_loss_oracle(omode, _np(rounded(hs32)), _np(rounded(W32)), y.numpy(), student_ce_weight=0.5,
                                   teacher_ce_weight=0.0, kl_weight=1.0, kl_temperature=2.0, divergence="reverse_kl",
                                   teacher_grads=False, grad_logits_dtype=D.grad_logits_dtype(ac_dtype), **kw)
    _check_scalars(out, ref, (mode, str(ac_dtype)))
    _check_grad(hs_d.grad, ref["grad_student_hidden"], ac_dtype, "grad_student_hidden")
    _check_grad(W_d.grad, ref["grad_weight"], ac_dtype, "grad_weight")


@pytest.mark.parametrize("profile", ["balanced", "debug"])
def test_retained_graph_scales_each_backward_once(profile):
    """backward(0.5, retain_graph=True) then backward(2.0): the gradients
    are the oracle's at grad_output 0.5, then accumulate to 2.5; a tensor
    returned by the first backward is not changed by the second.  Also
    autograd.grad followed by backward."""
    o = _orda()
    dtype = torch.bfloat16
    hs, W, ht, _, _, y = D.make_inputs(37, dtype, n=96)
    kw = dict(student_ce_weight=0.6, teacher_ce_weight=0.3, kl_weight=0.8, kl_temperature=2.0)

    def ref(go):
        return distillation_loss_oracle("tied", _np(hs), _np(W), y.numpy(), teacher_hidden=_np(ht), grad_output=go,
                                        grad_logits_dtype="bfloat16" if profile == "balanced" else None, **kw)

    hs_d, W_d, ht_d = (x.cuda().requires_grad_(True) for x in (hs, W, ht))
    out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TiedTeacher(ht_d), backend="triton", profile=profile, **kw)
    out.loss.backward(torch.tensor(0.5, device="cuda"), retain_graph=True)
    first = [t.grad.clone() for t in (hs_d, W_d, ht_d)]
    held = hs_d.grad  # the tensor autograd stored as .grad
    held_copy = held.clone()
    r = ref(0.5)
    for got, key in zip(first, ("grad_student_hidden", "grad_weight", "grad_teacher_hidden")):
        _check_grad(got, r[key], dtype, f"first backward {key}")
    out.loss.backward(torch.tensor(2.0, device="cuda"))
    torch.cuda.synchronize()
    r = ref(2.5)
    for t, key in zip((hs_d, W_d, ht_d), ("grad_student_hidden", "grad_weight", "grad_teacher_hidden")):
        _check_grad(t.grad, r[key], dtype, f"accumulated {key}")
    if hs_d.grad is not held:  # accumulation made a new tensor: the old one must be untouched
        assert torch.equal(held, held_copy)

    hs_d, W_d, ht_d = (x.cuda().requires_grad_(True) for x in (hs, W, ht))
    out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TiedTeacher(ht_d), backend="triton", profile=profile, **kw)
    g_hs, g_w = torch.autograd.grad(out.loss * 0.5, [hs_d, W_d], retain_graph=True)
    g_hs_copy = g_hs.clone()
    r = ref(0.5)
    _check_grad(g_hs, r["grad_student_hidden"], dtype, "autograd.grad grad_student_hidden")
    _check_grad(g_w, r["grad_weight"], dtype, "autograd.grad grad_weight")
    (out.loss * 2.0).backward()
    torch.cuda.synchronize()
    r = ref(2.0)
    _check_grad(hs_d.grad, r["grad_student_hidden"], dtype, "backward after autograd.grad grad_student_hidden")
    _check_grad(W_d.grad, r["grad_weight"], dtype, "backward after autograd.grad grad_weight")
    assert torch.equal(g_hs, g_hs_copy)
