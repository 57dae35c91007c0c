"""Public API contract (CPU): the reference's test/unit/test_public_api.py
cases, restated for this package, plus the additions (divergence keyword,
``hip`` backend alias, fail-loud behaviour)."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import orda_ce_kernel
from orda_ce_kernel import api as public_api


def _cpu_inputs():
    hs = torch.randn(4, 8, requires_grad=True)
    ht = torch.randn(4, 8, requires_grad=True)
    w = torch.randn(16, 8, requires_grad=True)
    y = torch.randint(0, 16, (4,))
    return hs, ht, w, y


def test_availability_flag_is_boolean():
    assert isinstance(orda_ce_kernel.is_available(), bool)


def test_exports_are_the_reference_surface():
    expected = {
        "DistillationLoss", "DistillationLossOutput", "KernelConfig", "PrecomputedTeacher", "SeparateTeacher",
        "TiedTeacher", "distillation_loss", "is_available",
    }
    assert set(orda_ce_kernel.__all__) == expected
    for name in expected:
        assert hasattr(orda_ce_kernel, name)


def test_mode_entry_points_exist():
    from orda_ce_kernel import ops
    from orda_ce_kernel.ops.precomputed_teacher import PrecomputedCEFunction
    from orda_ce_kernel.ops.separate_teacher import SeparateFullCEFunction, SeparateStudentCEFunction
    from orda_ce_kernel.ops.tied_teacher import TiedCEFunction

    assert set(ops.__all__) == {"precomputed_distillation_loss", "separate_distillation_loss", "tied_distillation_loss"}
    for fn in (TiedCEFunction, SeparateStudentCEFunction, SeparateFullCEFunction, PrecomputedCEFunction):
        assert issubclass(fn, torch.autograd.Function)


def test_tied_torch_backend_returns_named_output_and_backprops():
    hs, ht, w, y = _cpu_inputs()
    out = orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.TiedTeacher(ht), kl_weight=0.2,
                                           kl_temperature=1.5, backend="torch")
    assert isinstance(out, orda_ce_kernel.DistillationLossOutput)
    loss, s, t, k = out
    assert loss is out.loss and s is out.student_ce and t is out.teacher_ce and k is out.kl
    out.loss.backward()
    assert hs.grad is not None and ht.grad is not None and w.grad is not None


def test_auto_backend_on_cpu_equals_torch_backend():
    hs, ht, w, y = _cpu_inputs()
    teacher = orda_ce_kernel.TiedTeacher(ht)
    a = orda_ce_kernel.distillation_loss(hs, w, y, teacher, kl_weight=0.2, kl_temperature=1.5)
    b = orda_ce_kernel.distillation_loss(hs, w, y, teacher, kl_weight=0.2, kl_temperature=1.5, backend="torch")
    for x, z in zip(a, b):
        assert torch.allclose(x, z)


def test_separate_teacher_ce_defaults_to_zero():
    hs = torch.randn(3, 4, requires_grad=True)
    ht = torch.randn(3, 6, requires_grad=True)
    w = torch.randn(11, 4, requires_grad=True)
    wt = torch.randn(11, 6, requires_grad=True)
    y = torch.randint(0, 11, (3,))
    out = orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.SeparateTeacher(ht, wt), kl_weight=0.3,
                                           backend="torch")
    out.loss.backward()
    assert torch.equal(out.teacher_ce, torch.zeros_like(out.teacher_ce))
    assert wt.grad is None


def test_precomputed_hidden_weight_cache_in_torch_backend():
    hs = torch.randn(5, 4, requires_grad=True)
    w = torch.randn(13, 4, requires_grad=True)
    teacher = orda_ce_kernel.PrecomputedTeacher(teacher_hidden=torch.randn(5, 6), teacher_weight=torch.randn(13, 6))
    out = orda_ce_kernel.distillation_loss(hs, w, torch.randint(0, 13, (5,)), teacher, kl_weight=0.25,
                                           kl_temperature=1.7, backend="torch")
    out.loss.backward()
    assert torch.isfinite(out.loss)
    assert torch.equal(out.teacher_ce, torch.zeros_like(out.teacher_ce))
    assert hs.grad is not None and w.grad is not None


def test_precomputed_descriptor_rejections():
    logits = torch.randn(4, 16)
    th, tw = torch.randn(4, 8), torch.randn(16, 8)
    with pytest.raises(ValueError, match="logits or"):
        orda_ce_kernel.PrecomputedTeacher(logits=logits, teacher_hidden=th, teacher_weight=tw)
    with pytest.raises(ValueError, match="must provide"):
        orda_ce_kernel.PrecomputedTeacher()
    with pytest.raises(ValueError, match="both be provided"):
        orda_ce_kernel.PrecomputedTeacher(teacher_hidden=th)
    hs, _, w, y = _cpu_inputs()
    bad = torch.randn(4, 16, requires_grad=True)
    with pytest.raises(ValueError, match="must not require gradients"):
        orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.PrecomputedTeacher(logits=bad), backend="torch")
    with pytest.raises(ValueError, match="must not require gradients"):
        orda_ce_kernel.distillation_loss(
            hs, w, y, orda_ce_kernel.PrecomputedTeacher(teacher_hidden=th.requires_grad_(True), teacher_weight=tw),
            backend="torch")


def test_profiles_and_config_validation():
    assert public_api._resolve_profile("debug").fp32_grad_weight_accumulation is True
    assert public_api._resolve_profile("balanced").fp32_grad_weight_accumulation is False
    merged = public_api._resolve_config("debug", orda_ce_kernel.KernelConfig(chunk_size=7))
    assert merged.fp32_grad_weight_accumulation is True and merged.chunk_size == 7
    override = public_api._resolve_config(
        "debug", orda_ce_kernel.KernelConfig(fp32_grad_weight_accumulation=False, chunk_size=7))
    assert override.fp32_grad_weight_accumulation is False
    with pytest.raises(ValueError, match="profile"):
        public_api._resolve_profile("fast")
    hs, ht, w, y = _cpu_inputs()
    t = orda_ce_kernel.TiedTeacher(ht)
    K = orda_ce_kernel.KernelConfig
    with pytest.raises(ValueError, match="max_chunks"):
        orda_ce_kernel.distillation_loss(hs, w, y, t, config=K(max_chunks=0))
    with pytest.raises(ValueError, match="num_chunks"):
        orda_ce_kernel.distillation_loss(hs, w, y, t, config=K(num_chunks=0))
    with pytest.raises(ValueError, match="mutually exclusive"):
        orda_ce_kernel.distillation_loss(hs, w, y, t, config=K(chunk_size=2, num_chunks=2))
    with pytest.raises(ValueError, match="power of two"):
        orda_ce_kernel.distillation_loss(hs, w, y, t, config=K(max_fused_size=100))
    with pytest.raises(ValueError, match="num_chunks must be <= config.max_chunks"):
        orda_ce_kernel.distillation_loss(hs, w, y, t, config=K(num_chunks=3, max_chunks=2))


@pytest.mark.parametrize(
    "kwargs, match",
    [
        (dict(student_ce_weight=-1.0), "student_ce_weight"),
        (dict(teacher_ce_weight=-0.5), "teacher_ce_weight"),
        (dict(kl_weight=-0.1), "kl_weight"),
        (dict(kl_temperature=0.0), "kl_temperature"),
        (dict(reduction="none"), "reduction"),
        (dict(backend="cuda"), "backend"),
        (dict(divergence="wasserstein"), "divergence"),
        (dict(divergence="jsd", kl_weight=1.0, backend="torch"), None),
    ],
)
def test_argument_validation_messages(kwargs, match):
    hs, ht, w, y = _cpu_inputs()
    t = orda_ce_kernel.TiedTeacher(ht)
    if match is None:
        orda_ce_kernel.distillation_loss(hs, w, y, t, **kwargs)
        return
    with pytest.raises(ValueError, match=match):
        orda_ce_kernel.distillation_loss(hs, w, y, t, **kwargs)


def test_shape_validation_messages():
    hs, ht, w, y = _cpu_inputs()
    with pytest.raises(ValueError, match="student_hidden must be 2D"):
        orda_ce_kernel.distillation_loss(hs[0], w, y, orda_ce_kernel.TiedTeacher(ht))
    with pytest.raises(ValueError, match="weight must have shape"):
        orda_ce_kernel.distillation_loss(hs, w[:, :3], y, orda_ce_kernel.TiedTeacher(ht))
    with pytest.raises(ValueError, match="labels must have shape"):
        orda_ce_kernel.distillation_loss(hs, w, y[:2], orda_ce_kernel.TiedTeacher(ht))
    with pytest.raises(ValueError, match="TiedTeacher.hidden must have shape"):
        orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.TiedTeacher(ht[:, :3]))
    with pytest.raises(ValueError, match="SeparateTeacher.weight must have shape"):
        orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.SeparateTeacher(ht, torch.randn(15, 8)))
    with pytest.raises(TypeError, match="teacher must be"):
        orda_ce_kernel.distillation_loss(hs, w, y, object())


def test_bool_labels_are_rejected_before_dispatch():
    hs, ht, w, _ = _cpu_inputs()
    with pytest.raises(ValueError, match="integer class-index|torch.long"):
        orda_ce_kernel.distillation_loss(hs, w, torch.tensor([True, False, True, False]),
                                         orda_ce_kernel.TiedTeacher(ht), backend="torch")


def _manual_tied(hs, ht, w, y, *, kl_weight, kl_temperature, reduction):
    ls, lt = hs @ w.t(), ht @ w.t()
    mask = y != -100
    denom = max(int(mask.sum()), 1)
    ce_s = F.cross_entropy(ls, y, ignore_index=-100, reduction="none")
    ce_t = F.cross_entropy(lt, y, ignore_index=-100, reduction="none")
    T = float(kl_temperature)
    kl = F.kl_div(F.log_softmax(ls / T, -1), F.softmax(lt.detach() / T, -1), reduction="none").sum(-1) * T * T
    kl = kl.masked_fill(~mask, 0.0)
    if reduction == "mean":
        s, t, k = ce_s.sum() / denom, ce_t.sum() / denom, kl.sum() / denom
    else:
        s, t, k = ce_s.sum(), ce_t.sum(), kl.sum()
    return s + t + kl_weight * k, s, t, k


@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_torch_backend_reduction_contract(reduction):
    hs, ht, w, y = _cpu_inputs()
    y = y.clone()
    y[1] = -100
    out = orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.TiedTeacher(ht), kl_weight=0.35,
                                           kl_temperature=1.7, reduction=reduction, backend="torch")
    ref = _manual_tied(hs, ht, w, y, kl_weight=0.35, kl_temperature=1.7, reduction=reduction)
    for a, b in zip(out, ref):
        assert torch.allclose(a, b)


def test_components_are_detached_and_loss_backprops():
    hs, ht, w, y = _cpu_inputs()
    out = orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.TiedTeacher(ht), kl_weight=0.25, backend="torch")
    assert out.loss.requires_grad
    assert not out.student_ce.requires_grad and not out.teacher_ce.requires_grad and not out.kl.requires_grad
    out.loss.backward()
    assert hs.grad is not None


@pytest.mark.parametrize("backend", ["triton", "hip"])
def test_kernel_backend_fails_fast_on_cpu(backend):
    hs, ht, w, y = _cpu_inputs()
    with pytest.raises(RuntimeError, match=f"backend='{backend}'"):
        orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.TiedTeacher(ht), backend=backend)


def test_triton_backend_rejects_precomputed_teacher_ce():
    hs, _, w, y = _cpu_inputs()
    with pytest.raises(ValueError, match="requires teacher_ce_weight=0.0"):
        orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.PrecomputedTeacher(logits=torch.randn(4, 16)),
                                         teacher_ce_weight=0.5, backend="triton")


def test_mode_entry_points_need_hip_tensors():
    from orda_ce_kernel.ops import tied_distillation_loss

    hs, ht, w, y = _cpu_inputs()
    with pytest.raises((RuntimeError, ValueError), match="CUDA/HIP|HIP extension"):
        tied_distillation_loss(hs, ht, w, y)


def test_module_equals_functional():
    hs, ht, w, y = _cpu_inputs()
    t = orda_ce_kernel.TiedTeacher(ht)
    m = orda_ce_kernel.DistillationLoss(kl_weight=0.25, kl_temperature=1.3, backend="torch", divergence="jsd")
    a = m(hs, w, y, t)
    b = orda_ce_kernel.distillation_loss(hs, w, y, t, kl_weight=0.25, kl_temperature=1.3, backend="torch",
                                         divergence="jsd")
    for x, z in zip(a, b):
        assert torch.allclose(x, z)


def test_divergence_objects_and_defaults():
    from orda_ce_kernel.divergences import DIVERGENCES, Divergence, resolve_divergence

    assert len(DIVERGENCES) == 15
    assert resolve_divergence(None) == Divergence("forward_kl")
    assert resolve_divergence("jsd").beta == 0.5
    assert resolve_divergence(Divergence("skew_forward_kl")).alpha == 0.1
    for bad in (Divergence("renyi", alpha=1.0), Divergence("jsd", beta=1.0), Divergence("ab", alpha=0.5, beta=-0.5),
                Divergence("skew_reverse_kl", alpha=1.0), Divergence("amari_alpha", alpha=0.0)):
        with pytest.raises(ValueError):
            resolve_divergence(bad)


def test_kernel_config_autotune_is_accepted():
    hs, ht, w, y = _cpu_inputs()
    out = orda_ce_kernel.distillation_loss(hs, w, y, orda_ce_kernel.TiedTeacher(ht), backend="torch",
                                           config=orda_ce_kernel.KernelConfig(autotune=True))
    assert torch.isfinite(out.loss)
