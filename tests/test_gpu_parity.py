"""GPU parity: the HIP path (through the C ABI) against the float64 oracle.

Inputs are generated on the CPU with a seeded generator, rounded to the
compute dtype, and the oracle sees exactly those rounded values.  Tolerances
loss components within 1e-3 relative (plus a small
absolute floor for values near 0); gradients within atol/rtol 1e-2 of the
float64 oracle for 16-bit inputs, 1e-4 for float32 inputs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.orda_oracle import distillation_loss_oracle

pytestmark = pytest.mark.gpu

DIVS = [
    "forward_kl", "reverse_kl", "symmetric_kl", "soft_target_ce", "hellinger", "bhattacharyya", "renyi",
    "amari_alpha", "chi_squared", "squared_l2", "ab", "jsd", "skew_forward_kl", "skew_reverse_kl", "tvd",
]


def _orda():
    import orda_ce_kernel

    assert orda_ce_kernel.is_available(), "liborda_ce.so must load on a HIP device"
    return orda_ce_kernel


def _make(seed, N, H, V, dtype, *, Ht=None, ignore_frac=0.05, h_std=1.0, w_std=0.02, t_noise=None):
    g = torch.Generator().manual_seed(seed)
    hs = torch.randn(N, H, generator=g) * h_std
    if t_noise is not None:
        ht = hs + t_noise * torch.randn(N, H, generator=g)
    else:
        ht = torch.randn(N, Ht or H, generator=g) * h_std
    W = torch.randn(V, H, generator=g) * w_std
    Wt = torch.randn(V, Ht or H, generator=g) * w_std
    y = torch.randint(0, V, (N,), generator=g)
    n_ign = int(round(ignore_frac * N))
    if n_ign:
        y[torch.randperm(N, generator=g)[:n_ign]] = -100
    cast = lambda x: x.to(dtype)  # noqa: E731
    return cast(hs), cast(ht), cast(W), cast(Wt), y


def _np(x):
    return x.detach().double().cpu().numpy()


def _close_scalar(actual, expected, name, rtol=1e-3, atol=1e-5):
    a = float(actual)
    assert np.isfinite(a), f"{name} is not finite: {a}"
    assert abs(a - expected) <= atol + rtol * abs(expected), f"{name}: got {a:.9g}, expected {expected:.9g}"


def _close_grad(actual, expected, name, tol):
    """atol/rtol ``tol`` and, since these gradients
    are far smaller than 1e-2, bounds relative to their own scale: worst
    |err| <= c * max|ref| and ||err|| <= c * ||ref||, c = 2e-2 for 16-bit
    inputs (tol 1e-2) and 2e-4 for float32 (tol 1e-4)."""
    a = actual.detach().double().cpu().numpy()
    assert np.all(np.isfinite(a)), f"{name} has non-finite values"
    err = np.abs(a - expected)
    bound = tol + tol * np.abs(expected)
    worst = float((err - bound).max())
    assert worst <= 0, f"{name}: max |err| {err.max():.3e} exceeds atol/rtol {tol:g}"
    c = 2.0 * tol
    scale = float(np.abs(expected).max())
    if scale > 0:
        assert err.max() <= c * scale, f"{name}: max |err| {err.max():.3e} > {c:g} * max|ref| {scale:.3e}"
        rel = float(np.linalg.norm(a - expected) / np.linalg.norm(expected))
        assert rel <= c, f"{name}: relative Frobenius error {rel:.3e} > {c:g}"
    else:
        assert err.max() == 0.0, f"{name}: expected exact zeros, max |err| {err.max():.3e}"


def _grad_tol(dtype):
    return 1e-4 if dtype == torch.float32 else 1e-2


def _run(mode, dtype, *, N=96, H=64, V=1000, Ht=None, seed=0, reduction="mean", w_s=1.0, w_t=None, kl_w=0.5,
         T=1.0, div="forward_kl", config=None, ignore_frac=0.05, grad_teacher=True, grad_output=1.0,
         profile="balanced", w_std=0.02):
    o = _orda()
    hs, ht, W, Wt, y = _make(seed, N, H, V, dtype, Ht=Ht, ignore_frac=ignore_frac, w_std=w_std)
    dev = "cuda"
    hs_d = hs.to(dev).requires_grad_(True)
    W_d = W.to(dev).requires_grad_(True)
    y_d = y.to(dev)
    kw = {}
    if mode == "tied":
        ht_d = ht.to(dev).requires_grad_(grad_teacher)
        teacher = o.TiedTeacher(ht_d)
        kw = dict(teacher_hidden=_np(ht))
    elif mode == "separate":
        ht_d = ht.to(dev).requires_grad_(grad_teacher)
        Wt_d = Wt.to(dev).requires_grad_(grad_teacher)
        teacher = o.SeparateTeacher(ht_d, Wt_d)
        kw = dict(teacher_hidden=_np(ht), teacher_weight=_np(Wt))
    elif mode == "precomputed_logits":
        lt = (ht.float() @ Wt.float().t()).to(dtype)
        teacher = o.PrecomputedTeacher(logits=lt.to(dev))
        kw = dict(teacher_logits=_np(lt))
    else:
        teacher = o.PrecomputedTeacher(teacher_hidden=ht.to(dev), teacher_weight=Wt.to(dev))
        kw = dict(teacher_hidden=_np(ht), teacher_weight=_np(Wt))
    out = o.distillation_loss(
        hs_d, W_d, y_d, teacher, student_ce_weight=w_s, teacher_ce_weight=w_t, kl_weight=kl_w,
        kl_temperature=T, reduction=reduction, backend="triton", config=config, divergence=div, profile=profile,
    )
    (out.loss * grad_output).backward()
    omode = "precomputed" if mode.startswith("precomputed") else mode
    ref = distillation_loss_oracle(
        omode, _np(hs), _np(W), y.numpy(), student_ce_weight=w_s, teacher_ce_weight=w_t, kl_weight=kl_w,
        kl_temperature=T, reduction=reduction, divergence=div, grad_output=grad_output,
        teacher_grads=(w_t or 0.0) > 0 or mode == "tied", **kw,
    )
    torch.cuda.synchronize()
    return out, ref, hs_d, W_d, teacher


def _check(out, ref, hs_d, W_d, dtype, rtol=1e-3):
    for name in ("loss", "student_ce", "teacher_ce", "kl"):
        _close_scalar(getattr(out, name), ref[name], name, rtol=rtol)
    tol = _grad_tol(dtype)
    _close_grad(hs_d.grad, ref["grad_student_hidden"], "grad_student_hidden", tol)
    _close_grad(W_d.grad, ref["grad_weight"], "grad_weight", tol)


DTYPES = [torch.bfloat16, torch.float16, torch.float32]


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_tied_matches_oracle(dtype, reduction):
    out, ref, hs, W, teacher = _run("tied", dtype, reduction=reduction, T=1.7, kl_w=0.35, w_s=0.8, w_t=0.25)
    _check(out, ref, hs, W, dtype)
    _close_grad(teacher.hidden.grad, ref["grad_teacher_hidden"], "grad_teacher_hidden", _grad_tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("full", [False, True], ids=["student", "full"])
def test_separate_matches_oracle(dtype, full):
    out, ref, hs, W, teacher = _run("separate", dtype, Ht=96, T=2.0, w_t=1.0 if full else None, grad_teacher=full)
    _check(out, ref, hs, W, dtype)
    if full:
        tol = _grad_tol(dtype)
        _close_grad(teacher.hidden.grad, ref["grad_teacher_hidden"], "grad_teacher_hidden", tol)
        _close_grad(teacher.weight.grad, ref["grad_teacher_weight"], "grad_teacher_weight", tol)
    else:
        assert teacher.hidden.grad is None and teacher.weight.grad is None


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("source", ["precomputed_logits", "precomputed_hidden"])
def test_precomputed_matches_oracle(dtype, source):
    out, ref, hs, W, _ = _run(source, dtype, Ht=48, T=4.0)
    _check(out, ref, hs, W, dtype)


@pytest.mark.parametrize("div", DIVS)
@pytest.mark.parametrize("T", [1.0, 2.0])
def test_every_divergence_matches_oracle_fp32(div, T):
    out, ref, hs, W, _ = _run("tied", torch.float32, div=div, T=T, kl_w=0.7, N=64, V=700, H=32)
    _check(out, ref, hs, W, torch.float32)


@pytest.mark.parametrize("div", DIVS)
def test_every_divergence_matches_oracle_bf16_precomputed(div):
    out, ref, hs, W, _ = _run("precomputed_logits", torch.bfloat16, div=div, T=4.0, kl_w=1.0, N=64, V=700, H=64)
    _check(out, ref, hs, W, torch.bfloat16)


def test_config1_cpu_plumbing_shape_on_gpu():
    """fp32, N=512, H=256, V=4096, tied, T=2, alpha 0.5."""
    for w_t in (None, 0.0):
        out, ref, hs, W, teacher = _run("tied", torch.float32, N=512, H=256, V=4096, T=2.0, w_s=0.5, kl_w=0.5,
                                        w_t=w_t, seed=1001)
        _check(out, ref, hs, W, torch.float32)


def test_multi_chunk_backward_accumulates():
    from orda_ce_kernel import KernelConfig

    for cfg in (KernelConfig(num_chunks=4), KernelConfig(chunk_size=7)):
        out, ref, hs, W, teacher = _run("tied", torch.bfloat16, V=1500, N=64, config=cfg, T=1.3)
        _check(out, ref, hs, W, torch.bfloat16)
        _close_grad(teacher.hidden.grad, ref["grad_teacher_hidden"], "grad_teacher_hidden", 1e-2)


def test_ragged_shapes_and_padding():
    # N not a multiple of 8, H not a multiple of 8 (host pads), V tiny and ragged
    for N, H, V in ((9, 36, 17), (130, 40, 257), (1, 8, 5)):
        out, ref, hs, W, _ = _run("tied", torch.bfloat16, N=N, H=H, V=V, T=1.4, ignore_frac=0.0)
        _check(out, ref, hs, W, torch.bfloat16)


@pytest.mark.parametrize("profile", ["balanced", "debug"])
@pytest.mark.parametrize("div", ["reverse_kl", "jsd", "hellinger"])
@pytest.mark.parametrize("mode", ["separate", "precomputed_logits", "precomputed_hidden"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_ragged_shapes_every_teacher_mode(dtype, mode, div, profile):
    """The ragged shapes above for the teachers that are not tied: a single
    token, vocabularies below one tile and not a multiple of 4 (teacher
    logits staged by transposition), hidden sizes the host pads, teacher
    hidden sizes that differ from the student's; a one-pass, a two-pass and a
    power-family divergence; both schedules."""
    for N, H, Ht, V in ((9, 36, 44, 17), (130, 40, 24, 257), (1, 8, 16, 5)):
        out, ref, hs, W, _ = _run(mode, dtype, N=N, H=H, Ht=Ht, V=V, T=1.4, div=div, kl_w=1.0, ignore_frac=0.0,
                                  profile=profile)
        _check(out, ref, hs, W, dtype)


def test_grad_output_scaling():
    out, ref, hs, W, _ = _run("tied", torch.bfloat16, grad_output=3.5, reduction="sum")
    _check(out, ref, hs, W, torch.bfloat16)


def test_all_ignored_gives_exact_zeros():
    o = _orda()
    hs, ht, W, _, _ = _make(7, 16, 32, 300, torch.bfloat16)
    hs, ht, W = (x.cuda().requires_grad_(True) for x in (hs, ht, W))
    y = torch.full((16,), -100, dtype=torch.long, device="cuda")
    out = o.distillation_loss(hs, W, y, o.TiedTeacher(ht), kl_weight=0.5, kl_temperature=1.7, backend="triton")
    out.loss.backward()
    for t in out:
        assert torch.equal(t, torch.zeros_like(t))
    for t in (hs.grad, ht.grad, W.grad):
        assert torch.count_nonzero(t) == 0


def test_kl_weight_zero_reports_exact_zero_kl():
    out, ref, hs, W, _ = _run("separate", torch.float16, kl_w=0.0, Ht=48)
    assert float(out.kl) == 0.0
    _check(out, ref, hs, W, torch.float16)


def test_teacher_ce_zero_keeps_teacher_grad_zero():
    out, ref, hs, W, teacher = _run("tied", torch.float16, w_t=0.0, T=1.4)
    assert torch.count_nonzero(teacher.hidden.grad) == 0
    assert float(out.teacher_ce) == 0.0


def test_out_of_range_label_counts_as_class_zero():
    """Reference kernel quirk (ops/tied_teacher.py:42-44): without label
    validation an out-of-range label is treated as class 0."""
    o = _orda()
    hs, ht, W, _, y = _make(3, 24, 32, 300, torch.float32, ignore_frac=0.0)
    y[5] = 1000
    hs_d, ht_d, W_d = (x.cuda().requires_grad_(True) for x in (hs, ht, W))
    out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TiedTeacher(ht_d), kl_weight=0.3, backend="triton")
    out.loss.backward()
    ref = distillation_loss_oracle("tied", _np(hs), _np(W), y.numpy(), teacher_hidden=_np(ht), kl_weight=0.3)
    _check(out, ref, hs_d, W_d, torch.float32)


def test_loss_is_bit_stable_across_runs():
    o = _orda()
    hs, ht, W, _, y = _make(11, 200, 128, 3000, torch.bfloat16)
    args = (hs.cuda(), W.cuda(), y.cuda(), o.TiedTeacher(ht.cuda()))
    a = o.distillation_loss(*args, kl_weight=1.0, backend="triton")
    b = o.distillation_loss(*args, kl_weight=1.0, backend="triton")
    for x, z in zip(a, b):
        assert torch.equal(x, z)


def test_identical_teacher_gives_zero_divergence():
    o = _orda()
    hs, _, W, _, y = _make(5, 64, 64, 900, torch.float32)
    for div in DIVS:
        if div == "soft_target_ce":  # cross-entropy: equals T^2 H(p_t) at p_s = p_t, not 0
            continue
        out = o.distillation_loss(hs.cuda(), W.cuda(), y.cuda(), o.TiedTeacher(hs.cuda()), kl_weight=1.0,
                                  kl_temperature=1.3, backend="triton", divergence=div)
        assert abs(float(out.kl)) < 2e-5, (div, float(out.kl))


def test_gemm_engine_matches_torch():
    from orda_ce_kernel import _native

    g = torch.Generator().manual_seed(0)
    for dtype in DTYPES:
        for M, N, K in ((300, 270, 64), (256, 256, 512), (17, 513, 72), (1, 1, 8)):
            a = torch.randn(M, K, generator=g).to(dtype)
            b = torch.randn(N, K, generator=g).to(dtype)
            c = _native.gemm_abt(a.cuda(), b.cuda()).float().cpu()
            ref = a.double() @ b.double().t()
            tol = 1e-4 if dtype == torch.float32 else 2e-2
            err = (c.double() - ref).abs().max().item()
            assert err <= tol * max(1.0, ref.abs().max().item()), (dtype, M, N, K, err)


@pytest.mark.parametrize("profile", ["balanced", "debug"])
@pytest.mark.parametrize("mode", ["tied", "separate"])
def test_fp16_dlogits_keep_the_softmax_term(profile, mode):
    """fp16 with 1024 tokens and a 40000-word vocabulary: a dlogit times the
    mean scale, p / count ~ 2.5e-5 / 973, lies below half of fp16's smallest
    subnormal.  The library stores the dlogits unscaled and scales the
    gradients once (the reference's fp16 path does the same), so the hidden
    gradients keep their softmax terms.  Against a build that scaled the
    fp16 dlogits in the chunk, the default schedule failed here (teacher
    hidden gradient off by 2.3-3.8% of its largest entry against the 2%
    bound); grad_output 2.5 checks that the scales compose, in both
    schedules."""
    out, ref, hs, W, teacher = _run(mode, torch.float16, N=1024, H=64, V=40000, Ht=48 if mode == "separate" else None,
                                    T=1.0, kl_w=0.5, w_t=1.0, grad_output=2.5, profile=profile, w_std=0.1)
    _check(out, ref, hs, W, torch.float16)
    tol = _grad_tol(torch.float16)
    _close_grad(teacher.hidden.grad, ref["grad_teacher_hidden"], "grad_teacher_hidden", tol)
    if mode == "separate":
        _close_grad(teacher.weight.grad, ref["grad_teacher_weight"], "grad_teacher_weight", tol)


# ------------------------------------------------------------------ schedules
# profile="balanced" (default): gradients inside forward over token chunks
# with materialised logits (tied / separate, one-pass divergences);
# profile="debug" (fp32 grad-W accumulation): scan forward + recomputing
# backward.  Both against the oracle, and against each other.

@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("mode", ["tied", "separate"])
def test_two_phase_schedule_matches_oracle(dtype, mode):
    out, ref, hs, W, teacher = _run(mode, dtype, Ht=96 if mode == "separate" else None, T=1.6, kl_w=0.4, w_t=0.3,
                                    profile="debug")
    _check(out, ref, hs, W, dtype)
    tol = _grad_tol(dtype)
    _close_grad(teacher.hidden.grad, ref["grad_teacher_hidden"], "grad_teacher_hidden", tol)
    if mode == "separate":
        _close_grad(teacher.weight.grad, ref["grad_teacher_weight"], "grad_teacher_weight", tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("mode", ["tied", "separate"])
def test_grads_in_forward_over_ragged_token_chunks(dtype, mode):
    """chunk_size=20 -> 40-token chunks over N=96: 40 + 40 + 16, the last one
    ragged (zeroed padding columns), grad W accumulated across chunks."""
    from orda_ce_kernel import KernelConfig

    for div in ("forward_kl", "reverse_kl", "hellinger", "squared_l2", "jsd", "skew_forward_kl", "skew_reverse_kl",
                "tvd"):
        out, ref, hs, W, teacher = _run(mode, dtype, Ht=72 if mode == "separate" else None, T=1.3, kl_w=0.6,
                                        w_t=0.5, div=div, config=KernelConfig(chunk_size=20))
        _check(out, ref, hs, W, dtype)
        tol = _grad_tol(dtype)
        _close_grad(teacher.hidden.grad, ref["grad_teacher_hidden"], "grad_teacher_hidden", tol)
        if mode == "separate":
            _close_grad(teacher.weight.grad, ref["grad_teacher_weight"], "grad_teacher_weight", tol)


@pytest.mark.parametrize("div, T", [("forward_kl", 1.0), ("jsd", 2.0), ("skew_reverse_kl", 1.0)])
def test_schedules_agree_on_a_larger_problem(div, T):
    """N=600 tokens, V=5000, H=256 (several vocabulary tiles, split-K grad
    hidden, 3 token chunks): balanced vs debug gradients, for a one-pass
    divergence and two two-pass ones (second pass over the stored logits vs
    over recomputed ones)."""
    from orda_ce_kernel import KernelConfig

    res = {}
    for profile, cfg in (("balanced", KernelConfig(chunk_size=128)), ("debug", None)):
        out, ref, hs, W, teacher = _run("tied", torch.bfloat16, N=600, H=256, V=5000, T=T, kl_w=1.0, w_t=1.0,
                                        config=cfg, profile=profile, seed=3, div=div)
        _check(out, ref, hs, W, torch.bfloat16)
        res[profile] = (hs.grad.float(), W.grad.float(), teacher.hidden.grad.float())
    for a, b in zip(res["balanced"], res["debug"]):
        scale = b.abs().max().item()
        assert (a - b).abs().max().item() <= 2e-2 * scale


def test_persistent_workgroups_over_many_tiles():
    """V = 80000 (313 vocabulary tiles): the scan's workgroups each run three
    vocabulary tiles back to back and the grad-W GEMM has more tiles than the
    GPU has CUs, so workgroups move from tile to tile mid-pipeline."""
    from orda_ce_kernel import KernelConfig

    out, ref, hs, W, teacher = _run("tied", torch.bfloat16, N=512, H=256, V=80000, T=1.0, kl_w=1.0, w_t=1.0,
                                    config=KernelConfig(chunk_size=128), profile="balanced", seed=5)
    _check(out, ref, hs, W, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("mode", ["separate", "precomputed_logits", "precomputed_hidden"])
def test_staged_teacher_logits_feed_the_student_scan(dtype, mode):
    """Separate and precomputed teachers with 16-bit operands and H > 64: the
    chunk's teacher logits are written into the logits buffer first (teacher
    GEMM or transpose) and the scan runs the student GEMM alone, 256 tokens
    per workgroup.  N=600 in 256-token chunks (256 + 256 + 88: a ragged last
    tile), V=5000 (ragged last vocabulary tile); the power family (hellinger)
    keeps the two-operand scan.  Precomputed logits are read token-major by
    the scan when V is a multiple of 4 (V=5000) and transposed into the
    buffer first otherwise (V=4998)."""
    from orda_ce_kernel import KernelConfig

    grad_teacher = mode == "separate"
    cases = [("forward_kl", 1.0, 5000), ("forward_kl", 2.0, 5000), ("reverse_kl", 1.0, 5000),
             ("squared_l2", 2.0, 5000), ("hellinger", 1.0, 5000), ("jsd", 2.0, 5000), ("skew_reverse_kl", 1.0, 5000)]
    if mode == "precomputed_logits":
        cases += [("forward_kl", 1.0, 4998), ("reverse_kl", 2.0, 4998), ("skew_forward_kl", 2.0, 4998)]
    for div, T, V in cases:
        out, ref, hs, W, teacher = _run(mode, dtype, N=600, H=128, Ht=192, V=V, T=T, kl_w=0.8,
                                        w_t=0.4 if grad_teacher else None, div=div, grad_teacher=grad_teacher,
                                        config=KernelConfig(chunk_size=128), seed=21)
        _check(out, ref, hs, W, dtype)
        if grad_teacher:
            tol = _grad_tol(dtype)
            _close_grad(teacher.hidden.grad, ref["grad_teacher_hidden"], "grad_teacher_hidden", tol)
            _close_grad(teacher.weight.grad, ref["grad_teacher_weight"], "grad_teacher_weight", tol)


def test_grads_in_forward_are_bit_stable():
    o = _orda()
    hs, ht, W, _, y = _make(12, 300, 128, 2000, torch.bfloat16)
    grads = []
    for _ in range(2):
        hs_d, ht_d, W_d = (x.cuda().requires_grad_(True) for x in (hs, ht, W))
        out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TiedTeacher(ht_d), kl_weight=1.0, backend="triton",
                                  config=o.KernelConfig(chunk_size=64))
        out.loss.backward()
        grads.append((out.loss.detach(), hs_d.grad, W_d.grad, ht_d.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


# --------------------------------------------------------- general GEMM
def _gemm_case(dtype, a_mn, b_mn, M, N, K, splits=1, seed=0):
    from orda_ce_kernel import _native

    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g).to(dtype)
    b = torch.randn(N, K, generator=g).to(dtype)
    a_in = a.t().contiguous() if a_mn else a
    b_in = b.t().contiguous() if b_mn else b
    c = _native.gemm(a_in.cuda(), b_in.cuda(), a_mn=a_mn, b_mn=b_mn, splits=splits).float().cpu()
    ref = a.double() @ b.double().t()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    err = (c.double() - ref).abs().max().item()
    assert err <= tol * max(1.0, ref.abs().max().item()), (dtype, a_mn, b_mn, M, N, K, splits, err)


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("a_mn, b_mn", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_general_gemm_layouts_match_torch(dtype, a_mn, b_mn):
    for M, N, K in ((264, 272, 520), (8, 264, 64), (256, 256, 200), (520, 16, 1000)):
        _gemm_case(dtype, a_mn, b_mn, M, N, K)


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f16", "f32"])
def test_general_gemm_split_k_matches_torch(dtype):
    for M, N, K, splits in ((264, 272, 5000, 4), (40, 512, 3000, 7), (256, 256, 128, 3)):
        _gemm_case(dtype, 1, 1, M, N, K, splits=splits)


@pytest.mark.parametrize("dtype", DTYPES[:2], ids=["bf16", "f16"])
def test_general_gemm_persistent_many_tiles(dtype):
    """More output tiles (or split work items) than CUs, ragged edges: each
    workgroup of the persistent GEMM runs several tiles in one pipeline."""
    from orda_ce_kernel import _native

    g = torch.Generator().manual_seed(7)
    for a_mn, b_mn, M, N, K, splits in ((0, 0, 4104, 4104, 264, 1), (0, 1, 4104, 4104, 264, 1),
                                        (1, 1, 4104, 4104, 200, 1), (1, 1, 1040, 2056, 9000, 6)):
        a = torch.randn(M, K, generator=g).to(dtype).cuda()
        b = torch.randn(N, K, generator=g).to(dtype).cuda()
        a_in = a.t().contiguous() if a_mn else a
        b_in = b.t().contiguous() if b_mn else b
        c = _native.gemm(a_in, b_in, a_mn=a_mn, b_mn=b_mn, splits=splits).float()
        ref = a.float() @ b.float().t()
        err = (c - ref).abs().max().item()
        assert err <= 2e-2 * max(1.0, ref.abs().max().item()), (a_mn, b_mn, M, N, K, splits, err)


def test_peaked_rows_dlogits_sum_to_zero_within_rounding():
    """Softmax dlogits of a row sum to zero (shift invariance), so with a
    constant column in W the gradient along that column vanishes.  Peaked
    teacher rows with logits up to ~33 (bf16 ulp 0.25) stress the normaliser
    the dlogits pass uses: it must describe the logits as stored (rounded to
    bf16), not the fp32 values the statistics came from.  Emulation of this
    case: with fp32 normalisers the column reaches ~12% of the largest
    gradient entry; with the max-element correction ~4.4% (the rest is the
    rounding of the other logits)."""
    o = _orda()
    g = torch.Generator().manual_seed(21)
    N, H, V = 128, 64, 4000
    W = torch.randn(V, H, generator=g) / H ** 0.5
    W[:, 0] = 1.0
    ht = torch.randn(N, H, generator=g) * 6.4
    hs = torch.randn(N, H, generator=g) * 3.0
    y = torch.randint(0, V, (N,), generator=g)
    hs_d, ht_d, W_d = (x.bfloat16().cuda().requires_grad_(True) for x in (hs, ht, W))
    out = o.distillation_loss(hs_d, W_d, y.cuda(), o.TiedTeacher(ht_d), kl_weight=1.0, backend="triton")
    out.loss.backward()
    torch.cuda.synchronize()
    for name, gr in (("grad_teacher_hidden", ht_d.grad), ("grad_student_hidden", hs_d.grad)):
        gr = gr.float()
        ratio = float(gr[:, 0].abs().max() / gr[:, 1:].abs().max())
        print(f"{name}: max |column 0| / max |other columns| = {ratio:.4f}")
        assert ratio < 0.08, (name, ratio)


@pytest.mark.parametrize("V", [2000, 1998], ids=["in_place", "staged"])
def test_precomputed_logits_read_in_place_partial_quads(V):
    """Precomputed logits of the compute dtype with V a multiple of 8 are read
    in place, token-major, by the scan, the two-pass divergences' second pass
    and the dlogits pass (no copy into the chunk buffer; chunks of twice the
    tokens); V = 1998 takes the staged path.
    N = 203 in 128-token chunks (128 + 75): the last token quad is partial."""
    from orda_ce_kernel import KernelConfig

    for div, T in (("forward_kl", 1.0), ("reverse_kl", 2.0), ("hellinger", 1.0), ("jsd", 2.0), ("skew_forward_kl", 1.0),
                   ("tvd", 1.0)):
        out, ref, hs, W, _ = _run("precomputed_logits", torch.bfloat16, N=203, H=128, Ht=96, V=V, T=T, kl_w=0.9,
                                  div=div, config=KernelConfig(chunk_size=32), seed=31, grad_teacher=False)
        _check(out, ref, hs, W, torch.bfloat16)


def test_precomputed_logits_misaligned_view_matches_aligned():
    """A contiguous logits tensor that starts 2 bytes past a 16-byte boundary
    (a view into a larger buffer) gives the same result as an aligned copy."""
    o = _orda()
    hs, ht, W, Wt, y = _make(41, 96, 128, 1000, torch.bfloat16, Ht=64)
    lt = (ht.float() @ Wt.float().t()).bfloat16()
    buf = torch.empty(lt.numel() + 8, dtype=torch.bfloat16, device="cuda")
    lt_mis = buf[1:1 + lt.numel()].view(lt.shape)
    lt_mis.copy_(lt.cuda())
    assert lt_mis.data_ptr() % 16 != 0
    res = []
    for src in (lt.cuda(), lt_mis):
        hs_d, W_d = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
        out = o.distillation_loss(hs_d, W_d, y.cuda(), o.PrecomputedTeacher(logits=src), kl_weight=1.0,
                                  backend="triton")
        out.loss.backward()
        res.append((out.loss.detach(), hs_d.grad, W_d.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)
