"""GPU parity at the benchmark configurations' full sizes (configs 2-5).

The HIP path runs one forward + backward through the public API; a plain
PyTorch float32 reference of the same loss (``tests/_fp32_reference.py``,
itself pinned against the float64 oracle in ``tests/test_fp32_reference.py``)
runs on the same device-resident inputs, chunked over tokens.

Tolerances: loss components within 1e-3 relative;
gradients elementwise within atol/rtol 1e-2 of the float32 reference (atol
in units of the largest gradient where that exceeds 1: chi-squared at T = 1
against config 4's peaked teacher has a loss of ~8600 and gradients of
~30, whose bf16-logit rounding, 0.4% of the largest, exceeds an absolute
1e-2), and,
because these gradients are far smaller than 1e-2, also with the worst
elementwise error at most 2e-2 of the reference's largest magnitude and a
relative Frobenius error at most 2e-2 (grad W is accumulated in bf16 over
the token chunks, as in the reference's default profile: ~0.3% observed);
config 5's peaked teacher rows widen the elementwise bound (see its test).
Peak extra device memory is checked against the 2 GB target at config 2 and,
at every size, the peak beyond the gradients against the size of one [N x V]
logits tensor (none may exist).
"""
from __future__ import annotations

import math

import pytest
import torch

from tests._fp32_reference import DIVERGENCES, fp32_reference

pytestmark = pytest.mark.gpu


def _orda():
    import orda_ce_kernel

    assert orda_ce_kernel.is_available(), "liborda_ce.so must load on a HIP device"
    return orda_ce_kernel


def _inputs(seed, mode, N, H, V, *, Ht=None, ignore_frac=0.05, teacher_row_scale=None, dtype=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    bf = dtype
    hs = torch.randn(N, H, generator=g, device="cuda").to(bf)
    W = (0.02 * torch.randn(V, H, generator=g, device="cuda")).to(bf)
    ht = Wt = lt = None
    if mode == "tied":
        ht = torch.randn(N, H, generator=g, device="cuda")
        if teacher_row_scale is not None:
            ht *= teacher_row_scale(g, N)[:, None]
        ht = ht.to(bf)
    elif mode == "separate":
        ht = torch.randn(N, Ht, generator=g, device="cuda").to(bf)
        Wt = (0.02 * torch.randn(V, Ht, generator=g, device="cuda")).to(bf)
    else:
        lt = torch.empty(N, V, dtype=bf, device="cuda")
        for s in range(0, N, 1024):
            e = min(N, s + 1024)
            lt[s:e] = torch.log_softmax(3.0 * torch.randn(e - s, V, generator=g, device="cuda"), -1).to(bf)
    y = torch.randint(0, V, (N,), generator=g, device="cuda")
    n_ign = int(round(ignore_frac * N))
    y[torch.randperm(N, generator=g, device="cuda")[:n_ign]] = -100
    return hs, W, y, ht, Wt, lt


def _teacher(o, mode, ht, Wt, lt):
    if mode == "tied":
        return o.TiedTeacher(ht)
    if mode == "separate":
        return o.SeparateTeacher(ht, Wt)
    return o.PrecomputedTeacher(logits=lt)


def _grad_close(name, got, ref, max_frac=2e-2, frob_frac=2e-2):
    out_dtype = got.dtype
    got = got.float()
    err = (got - ref).abs()
    ref_max = float(ref.abs().max())
    ref_norm = float(torch.linalg.vector_norm(ref))
    # atol 1e-2 in units of the gradient's scale where that exceeds 1
    # (chi-squared at T = 1 against a peaked teacher: gradients ~30)
    ns_excess = float((err - (1e-2 * max(1.0, ref_max) + 1e-2 * ref.abs())).max())
    worst = float(err.max())
    frob = float(torch.linalg.vector_norm(got - ref)) / ref_norm
    # fp16 outputs: gradients of ~1e-6 are fp16 subnormals (a grid of
    # 2^-24), so the scale-relative bounds also allow twice the error of
    # rounding the exact gradient itself to fp16
    rep_max = rep_frob = 0.0
    if out_dtype == torch.float16:
        rep = ref.half().float() - ref
        rep_max = float(rep.abs().max())
        rep_frob = float(torch.linalg.vector_norm(rep)) / ref_norm
    print(f"{name}: max|ref| {ref_max:.3e} max|err| {worst:.3e} rel-frobenius {frob:.2e}"
          + (f" (fp16 rounding of the exact gradient: max {rep_max:.3e}, rel-frobenius {rep_frob:.2e})"
             if out_dtype == torch.float16 else ""), flush=True)
    assert torch.isfinite(got).all(), f"{name} has non-finite values"
    assert ns_excess <= 0, f"{name}: outside atol/rtol 1e-2"
    assert worst <= max_frac * ref_max + 2 * rep_max, \
        f"{name}: max |err| {worst:.3e} > {max_frac:g} x max|ref| {ref_max:.3e} (+ 2 x {rep_max:.3e})"
    assert frob <= frob_frac + 2 * rep_frob, f"{name}: relative Frobenius error {frob:.3e}"


def _run_fullsize(seed, mode, N, H, V, *, Ht=None, div="forward_kl", T=1.0, w_s=1.0, w_t=None, kl_w=1.0,
                  ignore_frac=0.05, teacher_row_scale=None, profile="balanced", peak_limit=None, max_frac=2e-2,
                  frob_frac=2e-2, dtype=torch.bfloat16, chunk=None):
    o = _orda()
    print(f"case: {mode} N={N} H={H} Ht={Ht} V={V} div={div} T={T} profile={profile} dtype={dtype} chunk={chunk}",
          flush=True)
    hs, W, y, ht, Wt, lt = _inputs(seed, mode, N, H, V, Ht=Ht, ignore_frac=ignore_frac,
                                   teacher_row_scale=teacher_row_scale, dtype=dtype)
    hs_d = hs.detach().requires_grad_(True)
    W_d = W.detach().requires_grad_(True)
    teacher = _teacher(o, mode, ht, Wt, lt)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = o.distillation_loss(hs_d, W_d, y, teacher, student_ce_weight=w_s, teacher_ce_weight=w_t, kl_weight=kl_w,
                              kl_temperature=T, backend="triton", divergence=div, profile=profile,
                              config=o.KernelConfig(chunk_size=chunk) if chunk else None)
    out.loss.backward()
    torch.cuda.synchronize()
    peak_extra = torch.cuda.max_memory_allocated() - base
    got = {k: float(getattr(out, k)) for k in ("loss", "student_ce", "teacher_ce", "kl")}
    del out
    grad_bytes = sum(g.numel() * g.element_size() for g in (hs_d.grad, W_d.grad))
    print(f"peak extra {peak_extra / 1e9:.3f} GB (gradients {grad_bytes / 1e9:.3f} GB); one [N x V] 16-bit tensor "
          f"is {N * V * 2 / 1e9:.2f} GB", flush=True)
    assert peak_extra - grad_bytes < N * V * 2, "working memory reaches the size of a full logits tensor"
    if peak_limit is not None:
        assert peak_extra < peak_limit, f"peak extra {peak_extra / 1e9:.3f} GB >= {peak_limit / 1e9:.1f} GB"
    ref = fp32_reference(mode, hs, W, y, ht=ht, Wt=Wt, lt=lt, student_ce_weight=w_s, teacher_ce_weight=w_t,
                         kl_weight=kl_w, kl_temperature=T, divergence=div)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        print(f"{k}: hip {got[k]:.7g} fp32-ref {ref[k]:.7g}", flush=True)
        assert math.isfinite(got[k]), k
        assert abs(got[k] - ref[k]) <= 1e-3 * abs(ref[k]) + 1e-5, (k, got[k], ref[k])
    _grad_close("grad_student_hidden", hs_d.grad, ref["grad_student_hidden"], max_frac, frob_frac)
    _grad_close("grad_weight", W_d.grad, ref["grad_weight"], max_frac, frob_frac)
    return ref


@pytest.mark.parametrize("profile", ["balanced", "debug"])
def test_config2_tied_forward_kl_fullsize(profile):
    """Config 2 (headline): tied, N=8192, H=4096, V=128256, forward KL, T=1.
    ``balanced`` runs gradients inside forward; ``debug`` the two-phase
    schedule with fp32 grad-W accumulation."""
    _run_fullsize(1002, "tied", 8192, 4096, 128256, peak_limit=2e9 if profile == "balanced" else None,
                  profile=profile)


def test_config2_tied_ragged_chunks_fullsize():
    """Config 2 with a requested chunk of 640 tokens: 1280-token chunks (10
    token tiles, which do not divide the 256 scan workgroups: the plan takes
    25 vocabulary ranges, not 26) and a last chunk of 512."""
    _run_fullsize(1002, "tied", 8192, 4096, 128256, peak_limit=2e9, chunk=640)


@pytest.mark.parametrize("div", ["squared_l2", "ab"])
def test_config2_tied_three_term_power_divergences_fullsize(div):
    """Config 2's shape with squared L2 and AB (alpha = beta = 0.5), which
    run as two-pass divergences: their second pass reads the chunk's stored
    16-bit logits."""
    _run_fullsize(1002, "tied", 8192, 4096, 128256, div=div, T=1.0, peak_limit=2e9)


@pytest.mark.parametrize("div", ["reverse_kl", "jsd", "squared_l2"])
def test_config3_separate_teacher_fullsize(div):
    """Config 3: student hidden 2048, teacher hidden 4096 (frozen), T=2."""
    _run_fullsize(1003, "separate", 8192, 2048, 128256, Ht=4096, div=div, T=2.0)


@pytest.mark.parametrize("T", [1.0, 4.0])
@pytest.mark.parametrize("div", DIVERGENCES)
def test_config4_precomputed_teacher_fullsize(div, T):
    """Config 4's sweep: bf16 teacher log-probs of N(0, 3) logits,
    [8192 x 128256], every divergence at T = 1 and 4 (default parameters:
    skew alpha 0.1, JSD beta 0.5).  TVD's gradient is a sign function of
    p_s - p_t, so where the two are within rounding of each other the kernels
    and the reference may take opposite sides: its gradients are held to
    the scale-relative bounds the small-shape TVD tests use (worst element
    0.5 and Frobenius 0.1 of the reference's scale; atol/rtol 1e-2 still
    apply)."""
    tvd = div == "tvd"
    _run_fullsize(1004, "precomputed", 8192, 4096, 128256, div=div, T=T, max_frac=0.5 if tvd else 2e-2,
                  frob_frac=0.1 if tvd else 2e-2)


def test_config5_long_sequence_stress_fullsize():
    """Config 5: N=32768, H=5120, V=152064, tied, alpha 0.7, 20% ignored.
    Each teacher row is scaled by c / tau_n with tau_n ~ U[0.5, 4]; c makes
    the teacher logit spread run from ~0.8 to ~6.4 standard deviations, so
    teacher entropies go from near-uniform to near one-hot (checked).
    Two things widen the worst elementwise error here, so it is held to
    5e-2 of the largest gradient (observed: 0.9% for grad hidden, 1.8% for
    grad W): the dlogits read the logits rounded to bf16 (as the reference's
    own bf16 logits are), and in the most peaked rows logits of |x| ~ 30
    carry rounding errors up to 0.06; grad W is rounded to bf16 after each
    of 32 token chunks (8 at configs 2-4)."""
    c = 6.4 * 0.5 / (0.02 * math.sqrt(5120))

    def row_scale(g, n):
        tau = 0.5 + 3.5 * torch.rand(n, generator=g, device="cuda")
        return c / tau

    ref = _run_fullsize(1005, "tied", 32768, 5120, 152064, w_s=0.7, kl_w=0.3, ignore_frac=0.20,
                        teacher_row_scale=row_scale, max_frac=5e-2)
    ent_min, ent_max = ref["teacher_entropy"]
    print(f"teacher entropy range: {ent_min:.3f} .. {ent_max:.3f} nats (log V = {math.log(152064):.3f})")
    assert ent_min < 3.0 and ent_max > math.log(152064) - 0.5


def _row_scale_c5(g, n):
    c = 6.4 * 0.5 / (0.02 * math.sqrt(5120))
    return c / (0.5 + 3.5 * torch.rand(n, generator=g, device="cuda"))


@pytest.mark.parametrize("cfg", ["c2f16", "c3f16", "c4f16", "c5f16", "h8192", "h3584"])
def test_launch_table_shapes_fullsize(cfg):
    """The launch table's further rows at their full sizes: configs 2-5 with
    fp16 inputs, and the tied headline workload at hidden 8192 / vocabulary
    128256 and hidden 3584 / vocabulary 152064 (bf16), against the same
    float32 reference.  In fp16 the dlogits are stored without the 1 / count
    mean scale (probability / count, ~1e-9 here, is below fp16's subnormals)
    and the gradients are scaled once at the end, as the reference's fp16
    path does; before that, grad hidden at config 2 in fp16 was off by 4% of
    its largest entry.  Config 5's peaked teacher rows keep its 5e-2
    elementwise bound (see its test)."""
    f16 = torch.float16
    # (fp16 gradients are also allowed twice the error of rounding the exact
    # gradient to fp16: config 5's grad hidden, ~3e-6, is all subnormals)
    if cfg == "c2f16":
        _run_fullsize(1102, "tied", 8192, 4096, 128256, peak_limit=2e9, dtype=f16)
    elif cfg == "c3f16":
        _run_fullsize(1103, "separate", 8192, 2048, 128256, Ht=4096, div="reverse_kl", T=2.0, dtype=f16)
    elif cfg == "c4f16":
        _run_fullsize(1104, "precomputed", 8192, 4096, 128256, div="forward_kl", T=1.0, dtype=f16)
    elif cfg == "c5f16":
        _run_fullsize(1105, "tied", 32768, 5120, 152064, w_s=0.7, kl_w=0.3, ignore_frac=0.20,
                      teacher_row_scale=_row_scale_c5, max_frac=5e-2, dtype=f16)
    elif cfg == "h8192":
        _run_fullsize(1106, "tied", 8192, 8192, 128256)
    else:
        _run_fullsize(1107, "tied", 8192, 3584, 152064, peak_limit=2e9)
