"""GPU: the torch.compile-friendly entry (custom ops) gives the drop-in's
results under ``torch.compile(fullgraph=True)``: losses bit-identical (the
same kernels and schedule), gradients identical at grad_output 1 and equal
to the drop-in's times grad_output otherwise (applied in the gradient dtype),
for tied, separate (student-only and full) and precomputed teachers."""
from __future__ import annotations

import pytest
import torch

from tests import _divgrad as D

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", ["tied", "separate", "separate_full", "precomputed_logits"])
@pytest.mark.parametrize("go", [1.0, 0.5])
def test_compiled_entry_matches_the_drop_in(mode, go):
    import orda_ce_kernel as o
    from orda_ce_kernel import compiled

    torch._dynamo.reset()
    hs, W, ht, hts, Wt, y = D.make_inputs(41, torch.bfloat16, n=200)
    full = mode == "separate_full"

    def build():
        t = {}
        t["hs"], t["W"] = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True)
        if mode == "tied":
            t["ht"] = ht.cuda().requires_grad_(True)
            teacher = o.TiedTeacher(t["ht"])
        elif mode.startswith("separate"):
            t["ht"], t["Wt"] = hts.cuda().requires_grad_(full), Wt.cuda().requires_grad_(full)
            teacher = o.SeparateTeacher(t["ht"], t["Wt"])
        else:
            teacher = o.PrecomputedTeacher(logits=(hts.float() @ Wt.float().t()).bfloat16().cuda())
        return t, teacher

    kw = dict(kl_weight=0.7, kl_temperature=2.0, divergence="reverse_kl",
              teacher_ce_weight=0.4 if (mode == "tied" or full) else None)
    t_e, teacher_e = build()
    out_e = o.distillation_loss(t_e["hs"], t_e["W"], y.cuda(), teacher_e, backend="triton", **kw)
    (out_e.loss * go).backward()

    t_c, teacher_c = build()
    step = torch.compile(lambda a, b, c, tch: compiled.distillation_loss(a, b, c, tch, **kw), fullgraph=True,
                         backend="aot_eager")
    out_c = step(t_c["hs"], t_c["W"], y.cuda(), teacher_c)
    (out_c.loss * go).backward()
    torch.cuda.synchronize()
    for a, b in zip(out_e, out_c):
        assert torch.equal(a.detach(), b.detach())
    for key in t_e:
        ge, gc = t_e[key].grad, t_c[key].grad
        assert (ge is None) == (gc is None), key
        if ge is None:
            continue
        if go == 1.0:
            assert torch.equal(ge, gc), key
        else:
            assert (ge.float() - gc.float()).abs().max() <= 1e-2 * ge.float().abs().max(), key


@pytest.mark.parametrize("ext", ["topk", "norm", "fp8", "norm_fp8"])
def test_compiled_extensions_match_the_drop_in(ext):
    """The top-k teacher, the fused RMSNorm and the fp8 logits GEMM through
    the custom ops under torch.compile: losses and gradients bit-identical to
    the drop-in's (the same kernels and schedule)."""
    import orda_ce_kernel as o
    from orda_ce_kernel import compiled

    torch._dynamo.reset()
    hs, W, ht, hts, Wt, y = D.make_inputs(43, torch.bfloat16, n=200, h=256)
    g = torch.Generator().manual_seed(7)
    nw = (1.0 + 0.2 * torch.randn(256, generator=g)).bfloat16()
    lp = torch.log_softmax(hts.double() @ Wt.double().t(), dim=1)
    vals, idx = lp.topk(16, dim=1)

    def build():
        t = {"hs": hs.cuda().requires_grad_(True), "W": W.cuda().requires_grad_(True)}
        kw = dict(kl_weight=0.7, kl_temperature=2.0)
        if "topk" in ext:
            teacher = o.TopKTeacher(idx.cuda(), vals.float().cuda())
        else:
            t["ht"] = ht.cuda().requires_grad_(True)
            teacher = o.TiedTeacher(t["ht"])
        if "norm" in ext:
            t["nw"] = nw.cuda().requires_grad_(True)
            kw["student_norm"] = o.StudentRMSNorm(t["nw"], eps=1e-5)
        if "fp8" in ext:
            kw["logits_gemm"] = "fp8"
        return t, teacher, kw

    t_e, teacher_e, kw_e = build()
    out_e = o.distillation_loss(t_e["hs"], t_e["W"], y.cuda(), teacher_e, backend="triton", **kw_e)
    out_e.loss.backward()
    t_c, teacher_c, kw_c = build()
    step = torch.compile(lambda a, b, c, tch: compiled.distillation_loss(a, b, c, tch, **kw_c), fullgraph=True,
                         backend="aot_eager")
    out_c = step(t_c["hs"], t_c["W"], y.cuda(), teacher_c)
    out_c.loss.backward()
    torch.cuda.synchronize()
    for a, b in zip(out_e, out_c):
        assert torch.equal(a.detach(), b.detach())
    for key in t_e:
        assert torch.equal(t_e[key].grad, t_c[key].grad), key


def _drop_in_and_compiled(build, kw, backend, go=1.0, retain=False):
    """Run the drop-in and the compiled entry on fresh copies of the same
    inputs; returns (tensors, outputs) of each."""
    import orda_ce_kernel as o
    from orda_ce_kernel import compiled

    torch._dynamo.reset()
    t_e, teacher_e = build()
    out_e = o.distillation_loss(t_e["hs"], t_e["W"], t_e["y"], teacher_e, backend="triton", **kw)
    (out_e.loss * go).backward(retain_graph=retain)
    t_c, teacher_c = build()
    step = torch.compile(lambda a, b, c, tch: compiled.distillation_loss(a, b, c, tch, **kw), fullgraph=True,
                         backend=backend)
    out_c = step(t_c["hs"], t_c["W"], t_c["y"], teacher_c)
    (out_c.loss * go).backward(retain_graph=retain)
    torch.cuda.synchronize()
    return (t_e, out_e), (t_c, out_c)


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
@pytest.mark.parametrize("case", ["ragged_h", "tied_ce_off", "logits_fp32"])
def test_compiled_entry_edge_cases_match_the_drop_in(case, backend):
    """A hidden size the kernels pad (H = 100: dense gradients come back
    through the custom op), a tied teacher that requires grad with its CE
    off (zeros, as the reference returns), and precomputed teacher logits in
    fp32 with a bf16 student (cast to the compute dtype, as the drop-in
    does): bit-identical to the drop-in, with inductor (the default
    backend) and aot_eager."""
    import orda_ce_kernel as o

    h = 100 if case == "ragged_h" else 128
    hs, W, ht, hts, Wt, y = D.make_inputs(47, torch.bfloat16, n=200, h=h)

    def build():
        t = {"hs": hs.cuda().requires_grad_(True), "W": W.cuda().requires_grad_(True), "y": y.cuda()}
        if case == "logits_fp32":
            teacher = o.PrecomputedTeacher(logits=(hts.float() @ Wt.float().t()).cuda())
        else:
            t["ht"] = ht.cuda().requires_grad_(True)
            teacher = o.TiedTeacher(t["ht"])
        return t, teacher

    kw = dict(kl_weight=0.7, kl_temperature=2.0, divergence="jsd")
    if case == "tied_ce_off":
        kw["teacher_ce_weight"] = 0.0
    (t_e, out_e), (t_c, out_c) = _drop_in_and_compiled(build, kw, backend)
    for a, b in zip(out_e, out_c):
        assert torch.equal(a.detach(), b.detach())
    for key in ("hs", "W", "ht"):
        if key not in t_e:
            continue
        ge, gc = t_e[key].grad, t_c[key].grad
        assert ge is not None and gc is not None, key
        assert gc.shape == ge.shape and gc.is_contiguous(), key
        assert torch.equal(ge, gc), key
    if case == "tied_ce_off":
        assert not torch.any(t_c["ht"].grad)


@pytest.mark.parametrize("backend", ["inductor", "aot_eager", "eager"])
def test_compiled_entry_retained_graph_second_backward(backend):
    """Two backwards through one retained graph, with different grad_output:
    each matches the drop-in's (which recomputes), and the first backward's
    gradients are not changed by the second; compiled (inductor, aot_eager)
    and called eagerly."""
    import orda_ce_kernel as o
    from orda_ce_kernel import compiled

    torch._dynamo.reset()
    hs, W, ht, _, _, y = D.make_inputs(53, torch.bfloat16, n=200)
    kw = dict(kl_weight=0.5, kl_temperature=1.5, divergence="forward_kl")
    res = {}
    for entry in ("drop_in", "compiled"):
        a, b, c = hs.cuda().requires_grad_(True), W.cuda().requires_grad_(True), ht.cuda()
        if entry == "drop_in":
            out = o.distillation_loss(a, b, y.cuda(), o.TiedTeacher(c), backend="triton", **kw)
        else:
            fn = lambda p, q, r, s: compiled.distillation_loss(p, q, r, o.TiedTeacher(s), **kw)  # noqa: E731
            step = fn if backend == "eager" else torch.compile(fn, fullgraph=True, backend=backend)
            out = step(a, b, y.cuda(), c)
        (out.loss * 0.5).backward(retain_graph=True)
        first = (a.grad, b.grad)
        snap = (a.grad.clone(), b.grad.clone())
        a.grad = b.grad = None
        (out.loss * 2.0).backward()
        torch.cuda.synchronize()
        assert torch.equal(first[0], snap[0]) and torch.equal(first[1], snap[1]), entry
        res[entry] = (snap, (a.grad, b.grad))
    for i in range(2):
        ref1, ref2 = res["drop_in"][0][i], res["drop_in"][1][i]
        got1, got2 = res["compiled"][0][i], res["compiled"][1][i]
        assert torch.equal(ref1, got1)
        # the second rescales bf16 gradients by 2.0 / 0.5 (exact powers of
        # two): equal to the drop-in's recomputation
        assert torch.equal(ref2, got2)


def test_compiled_entry_follows_autocast():
    """fp32 inputs under autocast(bfloat16): the compiled entry computes in
    bf16 like the drop-in (reference _runtime.py:41-80), and the gradients
    come back in the inputs' dtype."""
    import orda_ce_kernel as o

    hs, W, ht, _, _, y = D.make_inputs(59, torch.float32, n=200)

    def build():
        t = {"hs": hs.cuda().requires_grad_(True), "W": W.cuda().requires_grad_(True), "y": y.cuda()}
        return t, o.TiedTeacher(ht.cuda())

    kw = dict(kl_weight=0.5, kl_temperature=2.0)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        (t_e, out_e), (t_c, out_c) = _drop_in_and_compiled(build, kw, "aot_eager")
    for a, b in zip(out_e, out_c):
        assert torch.equal(a.detach(), b.detach())
    for key in ("hs", "W"):
        assert t_c[key].grad.dtype == torch.float32
        assert torch.equal(t_e[key].grad, t_c[key].grad), key
