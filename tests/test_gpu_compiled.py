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
