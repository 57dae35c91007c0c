"""CPU: the torch.compile-friendly entry (``orda_ce_kernel.compiled``) traces
in one graph (``fullgraph=True``) for every teacher mode, through forward and
backward, on meta tensors (the op's fake implementation gives the shapes; no
kernel runs).  The GPU results are checked in ``test_gpu_compiled.py``."""
from __future__ import annotations

import pytest
import torch

from orda_ce_kernel import PrecomputedTeacher, SeparateTeacher, TiedTeacher, compiled


def _meta(*shape, dtype=torch.bfloat16, grad=False):
    return torch.empty(*shape, dtype=dtype, device="meta", requires_grad=grad)


@pytest.mark.parametrize("mode", ["tied", "separate", "separate_full", "precomputed_logits", "precomputed_hidden"])
def test_compiled_entry_traces_without_graph_breaks(mode):
    torch._dynamo.reset()
    N, H, Ht, V = 48, 32, 24, 100
    hs, W = _meta(N, H, grad=True), _meta(V, H, grad=True)
    y = torch.empty(N, dtype=torch.long, device="meta")
    w_t = None
    if mode == "tied":
        ht = _meta(N, H, grad=True)
        make = lambda: TiedTeacher(ht)  # noqa: E731
        expect = {"ht": (N, H)}
    elif mode.startswith("separate"):
        full = mode == "separate_full"
        ht, Wt = _meta(N, Ht, grad=full), _meta(V, Ht, grad=full)
        w_t = 1.0 if full else None
        make = lambda: SeparateTeacher(ht, Wt)  # noqa: E731
        expect = {"ht": (N, Ht), "Wt": (V, Ht)} if full else {}
    elif mode == "precomputed_logits":
        lt = _meta(N, V)
        make = lambda: PrecomputedTeacher(logits=lt)  # noqa: E731
        expect = {}
    else:
        ht, Wt = _meta(N, Ht), _meta(V, Ht)
        make = lambda: PrecomputedTeacher(teacher_hidden=ht, teacher_weight=Wt)  # noqa: E731
        expect = {}

    def step(hs, W, y):
        out = compiled.distillation_loss(hs, W, y, make(), kl_weight=0.5, kl_temperature=2.0, teacher_ce_weight=w_t,
                                         divergence="jsd")
        return out.loss * 2.0

    loss = torch.compile(step, fullgraph=True, backend="aot_eager")(hs, W, y)
    assert loss.shape == () and loss.dtype == torch.float32
    loss.backward()
    assert hs.grad.shape == (N, H) and W.grad.shape == (V, H)
    if "ht" in expect:
        assert ht.grad.shape == expect["ht"]
    if "Wt" in expect:
        assert Wt.grad.shape == expect["Wt"]


def test_compiled_entry_validates_like_the_drop_in():
    hs, W = _meta(8, 16), _meta(50, 16)
    y = torch.empty(8, dtype=torch.long, device="meta")
    with pytest.raises(ValueError, match="kl_temperature"):
        compiled.distillation_loss(hs, W, y, TiedTeacher(_meta(8, 16)), kl_temperature=0.0)
    with pytest.raises(ValueError, match="TiedTeacher.hidden must have shape"):
        compiled.distillation_loss(hs, W, y, TiedTeacher(_meta(7, 16)))
    with pytest.raises(ValueError, match="teacher_ce_weight"):
        compiled.distillation_loss(hs, W, y, PrecomputedTeacher(logits=_meta(8, 50)), teacher_ce_weight=1.0)


@pytest.mark.parametrize("ext", ["topk", "norm", "fp8", "norm_topk"])
def test_compiled_entry_traces_the_extensions(ext):
    """The top-k teacher, the fused RMSNorm (its weight gets a gradient) and
    the fp8 logits GEMM trace in one graph too."""
    from orda_ce_kernel import StudentRMSNorm, TopKTeacher

    torch._dynamo.reset()
    N, H, V, k = 48, 256, 100, 8
    hs, W = _meta(N, H, grad=True), _meta(V, H, grad=True)
    y = torch.empty(N, dtype=torch.long, device="meta")
    nw = _meta(H, grad=True)
    if "topk" in ext:
        idx = torch.empty(N, k, dtype=torch.long, device="meta")
        lp = torch.empty(N, k, dtype=torch.float32, device="meta")
        make = lambda: TopKTeacher(idx, lp)  # noqa: E731
    else:
        ht = _meta(N, H, grad=True)
        make = lambda: TiedTeacher(ht)  # noqa: E731
    kw = {}
    if "norm" in ext:
        kw["student_norm"] = StudentRMSNorm(nw, eps=1e-5)
    if ext == "fp8":
        kw["logits_gemm"] = "fp8"

    def step(hs, W, y):
        return compiled.distillation_loss(hs, W, y, make(), kl_weight=0.5, kl_temperature=2.0, **kw).loss

    loss = torch.compile(step, fullgraph=True, backend="aot_eager")(hs, W, y)
    loss.backward()
    assert hs.grad.shape == (N, H) and W.grad.shape == (V, H)
    if "norm" in ext:
        assert nw.grad.shape == (H,)
    else:
        assert nw.grad is None
