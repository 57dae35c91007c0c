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


def test_compiled_op_retries_a_device_oom_with_halved_chunks(monkeypatch):
    """The op's OOM retry (the dispatcher's, reference
    ``utils/dispatcher.py:244-293``): a device out-of-memory error doubles
    the chunk count (halves the token chunk) and calls again, up to
    ``2 * max(1, BT // 512)`` chunks, then re-raises; any other error, or an
    explicit chunk size, is raised at once.  The library call is replaced on
    the host (no kernel runs)."""
    from orda_ce_kernel.ops import _engine

    BT, H, V = 2048, 16, 64
    hs, W = torch.randn(BT, H, dtype=torch.bfloat16), torch.randn(V, H, dtype=torch.bfloat16)
    y = torch.randint(0, V, (BT,))
    chunks = []

    def fake_run(fail_times, exc):
        def run(call):
            chunks.append(call.token_chunk)
            if len(chunks) <= fail_times:
                raise exc
            outs = tuple(torch.zeros((), dtype=torch.float32) for _ in range(4))
            return outs, (torch.zeros(BT, H, dtype=torch.bfloat16), None, None, None, None), None
        return run

    def op(chunk_size=0):
        return compiled.fused_loss(hs, W, y, None, None, None, None, None, None, "tied", 1.0, 0.0, 0.0, 1.0,
                                   -100, "mean", "forward_kl", float("nan"), float("nan"),
                                   [True, False, False, False, False], chunk_size, 1e-6, False, "")

    oom = torch.cuda.OutOfMemoryError("HIP out of memory. Tried to allocate 2.00 GiB")
    monkeypatch.setattr(_engine, "run_fused_call", fake_run(2, oom))
    res = op()
    assert len(res) == 10 and res[4].shape == (BT, H)
    assert len(chunks) == 3 and chunks[1] * 2 == chunks[0] and chunks[2] * 2 == chunks[1]
    # the limit: 2 * (2048 // 512) = 8 chunks, then the error goes to the caller
    chunks.clear()
    monkeypatch.setattr(_engine, "run_fused_call", fake_run(100, oom))
    with pytest.raises(torch.cuda.OutOfMemoryError):
        op()
    assert chunks[-1] * 8 >= BT and len(chunks) <= 4
    # not an OOM, or an explicit chunk size: no retry
    for exc, cs in ((RuntimeError("invalid argument"), 0), (oom, 256)):
        chunks.clear()
        monkeypatch.setattr(_engine, "run_fused_call", fake_run(1, exc))
        with pytest.raises(type(exc)):
            op(cs)
        assert len(chunks) == 1


def test_compiled_op_returns_dense_gradients_like_its_fake(monkeypatch):
    """H = 100 (not a multiple of the kernels' 16 bytes): the library hands
    back gradients with padded rows (pitch 104); the op cuts them to dense
    (N, 100) tensors, whose shape and strides equal the fake's, so compiled
    code that relies on the fake's layout reads them correctly.  The library
    call is replaced on the host (no kernel runs)."""
    from orda_ce_kernel.ops import _engine

    BT, H, Hp, V = 64, 100, 104, 50

    def run(call):
        outs = tuple(torch.zeros((), dtype=torch.float32) for _ in range(4))
        g = torch.arange(BT * Hp, dtype=torch.float32).reshape(BT, Hp).to(torch.bfloat16)
        gw = torch.ones(V, Hp, dtype=torch.bfloat16)
        return outs, (g, gw, None, None, None), None

    monkeypatch.setattr(_engine, "run_fused_call", run)
    args = lambda dev: (torch.randn(BT, H, dtype=torch.bfloat16, device=dev),  # noqa: E731
                        torch.randn(V, H, dtype=torch.bfloat16, device=dev),
                        torch.randint(0, V, (BT,), device=dev), None, None, None, None, None, None, "tied", 1.0, 0.0,
                        0.0, 1.0, -100, "mean", "forward_kl", float("nan"), float("nan"),
                        [True, True, False, False, False], 0, 1e-6, False, "")
    real = compiled.fused_loss(*args("cpu"))
    fake = compiled.fused_loss(*args("meta"))
    for i in (4, 5):
        assert real[i].shape == fake[i].shape and real[i].stride() == fake[i].stride(), i
        assert real[i].is_contiguous()
    assert real[4].shape == (BT, H) and real[5].shape == (V, H)
    assert torch.equal(real[4].float(), torch.arange(BT * Hp, dtype=torch.float32).reshape(BT, Hp)[:, :H]
                       .to(torch.bfloat16).float())
