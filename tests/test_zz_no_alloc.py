"""GPU: orda_forward_static (no workspace, no allocation) against
orda_forward with a torch workspace, through the C ABI.

Two calls in a row, the second with a smaller problem (the scratch keeps the
first call's contents), for the gradients-in-forward schedule (losses and
every gradient) and a forward-only call; results must be bit-identical (the
same kernels, fixed reduction orders).  A problem whose workspace exceeds
the static scratch is rejected before anything is launched.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call(mode, N, H, V, *, seed, grads, div="forward_kl", T=1.0, token_chunk=0, Ht=None):
    from orda_ce_kernel import _native
    from orda_ce_kernel.divergences import resolve_divergence
    from orda_ce_kernel.ops._engine import FusedCall, _alloc_grads, _problem

    g = torch.Generator().manual_seed(seed)
    dt = torch.bfloat16
    hs = torch.randn(N, H, generator=g).to(dt).cuda()
    W = (torch.randn(V, H, generator=g) * 0.1).to(dt).cuda()
    y = torch.randint(0, V, (N,), generator=g)
    y[::11] = -100
    y = y.cuda()
    ht = wt = None
    if mode == "tied":
        ht = torch.randn(N, H, generator=g).to(dt).cuda()
    else:
        ht = torch.randn(N, Ht, generator=g).to(dt).cuda()
        wt = (torch.randn(V, Ht, generator=g) * 0.1).to(dt).cuda()
    call = FusedCall(
        mode=mode, student_hidden=hs, weight=W, labels=y, teacher_hidden=ht, teacher_weight=wt, teacher_logits=None,
        student_ce_weight=0.7, teacher_ce_weight=0.4 if mode == "tied" else 0.0, kl_weight=0.9, kl_temperature=T,
        ignore_index=-100, reduction="mean", vocab_chunk=0, divergence=resolve_divergence(div),
        compute_teacher_ce=mode == "tied", need_grad_student_hidden=grads, need_grad_weight=grads,
        need_grad_teacher_hidden=grads and mode == "tied", grads_in_forward=grads, token_chunk=token_chunk,
    )
    problem = _problem(call, H, ht.shape[1], None)
    results = []
    for static in (False, True):
        saved = torch.empty(_native.saved_bytes(problem), dtype=torch.uint8, device="cuda")
        outs = [torch.full((), float("nan"), device="cuda") for _ in range(4)]
        gr = _alloc_grads(problem.flags, hs, W, ht, wt)[:4] if grads else (None,) * 4
        for x in gr:
            if x is not None:
                x.fill_(float("nan"))
        t = _native.Tensors()
        t.student_hidden, t.weight, t.labels = hs.data_ptr(), W.data_ptr(), y.data_ptr()
        t.teacher_hidden = ht.data_ptr()
        t.teacher_weight = wt.data_ptr() if wt is not None else None
        t.out_loss, t.out_student_ce, t.out_teacher_ce, t.out_kl = (o.data_ptr() for o in outs)
        t.saved = saved.data_ptr()
        t.grad_student_hidden, t.grad_weight, t.grad_teacher_hidden, t.grad_teacher_weight = (
            x.data_ptr() if x is not None else None for x in gr)
        print(f"[no_alloc] {mode} N={N} H={H} V={V} grads={grads} div={div} static={static}", flush=True)
        if static:
            _native.forward_static(problem, t, hs.device)
        else:
            ws = torch.empty(_native.forward_workspace_bytes(problem), dtype=torch.uint8, device="cuda")
            _native.forward(problem, t, ws)
        torch.cuda.synchronize()
        results.append([o.clone() for o in outs] + [x.clone() for x in gr if x is not None])
    ref, got = results
    assert all(torch.isfinite(o).all() for o in ref[:4])
    for i, (a, b) in enumerate(zip(ref, got)):
        assert torch.equal(a, b), (mode, N, H, V, grads, div, i)


def test_static_entry_matches_workspace_entry_two_calls():
    # gradients-in-forward, tied, 2 token chunks; then a smaller separate one
    _call("tied", 600, 256, 5000, seed=1, grads=True, div="forward_kl", T=1.5, token_chunk=160)
    _call("separate", 200, 128, 3000, seed=2, grads=True, div="jsd", T=2.0, Ht=96)


def test_static_entry_forward_only_two_calls():
    _call("tied", 900, 256, 7000, seed=3, grads=False, div="reverse_kl", T=2.0)
    _call("tied", 100, 64, 1000, seed=4, grads=False, div="hellinger", T=1.0)


def test_static_entry_rejects_a_problem_larger_than_its_scratch():
    from orda_ce_kernel import _native
    from orda_ce_kernel.divergences import resolve_divergence
    from orda_ce_kernel.ops._engine import FusedCall, _problem

    N, H, V = 8192, 4096, 128256
    hs = torch.empty(N, H, dtype=torch.bfloat16, device="cuda")
    W = torch.empty(V, H, dtype=torch.bfloat16, device="cuda")
    call = FusedCall(
        mode="tied", student_hidden=hs, weight=W, labels=torch.zeros(N, dtype=torch.long, device="cuda"),
        teacher_hidden=hs, teacher_weight=None, teacher_logits=None, student_ce_weight=1.0, teacher_ce_weight=1.0,
        kl_weight=1.0, kl_temperature=1.0, ignore_index=-100, reduction="mean", vocab_chunk=0,
        divergence=resolve_divergence("forward_kl"), compute_teacher_ce=True, need_grad_student_hidden=True,
        need_grad_weight=True, grads_in_forward=True, token_chunk=0,
    )
    problem = _problem(call, H, H, None)
    assert _native.forward_workspace_bytes(problem) > _native.STATIC_SCRATCH_BYTES
    with pytest.raises(RuntimeError, match="static scratch"):
        _native.forward_static(problem, _native.Tensors(), hs.device)
