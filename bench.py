#!/usr/bin/env python
"""Benchmark: fused CE + distillation loss, forward + backward, on one MI355X.

Default workload is BASELINE config 2 (tied teacher, bf16, N=8192 tokens
(B=4 x T=2048), hidden 4096, vocab 128256, forward KL, T=1, kl_weight 1,
student and teacher CE weight 1, gradients for student hidden and W; the
teacher hidden is frozen).  A step is ``loss = distillation_loss(...);
loss.backward()`` on inputs resident in HBM.  Prints ONE JSON line.

Extra fields beyond the driver contract:
  roofline      dominant kernel class: algorithmic flops per launch / mean
                launch time (hipEvents recorded by the library on its launch
                stream during the timed steps) against 2.5 PFLOP/s bf16
  step_roofline whole step: algorithmic flops (5 x 2NVH at config 2) / step time
  kernels       per kernel class: launches, ms per step, executed and
                algorithmic TFLOP/s
  peak_extra_hbm_gb  max_memory_allocated - memory_allocated before a step
                (gradients count), the reference's own method
  cpu_baseline  the oracle's unfused PyTorch restatement (fp32) on the
                host cores, on a bounded token sample of the same workload
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "orda-knowledge-distillation-kernel_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "fwd+bwd tokens/s, CE+KL distill, h4096 V128256 bf16; peak extra HBM GB"
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    # name: (mode, N, H, Ht, V, dtype, divergence, T, w_s, w_t, kl_w, ignore_frac)
    "c1": ("tied", 512, 256, 256, 4096, "float32", "forward_kl", 2.0, 0.5, None, 0.5, 0.05),
    "c2": ("tied", 8192, 4096, 4096, 128256, "bfloat16", "forward_kl", 1.0, 1.0, None, 1.0, 0.05),
    "c3": ("separate", 8192, 2048, 4096, 128256, "bfloat16", "reverse_kl", 2.0, 1.0, None, 1.0, 0.05),
    "c3jsd": ("separate", 8192, 2048, 4096, 128256, "bfloat16", "jsd", 2.0, 1.0, None, 1.0, 0.05),
    "c4": ("precomputed", 8192, 4096, 4096, 128256, "bfloat16", "forward_kl", 1.0, 1.0, None, 1.0, 0.05),
    "c5": ("tied", 32768, 5120, 5120, 152064, "bfloat16", "forward_kl", 1.0, 0.7, None, 0.3, 0.20),
    # config 4's teacher as its top-64 (id, log-prob) pairs per token (TopKTeacher)
    "c4topk": ("topk", 8192, 4096, 4096, 128256, "bfloat16", "forward_kl", 1.0, 1.0, None, 1.0, 0.05),
    # launch-table shapes beyond the benchmark configurations: configs 2-5 in fp16, and two
    # other (hidden, vocabulary) pairs of the tied headline workload (8192 tokens)
    "c2f16": ("tied", 8192, 4096, 4096, 128256, "float16", "forward_kl", 1.0, 1.0, None, 1.0, 0.05),
    "c3f16": ("separate", 8192, 2048, 4096, 128256, "float16", "reverse_kl", 2.0, 1.0, None, 1.0, 0.05),
    "c4f16": ("precomputed", 8192, 4096, 4096, 128256, "float16", "forward_kl", 1.0, 1.0, None, 1.0, 0.05),
    "c5f16": ("tied", 32768, 5120, 5120, 152064, "float16", "forward_kl", 1.0, 0.7, None, 0.3, 0.20),
    "h8192": ("tied", 8192, 8192, 8192, 128256, "bfloat16", "forward_kl", 1.0, 1.0, None, 1.0, 0.05),
    "h3584": ("tied", 8192, 3584, 3584, 152064, "bfloat16", "forward_kl", 1.0, 1.0, None, 1.0, 0.05),
}
TOPK = 64
# config 5: teacher rows scaled by c / tau_n, tau_n ~ U[0.5, 4]; c puts the teacher logit spread at
# ~6.4 standard deviations for tau = 0.5 (entropy of a few nats) and ~0.8 for tau = 4 (near uniform)
ROW_TEMPERATURE = {"c5": (0.5, 4.0, 6.4 * 0.5 / (0.02 * 5120 ** 0.5)),
                   "c5f16": (0.5, 4.0, 6.4 * 0.5 / (0.02 * 5120 ** 0.5))}


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_inputs(cfg, device, seed, row_tau=None):
    import torch

    mode, N, H, Ht, V, dtype_name, *_rest, ignore_frac = cfg
    dtype = getattr(torch, dtype_name)
    g = torch.Generator(device=device).manual_seed(seed)
    hs = torch.randn(N, H, generator=g, device=device).to(dtype)
    if mode == "tied":
        ht = torch.randn(N, H, generator=g, device=device)
        if row_tau is not None:
            lo, hi, c = row_tau
            ht *= (c / (lo + (hi - lo) * torch.rand(N, generator=g, device=device)))[:, None]
        ht = ht.to(dtype)
        Wt = None
    else:
        ht = torch.randn(N, Ht, generator=g, device=device).to(dtype)
        Wt = (0.02 * torch.randn(V, Ht, generator=g, device=device)).to(dtype)
    W = (0.02 * torch.randn(V, H, generator=g, device=device)).to(dtype)
    y = torch.randint(0, V, (N,), generator=g, device=device)
    n_ign = int(round(ignore_frac * N))
    y[torch.randperm(N, generator=g, device=device)[:n_ign]] = -100
    lt = None
    if mode in ("precomputed", "topk"):
        # teacher log-probs of N(0, 3) logits, stored bf16 (config 4)
        lt = torch.empty(N, V, dtype=dtype, device=device)
        for s in range(0, N, 1024):
            e = min(N, s + 1024)
            lt[s:e] = torch.log_softmax(3.0 * torch.randn(e - s, V, generator=g, device=device), -1).to(dtype)
    if mode == "topk":
        vals, idx = lt.float().topk(TOPK, dim=1)
        del lt
        lt = (idx, vals)
    return hs, ht, W, Wt, lt, y


def algorithmic_flops(cfg) -> float:
    """GEMM flops the reference's algorithm needs per step (no recompute):
    forward one 2NVH per logits distribution; backward one per requested
    grad_hidden and one per dlogits source feeding grad_W."""
    mode, N, H, Ht, V = cfg[:5]
    w_t = cfg[9]
    G = lambda h: 2.0 * N * V * h  # noqa: E731
    if mode == "tied":
        teacher_ce = (1.0 if w_t is None else w_t) != 0.0
        return G(H) * (2 + 1 + (2 if teacher_ce else 1))
    if mode == "separate":
        return G(Ht) + 3 * G(H)
    return 3 * G(H)


def run_gpu(cfg, steps, warmup, seed, timing, row_tau=None, chunk=None, splits=None, student_norm=False,
            logits_gemm="default", teacher_logits_fp32=False, compiled_backend=None):
    import torch

    import orda_ce_kernel as orda
    from orda_ce_kernel import _native
    from orda_ce_kernel.ops import _engine

    # launch-table sweeps: an explicit requested chunk and grad-hidden split count
    config = orda.KernelConfig(chunk_size=chunk) if chunk else None
    _engine.LAUNCH_OVERRIDES["grad_hidden_splits"] = splits

    mode, N, H, Ht, V, dtype_name, div, T, w_s, w_t, kl_w, _ = cfg
    device = "cuda"
    hs, ht, W, Wt, lt, y = make_inputs(cfg, device, seed, row_tau)
    hs.requires_grad_(True)
    W.requires_grad_(True)
    if mode == "tied":
        teacher = orda.TiedTeacher(ht)
    elif mode == "separate":
        teacher = orda.SeparateTeacher(ht, Wt)
    elif mode == "topk":
        teacher = orda.TopKTeacher(*lt)
    else:
        if teacher_logits_fp32:  # the same log-probs held in float32 (cast to the compute dtype per chunk)
            lt = lt.float()
        teacher = orda.PrecomputedTeacher(logits=lt)
    norm = None
    if student_norm:
        # the student's final RMSNorm fused in front of the loss (hs is its input)
        nw = (1.0 + 0.1 * torch.randn(H, generator=torch.Generator(device=device).manual_seed(seed + 7),
                                      device=device)).to(hs.dtype).requires_grad_(True)
        norm = orda.StudentRMSNorm(nw)

    if compiled_backend:
        # the torch.compile-friendly entry (custom ops) in one compiled graph
        from orda_ce_kernel import compiled

        def loss_fn(a, b, c, tch):
            return compiled.distillation_loss(a, b, c, tch, student_ce_weight=w_s, teacher_ce_weight=w_t,
                                              kl_weight=kl_w, kl_temperature=T, divergence=div, chunk_size=chunk,
                                              student_norm=norm, logits_gemm=logits_gemm)

        compiled_fn = torch.compile(loss_fn, fullgraph=True, backend=compiled_backend)

    def step():
        if compiled_backend:
            out = compiled_fn(hs, W, y, teacher)
        else:
            out = orda.distillation_loss(hs, W, y, teacher, student_ce_weight=w_s, teacher_ce_weight=w_t,
                                         kl_weight=kl_w, kl_temperature=T, backend="triton", divergence=div,
                                         config=config, student_norm=norm, logits_gemm=logits_gemm)
        out.loss.backward()
        hs.grad = None
        W.grad = None
        if norm is not None:
            norm.weight.grad = None
        return out

    _log(f"[bench] warmup {warmup} step(s)")
    for _ in range(max(warmup, 1)):
        out = step()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = step()
    torch.cuda.synchronize()
    peak_extra = torch.cuda.max_memory_allocated() - base
    loss_val = float(out.loss)
    _log(f"[bench] loss={loss_val:.6f} peak extra {peak_extra / 1e9:.3f} GB; timing {steps} steps")

    if timing:
        _native.timing_enable(True)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern = _native.timing_collect() if timing else None
    if timing:
        _native.timing_enable(False)
    ms_step = start.elapsed_time(stop) / steps
    _log(f"[bench] {ms_step:.3f} ms/step (wall {wall * 1e3 / steps:.3f})")
    return ms_step, peak_extra, loss_val, kern


def launch_plan_of(cfg, chunk, splits):
    """The library's launch plan for the benchmark call (gfx950 launch
    table row, token chunk, grad-hidden split count)."""
    from orda_ce_kernel import _native

    mode, N, H, Ht, V, dtype_name, div, T, w_s, w_t, kl_w, _ = cfg
    p = _native.Problem()
    p.abi_version = _native.ABI_VERSION
    p.mode = {"tied": 0, "separate": 1, "precomputed": 2, "topk": 4}[mode]
    p.topk = TOPK if mode == "topk" else 0
    p.dtype = p.logits_dtype = {"bfloat16": 0, "float16": 1, "float32": 2}[dtype_name]
    p.n_rows, p.vocab, p.hidden, p.teacher_hidden = N, V, H, Ht
    p.ignore_index = -100
    w_t_eff = (1.0 if mode == "tied" else 0.0) if w_t is None else w_t
    f = _native.FLAG
    p.flags = f["need_grad_student_hidden"] | f["need_grad_weight"] | f["grads_in_forward"]
    if w_t_eff != 0.0:
        p.flags |= f["compute_teacher_ce"]
    if kl_w != 0.0:
        p.flags |= f["compute_divergence"]
    from orda_ce_kernel.divergences import resolve_divergence

    d = resolve_divergence(div)
    p.divergence = d.code
    p.div_alpha = d.alpha or 0.0
    p.div_beta = d.beta or 0.0
    p.temperature = T
    p.student_ce_weight, p.teacher_ce_weight, p.kl_weight = w_s, w_t_eff, kl_w
    p.token_chunk = chunk or 512  # the dispatcher's auto chunk at these sizes
    p.grad_hidden_splits = splits or 0
    info = _native.plan_info(p)
    return {k: info[k] for k in ("table_entry", "token_chunk", "n_token_chunks", "grad_hidden_splits",
                                 "scan_workgroups", "scan_engine")}


def kernel_report(kern, steps, peak_tflops):
    rows = {}
    for name, k in kern.items():
        if k["launches"] == 0:
            continue
        sec = k["ms"] / 1e3
        rows[name] = {
            "launches_per_step": k["launches"] / steps,
            "ms_per_step": k["ms"] / steps,
            "mean_launch_ms": k["ms"] / k["launches"],
            "executed_tflops": (k["executed_flops"] / sec / 1e12) if sec > 0 else 0.0,
            "algorithmic_tflops": (k["algorithmic_flops"] / sec / 1e12) if sec > 0 else 0.0,
            "executed_mfma_frac": (k["executed_flops"] / sec / 1e12 / peak_tflops) if sec > 0 else 0.0,
        }
    return rows


def cpu_baseline(cfg, seed, budget_s, row_tau=None):
    """Time the oracle's unfused torch restatement (fp32) on a token sample."""
    import torch

    from oracle.torch_unfused import tied_forward_kl_loss

    mode, N, H, Ht, V, dtype_name, div, T, w_s, w_t, kl_w, _ = cfg
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    hs, ht, W, _, _, y = make_inputs(cfg, "cuda", seed, row_tau)
    Wc = W.float().cpu()
    hs_c, ht_c, y_c = hs.float().cpu(), ht.float().cpu(), y.cpu()
    del hs, ht, W
    w_t_eff = 1.0 if w_t is None else w_t

    Wc.requires_grad_(True)

    def run(n):
        a = hs_c[:n].clone().requires_grad_(True)
        Wc.grad = None
        t0 = time.perf_counter()
        loss, *_ = tied_forward_kl_loss(a, ht_c[:n], Wc, y_c[:n], student_ce_weight=w_s,
                                        teacher_ce_weight=w_t_eff, kl_weight=kl_w, kl_temperature=T)
        loss.backward()
        return time.perf_counter() - t0

    run(16)  # warm up allocator and thread pool
    probe = 64
    t_probe = run(probe)
    per_tok = t_probe / probe
    # one warm-up run of the sample size, then the median of 3: about budget_s in all
    n = int(max(probe, min(N, (budget_s / 4.0) / per_tok)))
    n = max(probe, (n // 64) * 64)
    run(n)
    times = [run(n) for _ in range(3)]
    t = statistics.median(times)
    cpu_name = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": n / t,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{n} of {N} tokens of the same workload (full V={V}, H={H}), fp32 unfused torch restatement "
                   f"of the reference loss (oracle/torch_unfused.py), fwd+bwd, median of {len(times)} runs after "
                   f"1 warm-up; torch threads {torch.get_num_threads()} = os.cpu_count()={os.cpu_count()}, "
                   f"{cpu_name}"),
    }


def profiled_traffic(config: str, kernel_class: str):
    """HBM bytes per launch of ``kernel_class`` at ``config`` from the
    committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary (profiles/*_pmc_traffic.md,
    one fenced json line per kernel class), or None when none covers it."""
    for md in sorted((ROOT / "profiles").glob("*_pmc_traffic.md")):
        for line in md.read_text().splitlines():
            line = line.strip()
            if not (line.startswith("{") and "traffic_bytes_per_launch" in line):
                continue
            rec = json.loads(line)
            if rec.get("workload") == config and rec.get("class") == kernel_class:
                return float(rec["traffic_bytes_per_launch"]), md.name
    return None, None


def copy_calibration(mib: int) -> int:
    """Three device copies of ``mib`` MiB each through an elementwise kernel
    (dst = src * 1, fp32; a blit could go to the DMA engines and show no
    dispatch): its HBM traffic is known exactly, mib MiB read + mib MiB
    written per launch."""
    import torch

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    n = mib << 20
    src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ev[0].record()
    for i in range(3):
        torch.mul(src, 1.0, out=dst)
        ev[i + 1].record()
    torch.cuda.synchronize()
    ms = [ev[i].elapsed_time(ev[i + 1]) for i in (1, 2)]  # (the first launch warms up)
    gbps = 2 * n / (sum(ms) / 2) / 1e6
    print(json.dumps({"copy_calibration_bytes": n, "launches": 3, "ms_per_copy": ms,
                      "copy_gbps": gbps}), flush=True)
    return 0


def library_gemms() -> int:
    """The config-2 GEMM shapes through torch.mm (hipBLASLt on ROCm) with
    random bf16 data, as the library GEMM this build's kernels compare with:
    one json line per shape with ms and TFLOP/s (10 timed calls after 3)."""
    import torch

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    torch.manual_seed(0)
    V, H, n = 128256, 4096, 1024
    dev = "cuda"

    def timed(f, flops, shape):
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(10):
            f()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / 10
        print(json.dumps({"library_gemm": shape, "ms": ms, "tflops": flops / ms / 1e9}), flush=True)

    L = (torch.randn(V, 2 * n, device=dev) * 1e-3).bfloat16()
    hT = torch.randn(2 * n, H, device=dev).bfloat16()
    C = (torch.randn(V, H, device=dev) * 1e-2).bfloat16()
    timed(lambda: torch.mm(L, hT, out=C), 2.0 * V * H * 2 * n, "grad W store [V x 2n] @ [2n x H]")
    timed(lambda: C.addmm_(L, hT), 2.0 * V * H * 2 * n, "grad W accumulate (addmm_) [V x 2n] @ [2n x H]")
    W = (torch.randn(V, H, device=dev) * 0.02).bfloat16()
    LT = L[:, :n].t()
    timed(lambda: torch.mm(LT, W), 2.0 * n * V * H, "grad hidden [n x V] @ [V x H]")
    X = torch.randn(2 * n, H, device=dev).bfloat16()
    timed(lambda: torch.mm(X, W.t()), 2.0 * V * H * 2 * n, "logits [2n x H] @ [H x V]")
    A, B = torch.randn(8192, 4096, device=dev).bfloat16(), torch.randn(4096, 4096, device=dev).bfloat16()
    timed(lambda: torch.mm(A, B), 2.0 * 8192 * 4096 * 4096, "square 8192 x 4096 x 4096")
    return 0


TWO_PASS = ("jsd", "skew_forward_kl", "skew_reverse_kl", "tvd")
SWEEP_DIVERGENCES = ("forward_kl", "reverse_kl", "symmetric_kl", "soft_target_ce", "hellinger", "bhattacharyya",
                     "renyi", "amari_alpha", "chi_squared", "squared_l2", "ab", "jsd", "skew_forward_kl",
                     "skew_reverse_kl", "tvd")


def sweep(cfg, args, row_tau) -> int:
    """ms per fwd+bwd step for every divergence at T = 1 and 4 (default
    alpha/beta: skew 0.1, JSD 0.5), with the kernel-class split."""
    mode, N, H, Ht, V, dtype_name = cfg[:6]
    for T in (1.0, 4.0):
        for div in SWEEP_DIVERGENCES:
            c = cfg[:6] + (div, T) + cfg[8:]
            ms, peak_extra, loss, kern = run_gpu(c, args.steps, args.warmup, args.seed, True, row_tau)
            rows = kernel_report(kern, args.steps, PEAK_BF16_TFLOPS)
            print(json.dumps({
                "config": args.config, "divergence": div, "temperature": T, "ms_per_step": ms,
                "tokens_per_s": N / (ms / 1e3), "step_tflops": algorithmic_flops(c) / (ms / 1e3) / 1e12,
                "peak_extra_hbm_gb": peak_extra / 1e9, "loss": loss,
                "ms_per_step_by_class": {k: round(r["ms_per_step"], 4) for k, r in rows.items()},
            }), flush=True)
    return 0


# Launch-table sweep: (requested chunk, grad-hidden split count) per config;
# the chunk is the dispatcher's chunk_size, which the library scales by the
# table's chunk_scale (so 512 -> 1024 tokens at scale 2).  A split count of
# None is the library's own choice (the table entry, or the rule for shapes
# the table does not list).
TABLE_SWEEP = {
    "c2": [(c, s) for c in (256, 512) for s in (4, 8, 12, 16)],
    "c3": [(c, s) for c in (512, 1024) for s in (4, 8, 16)],
    "c4": [(c, s) for c in (256, 512) for s in (2, 4, 8)],
    "c5": [(256, 16), (512, 4), (512, 8), (512, 16), (1024, 8)],
    "c2f16": [(c, s) for c in (256, 512) for s in (None, 4, 8, 16)],
    "c3f16": [(c, s) for c in (512, 1024) for s in (None, 4, 8)],
    "c4f16": [(c, s) for c in (256, 512) for s in (None, 2, 4, 8)],
    "c5f16": [(256, None), (512, None), (512, 4), (512, 8), (512, 16), (1024, 8), (1024, 16)],
    "h8192": [(c, s) for c in (256, 512, 1024) for s in (None, 2, 4, 8)],
    "h3584": [(c, s) for c in (256, 512, 1024) for s in (None, 4, 8, 16)],
}


def table_sweep(args) -> int:
    """ms per step for each launch-table candidate of every configuration
    (one json line each); the rows behind csrc/launch_table.hpp."""
    import torch

    only = set(args.sweep_configs.split(",")) if args.sweep_configs else None
    for name, cases in TABLE_SWEEP.items():
        if only is not None and name not in only:
            continue
        cfg = CONFIGS[name]
        row_tau = ROW_TEMPERATURE.get(name)
        for chunk, splits in cases:
            ms, peak_extra, _, kern = run_gpu(cfg, args.steps, args.warmup, args.seed, True, row_tau, chunk=chunk,
                                              splits=splits)
            rows = kernel_report(kern, args.steps, PEAK_BF16_TFLOPS)
            plan = launch_plan_of(cfg, chunk, splits)
            print(json.dumps({
                "config": name, "chunk": chunk, "splits": splits, "token_chunk": plan["token_chunk"],
                "used_splits": plan["grad_hidden_splits"], "table_entry": plan["table_entry"],
                "ms_per_step": round(ms, 3), "peak_extra_hbm_gb": round(peak_extra / 1e9, 3),
                "ms_per_step_by_class": {k: round(r["ms_per_step"], 3) for k, r in rows.items()},
            }), flush=True)
            torch.cuda.empty_cache()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--seed", type=int, default=1002)
    ap.add_argument("--divergence", default=None, help="override the config's divergence (config 4 sweep)")
    ap.add_argument("--temperature", type=float, default=None, help="override the config's temperature")
    ap.add_argument("--sweep", action="store_true",
                    help="instead of the one-line benchmark, time every divergence at T=1 and T=4 on --config "
                         "(one json line per case; config 4's divergence sweep)")
    ap.add_argument("--chunk", type=int, default=None,
                    help="requested token chunk (KernelConfig.chunk_size; the library scales it by the launch "
                         "table's chunk_scale), for launch-table sweeps")
    ap.add_argument("--splits", type=int, default=None,
                    help="grad-hidden split-K count instead of the launch table's, for launch-table sweeps")
    ap.add_argument("--table-sweep", action="store_true",
                    help="instead of the one-line benchmark, time the launch-table candidates (requested chunk x "
                         "grad-hidden splits) of configs 2-5, one json line each")
    ap.add_argument("--sweep-configs", default=None, metavar="NAMES",
                    help="with --table-sweep: only these configurations (comma-separated)")
    ap.add_argument("--student-norm", action="store_true",
                    help="fuse the student's final RMSNorm in front of the loss (StudentRMSNorm)")
    ap.add_argument("--logits-gemm", default="default", choices=("default", "fp8"),
                    help="fp8: the logits GEMM on e4m3 operands (its own tolerance; not the headline number)")
    ap.add_argument("--teacher-logits-fp32", action="store_true",
                    help="precomputed configurations: hold the teacher's logits in float32 (an input-format variant)")
    ap.add_argument("--compiled", nargs="?", const="inductor", default=None, metavar="BACKEND",
                    help="run the step through the torch.compile-friendly entry (orda_ce_kernel.compiled) under "
                         "torch.compile(fullgraph=True, backend=BACKEND; default inductor)")
    ap.add_argument("--cpu-budget", type=float, default=24.0, help="seconds of CPU-baseline work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-timing", action="store_true")
    ap.add_argument("--library-gemms", action="store_true",
                    help="instead of the benchmark, time the config-2 GEMM shapes through torch.mm (hipBLASLt) and exit")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run 3 plain device copies of MIB MiB (the known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings into bytes) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.library_gemms:
        return library_gemms()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every GPU box has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    cfg = CONFIGS[args.config]
    if args.divergence is not None or args.temperature is not None:
        cfg = cfg[:6] + (args.divergence or cfg[6], cfg[7] if args.temperature is None else args.temperature) + cfg[8:]
    row_tau = ROW_TEMPERATURE.get(args.config)
    if args.sweep:
        return sweep(cfg, args, row_tau)
    if args.table_sweep:
        return table_sweep(args)
    mode, N, H, Ht, V, dtype_name, div, T, w_s, w_t, kl_w, ignore_frac = cfg
    ms_step, peak_extra, loss_val, kern = run_gpu(cfg, args.steps, args.warmup, args.seed, not args.no_timing,
                                                 row_tau, chunk=args.chunk, splits=args.splits,
                                                 student_norm=args.student_norm, logits_gemm=args.logits_gemm,
                                                 teacher_logits_fp32=args.teacher_logits_fp32,
                                                 compiled_backend=args.compiled)
    peak = PEAK_FP32_TFLOPS if dtype_name == "float32" else PEAK_BF16_TFLOPS
    alg = algorithmic_flops(cfg)
    step_tflops = alg / (ms_step / 1e3) / 1e12

    result = {
        "metric": METRIC,
        "value": N / (ms_step / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"bfloat16": "bf16", "float32": "f32", "float16": "f16"}[dtype_name]
                 + (" (fp8 e4m3 logits GEMM)" if args.logits_gemm == "fp8" else ""),
        "data": "synthetic (seeded randn hidden/weights, uniform labels with ignore_index; no checkpoint)",
        "config": {
            "workload": f"{args.config}: {mode} teacher, N={N} tokens, hidden={H}"
                        + (f", teacher hidden={Ht}" if mode != "tied" else "")
                        + f", vocab={V}, {div}, T={T}, fwd+bwd (grad hidden + grad W)"
                        + (f", top-{TOPK} teacher" if mode == "topk" else "")
                        + (", student RMSNorm fused (grad x + grad norm weight)" if args.student_norm else "")
                        + (", fp8 (e4m3) logits GEMM" if args.logits_gemm == "fp8" else "")
                        + (", teacher logits held in float32" if args.teacher_logits_fp32 else "")
                        + (f", torch.compile(fullgraph=True, backend={args.compiled}) through the custom-op entry"
                           if args.compiled else ""),
            "tokens": N, "hidden": H, "vocab": V, "teacher": mode, "divergence": div, "temperature": T,
            "student_ce_weight": w_s, "teacher_ce_weight": w_t, "kl_weight": kl_w, "ignore_frac": ignore_frac,
        },
        "launch_plan": launch_plan_of(cfg, args.chunk, args.splits),
        "peak_extra_hbm_gb": peak_extra / 1e9,
        "loss": loss_val,
        "step_roofline": {
            "bound": "mfma", "achieved": step_tflops, "peak": peak, "unit": "TFLOP/s", "frac": step_tflops / peak,
            "algorithmic_tflop_per_step": alg / 1e12,
        },
    }
    if kern is not None:
        rows = kernel_report(kern, args.steps, peak)
        result["kernels"] = rows
        # dominant kernel class by time among those that carry algorithmic flops
        dominant = max((r for r in rows if rows[r]["algorithmic_tflops"] > 0), key=lambda r: rows[r]["ms_per_step"])
        k = kern[dominant]
        mean_ms = k["ms"] / k["launches"]
        alg_per_launch = k["algorithmic_flops"] / k["launches"]
        achieved = alg_per_launch / (mean_ms / 1e3) / 1e12
        traffic, source = profiled_traffic(args.config, dominant)
        result["roofline"] = {
            "bound": "mfma", "achieved": achieved, "peak": peak, "unit": "TFLOP/s", "frac": achieved / peak,
            "traffic": traffic, "kernel": dominant, "mean_launch_ms": mean_ms,
            "algorithmic_tflop_per_launch": alg_per_launch / 1e12,
        }
        if traffic is not None:
            result["roofline"]["traffic_source"] = f"profiles/{source} (rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated)"
        if "dlogits" in kern and kern["dlogits"]["launches"] > 0:
            # the HBM-bound streaming pass over the materialised logits: student logits read and
            # dlogits written in place, teacher logits read when the divergence or the teacher CE
            # needs them, teacher dlogits written when the teacher CE has a gradient
            es = 4 if dtype_name == "float32" else 2
            w_t_eff = (1.0 if mode == "tied" else 0.0) if w_t is None else w_t
            tgrad = w_t_eff != 0.0
            # (a top-k teacher has no dense teacher logits to read)
            passes = 2 + (1 if ((kl_w != 0.0 and mode != "topk") or tgrad) else 0) + (1 if tgrad else 0)
            if kl_w != 0.0 and div in TWO_PASS:
                passes += 2  # the second pass of the two-pass divergences reads both halves again
            d = kern["dlogits"]
            gbs = passes * N * V * es * args.steps / (d["ms"] / 1e3) / 1e9  # every launch of the timed steps
            result["stream"] = {
                "bound": "hbm", "kernel": "dlogits", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": gbs / PEAK_HBM_GBS, "algorithmic_bytes_per_step": passes * N * V * es,
                "mean_launch_ms": d["ms"] / d["launches"],
            }
    if not args.no_cpu_baseline and mode == "tied":
        _log("[bench] CPU baseline")
        result["cpu_baseline"] = cpu_baseline(cfg, args.seed, args.cpu_budget, row_tau)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
