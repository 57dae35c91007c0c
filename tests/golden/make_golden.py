"""Writes tests/golden/golden.json: float64 oracle outputs on seeded inputs.

Cases: BASELINE config 1 (tied, N=512, H=256, V=4096, T=2, alpha 0.5 ->
student_ce_weight 0.5 / kl_weight 0.5, teacher CE weight default 1.0 and
0.0) and every divergence on a small tied problem (N=16, H=8, V=40, T=1.5).
Inputs come from torch's CPU generator (seed in the fixture); the fixture
stores a SHA-256 of the input bytes so a generator change is detected.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.orda_oracle import DIVERGENCE_DEFS, distillation_loss_oracle  # noqa: E402


def config1_inputs(seed=1001):
    g = torch.Generator().manual_seed(seed)
    N, H, V = 512, 256, 4096
    hs = torch.randn(N, H, generator=g)
    ht = hs + 0.1 * torch.randn(N, H, generator=g)
    W = 0.02 * torch.randn(V, H, generator=g)
    y = torch.randint(0, V, (N,), generator=g)
    y[torch.randperm(N, generator=g)[:26]] = -100
    return hs, ht, W, y


def small_inputs(seed=77):
    g = torch.Generator().manual_seed(seed)
    N, H, V = 16, 8, 40
    hs = 0.6 * torch.randn(N, H, generator=g)
    ht = 0.6 * torch.randn(N, H, generator=g)
    W = 0.6 * torch.randn(V, H, generator=g)
    y = torch.randint(0, V, (N,), generator=g)
    y[::5] = -100
    return hs, ht, W, y


def digest(*tensors):
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().numpy().tobytes())
    return h.hexdigest()


def summarize(out):
    res = {k: out[k] for k in ("loss", "student_ce", "teacher_ce", "kl")}
    for key in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden"):
        g = out[key]
        res[key] = {"sum": float(g.sum()), "abs_sum": float(np.abs(g).sum()), "l2": float(np.sqrt((g * g).sum())),
                    "corner": g[:2, :3].tolist()}
    return res


def main():
    f64 = lambda t: t.double().numpy()  # noqa: E731
    hs, ht, W, y = config1_inputs()
    cases = {}
    for name, w_t in (("config1_teacher_ce_default", None), ("config1_teacher_ce_zero", 0.0)):
        out = distillation_loss_oracle("tied", f64(hs), f64(W), y.numpy(), teacher_hidden=f64(ht), student_ce_weight=0.5,
                                       teacher_ce_weight=w_t, kl_weight=0.5, kl_temperature=2.0)
        cases[name] = summarize(out)
    s_hs, s_ht, s_W, s_y = small_inputs()
    for div in sorted(DIVERGENCE_DEFS):
        out = distillation_loss_oracle("tied", f64(s_hs), f64(s_W), s_y.numpy(), teacher_hidden=f64(s_ht),
                                       kl_weight=0.8, kl_temperature=1.5, divergence=div)
        cases[f"small_{div}"] = summarize(out)
    golden = {
        "generator": "torch.Generator (CPU)",
        "config1": {"seed": 1001, "sha256": digest(hs, ht, W, y)},
        "small": {"seed": 77, "sha256": digest(s_hs, s_ht, s_W, s_y)},
        "cases": cases,
    }
    path = Path(__file__).with_name("golden.json")
    path.write_text(json.dumps(golden, indent=1, sort_keys=True))
    print(f"wrote {path} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
