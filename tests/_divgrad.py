"""Shared cases and bounds for the distillation-gradient parity tests.

The distillation term is isolated (``student_ce_weight = 0``,
``teacher_ce_weight = 0``, ``kl_weight = 1``), so the gradients checked are
``T * dD/dz_s`` pushed through the LM-head GEMMs and nothing else.  Logits
have a spread of about 1.5 nats and the teacher is independent of the student,
so ``p_t`` and ``p_s`` differ everywhere and every divergence's gradient is of
the same order as the gradient itself (at ``W ~ N(0, 0.02)`` both
distributions are near uniform and every divergence's gradient is a tiny
correction that a loose bound cannot see).

Expected gradients come from the float64 oracle; for 16-bit inputs with
``grad_logits_dtype`` set to the compute dtype, so the dlogits are formed
from the logits rounded as the kernels store them (as the reference's row
kernel reads its bf16 logits).  Bounds (``grad_errors`` / ``grad_ok``),
relative to the scale of the expected gradient:

* worst elementwise ``|err| <= c_max * max|ref|``;
* relative Frobenius ``||err|| <= c_fro * ||ref||``;

with ``c_fro = 2e-2`` and ``c_max = 4e-2`` for 16-bit inputs and ``1e-4`` /
``2e-4`` for float32.  The 16-bit worst-element bound has room for the
rounding of the stored logits that the row constants do not see: the
kernels take the row statistics from the fp32 logits and the dlogits from
the rounded ones, which Renyi(alpha = 2) at T = 1 amplifies most (the
teacher's rounding enters twice; 2.6% measured on the GPU, Frobenius 1.2%).
TVD's gradient is a sign function of ``p_s - p_t``: where the two are within
rounding of each other a result may take either side, so TVD gets ``c_max =
0.5``, ``c_fro = 0.1`` in 16 bits and ``5e-3`` / ``1e-3`` in float32.
``tests/test_divergence_grad_bounds.py`` shows on the CPU that at these
shapes every planted slip in the oracle's divergence gradient (zeroed,
sign-flipped, dropped temperature factor, softmax Jacobian without its
centring term, the probabilities taken at T = 1, forward KL's gradient in
place of another divergence's) breaks the bound, and that an emulation of
the 16-bit path's roundings stays inside it.
"""
from __future__ import annotations

import numpy as np
import torch

# (id, name, alpha, beta): every divergence at its defaults, plus non-default
# parameters for the parametrised ones (at the defaults AB(1/2, 1/2) equals
# Amari(1/2) and Renyi(1/2) is twice Bhattacharyya, so defaults alone cannot
# tell those kernels apart).
DIV_CASES = [
    ("forward_kl", "forward_kl", None, None),
    ("reverse_kl", "reverse_kl", None, None),
    ("symmetric_kl", "symmetric_kl", None, None),
    ("soft_target_ce", "soft_target_ce", None, None),
    ("hellinger", "hellinger", None, None),
    ("bhattacharyya", "bhattacharyya", None, None),
    ("renyi", "renyi", None, None),
    ("renyi_a2", "renyi", 2.0, None),
    ("amari_alpha", "amari_alpha", None, None),
    ("amari_a0.3", "amari_alpha", 0.3, None),
    ("chi_squared", "chi_squared", None, None),
    ("squared_l2", "squared_l2", None, None),
    ("ab", "ab", None, None),
    ("ab_0.6_0.3", "ab", 0.6, 0.3),
    ("jsd", "jsd", None, None),
    ("jsd_b0.25", "jsd", None, 0.25),
    ("skew_forward_kl", "skew_forward_kl", None, None),
    ("skew_forward_kl_a0.3", "skew_forward_kl", 0.3, None),
    ("skew_reverse_kl", "skew_reverse_kl", None, None),
    ("skew_reverse_kl_a0.3", "skew_reverse_kl", 0.3, None),
    ("tvd", "tvd", None, None),
]
DIV_IDS = [c[0] for c in DIV_CASES]
TEMPERATURES = (1.0, 2.0, 4.0)

# Shapes of the GPU cases: several vocabulary tiles with a ragged last one,
# two token tiles with a ragged last one, H a few K steps deep.
N, H, HT, V = 160, 128, 96, 1000
LOGIT_SCALE = 1.5


def bounds(dtype, divergence: str = "forward_kl") -> tuple[float, float]:
    """(c_max, c_fro) for inputs of ``dtype``."""
    if dtype == torch.float32:
        return (5e-3, 1e-3) if divergence == "tvd" else (2e-4, 1e-4)
    return (0.5, 0.1) if divergence == "tvd" else (4e-2, 2e-2)


def grad_logits_dtype(dtype) -> str | None:
    """The oracle's ``grad_logits_dtype`` for inputs of ``dtype``."""
    return {torch.bfloat16: "bfloat16", torch.float16: "float16"}.get(dtype)


def make_inputs(seed: int, dtype, *, n=N, h=H, ht_dim=HT, v=V, ignore_frac=0.05):
    """Student and teacher hidden states and weights with logits of spread
    ~LOGIT_SCALE; the teacher is independent of the student.  Returns CPU
    tensors in ``dtype``: hs [n, h], W [v, h], ht [n, h] (tied teacher),
    hts [n, ht_dim] and Wt [v, ht_dim] (separate / precomputed teacher), and
    labels [n] with ``ignore_frac`` of them -100."""
    g = torch.Generator().manual_seed(seed)
    hs = torch.randn(n, h, generator=g)
    W = torch.randn(v, h, generator=g) * (LOGIT_SCALE / h ** 0.5)
    ht = torch.randn(n, h, generator=g) * 1.2
    hts = torch.randn(n, ht_dim, generator=g)
    Wt = torch.randn(v, ht_dim, generator=g) * (1.2 * LOGIT_SCALE / ht_dim ** 0.5)
    y = torch.randint(0, v, (n,), generator=g)
    n_ign = int(round(ignore_frac * n))
    if n_ign:
        y[torch.randperm(n, generator=g)[:n_ign]] = -100
    cast = lambda x: x.to(dtype)  # noqa: E731
    return cast(hs), cast(W), cast(ht), cast(hts), cast(Wt), y


def grad_errors(actual: np.ndarray, expected: np.ndarray) -> tuple[float, float]:
    """(worst |err| / max|ref|, ||err|| / ||ref||)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    err = a - e
    scale = float(np.abs(e).max())
    fro = float(np.linalg.norm(e))
    worst = float(np.abs(err).max()) / scale if scale > 0 else float(np.abs(err).max())
    rel = float(np.linalg.norm(err)) / fro if fro > 0 else float(np.linalg.norm(err))
    return worst, rel


def grad_ok(actual: np.ndarray, expected: np.ndarray, dtype, divergence: str = "forward_kl") -> tuple[bool, str]:
    c_max, c_fro = bounds(dtype, divergence)
    worst, rel = grad_errors(actual, expected)
    ok = bool(np.all(np.isfinite(actual))) and worst <= c_max and rel <= c_fro
    return ok, f"worst/max {worst:.3e} (<= {c_max:g}), frobenius {rel:.3e} (<= {c_fro:g})"
