"""CPU oracle for the fused CE + distillation loss -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module, and only as the checker or the timed CPU
baseline.  The product (``orda_ce_kernel``) never imports it.

A float64 numpy restatement of the reference's algorithm (reference paths
relative to ``src/orda_ce_kernel/``):

* logits ``x_s = h_s W^T`` and ``x_t`` by teacher mode
  (``api.py:287-300``);
* per-row CE with the Triton kernels' label handling: ignored rows give 0,
  a label outside ``[0, V)`` counts as class 0 (``ops/tied_teacher.py:42-44,
  116-127``);
* the distillation term ``T^2 D(softmax(x_t/T) || softmax(x_s/T))`` masked on
  ignored rows (``ops/tied_teacher.py:182,188-189``, ``api.py:317-322``) --
  the reference has forward KL only; the other fourteen divergences are
  written from their published definitions (see ``DIVERGENCE_DEFS``);
* mean over non-ignored rows (``clamp(count, 1)``) or sum
  (``ops/tied_teacher.py:499-516``); ``loss = w_s CE_s + w_t CE_t + w_kl KL``;
  the teacher CE is reported as 0 when ``w_t == 0`` (``api.py:333``);
* with ``kernel_semantics=True`` the divergence is reported as 0 when
  ``kl_weight == 0`` (the Triton kernels skip it: ``COMPUTE_KL``,
  ``ops/tied_teacher.py:143,188``); the torch backend reports it
  (``api.py:317-331``);
* with ``grad_logits_dtype="bfloat16"`` / ``"float16"`` the dlogits are
  formed from the logits rounded to that dtype, as the reference's kernels
  form them: the chunk's logits are a matmul output in the compute dtype
  (``ops/tied_teacher.py:444-445``) that the row kernel loads and widens to
  fp32 (``:145-147``); loss values still come from the unrounded logits;
* gradients in closed form: student dlogits
  ``s [w_s (p_s - 1_y) + w_kl T dD/dz_s]`` and teacher dlogits
  ``s w_t (p_t - 1_y)`` (``ops/tied_teacher.py:153-186``), with
  ``dD/dz_s = p_s (g - <p_s, g>)``, ``g = dD/dp_s`` taken from each
  definition; then the GEMMs of ``ops/tied_teacher.py:468-495`` and the
  ``grad_output * mean_scale`` scaling of ``:538-545``.

Two teachers and a prologue that the reference's loss API does not have
(its benchmark producer and cache have them; see the tests named here):

* a top-k teacher read as precomputed logits ``lp`` on its ids and ``-inf``
  elsewhere (``topk_dense_logits``; ``tests/test_topk_teacher.py``);
* the student's final RMSNorm in front of the loss, ``y = x rsqrt(mean(x^2)
  + eps) w`` (the reference producer, ``test/benchmark/src/core.py:13-14``),
  with ``dx``, ``dw`` by the chain rule (``student_norm_weight=``;
  ``tests/test_rmsnorm_prologue.py``);
* the fp8 logits GEMM's operands: rows scaled by a power of two and rounded
  to OCP E4M3 (``quantize_rows_e4m3``, ``fp8_operands=``; pinned against
  torch's ``float8_e4m3fn`` in ``tests/test_fp8_logits.py``).

How it is pinned (``tests/test_oracle.py``): against torch float64 autograd
of ``F.cross_entropy`` / ``F.log_softmax`` / ``F.kl_div`` (the reference's own
test oracle, ``test/utils/reference.py:60-93``) on the reference's CPU test
cases; divergence values against scipy (``entropy``, ``jensenshannon``) and
closed-form identities (Renyi -> KL as alpha -> 1, AB(1/2,1/2) = 4 Hellinger^2,
AB(a,1-a) = Amari, Amari(1/2) = 4 Hellinger^2, ...); divergence gradients
against torch autograd and central finite differences; invariants
(all-ignored -> zeros, D(p||p) = 0, logit-shift invariance).
"""
from __future__ import annotations

import numpy as np

__all__ = ["DIVERGENCE_DEFS", "divergence_value_and_grad", "distillation_loss_oracle", "log_softmax",
           "quantize_rows_e4m3", "round_e4m3", "round_to", "topk_dense_logits"]


def round_e4m3(x: np.ndarray) -> np.ndarray:
    """``x`` rounded to the nearest OCP FP8 E4M3 value (ties to even; |x| <=
    448 assumed, as the callers scale it): normal values keep 3 mantissa
    bits (spacing ``2^(E - 3)`` for ``2^E <= |x| < 2^(E + 1)``, ``E >= -6``),
    subnormals are multiples of ``2^-9``.  Returned as float64."""
    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    with np.errstate(divide="ignore"):
        E = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    step = np.exp2(np.maximum(E, -6.0) - 3.0)
    q = np.round(a / step) * step  # numpy rounds half to even
    return np.sign(x) * np.minimum(q, 448.0)


def quantize_rows_e4m3(x: np.ndarray) -> np.ndarray:
    """Each row scaled by the power of two ``2^-e`` that puts its amax in
    ``(224, 448]`` (``e = 0`` for a zero row), rounded to E4M3, and scaled back
    (dequantised, float64): the operands of the fp8 logits GEMM."""
    x = np.asarray(x, dtype=np.float64)
    amax = np.abs(x).max(axis=1)
    m, k = np.frexp(np.where(amax > 0, amax, 1.0))
    e = np.where(amax > 0, k - 9 + (m > 0.875), 0).astype(np.float64)
    sc = np.exp2(e)[:, None]
    return round_e4m3(x / sc) * sc


def topk_dense_logits(indices: np.ndarray, logprobs: np.ndarray, V: int) -> np.ndarray:
    """A top-k teacher as dense teacher logits: its log-probabilities at its k
    vocabulary ids, -inf elsewhere.  Softmax of these (over V, at any
    temperature) is the teacher renormalised over its k ids, zero elsewhere --
    the distribution a top-k teacher stands for; the precomputed-logits path
    of the oracle then gives its loss and gradients."""
    idx = np.asarray(indices, dtype=np.int64)
    lp = np.asarray(logprobs, dtype=np.float64)
    out = np.full((idx.shape[0], int(V)), -np.inf)
    np.put_along_axis(out, idx, lp, axis=1)
    return out


def round_to(x: np.ndarray, dtype: str | None) -> np.ndarray:
    """``x`` rounded to float32, then to ``dtype`` ("bfloat16" / "float16",
    round to nearest even; None: unchanged), returned as float64.  The GPU
    kernels round an fp32 accumulator, so the float32 step is part of it."""
    if dtype is None:
        return np.asarray(x, dtype=np.float64)
    f = np.asarray(x, dtype=np.float32)
    if dtype == "float16":
        return f.astype(np.float16).astype(np.float64)
    if dtype != "bfloat16":
        raise ValueError(f"unknown dtype {dtype!r}")
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def log_softmax(x: np.ndarray) -> np.ndarray:
    m = x.max(axis=-1, keepdims=True)
    z = x - m
    return z - np.log(np.exp(z).sum(axis=-1, keepdims=True))


def _xlogy_ratio(p: np.ndarray, lp: np.ndarray, lq: np.ndarray) -> np.ndarray:
    """p * (log p - log q) with the 0 * (...) = 0 convention."""
    with np.errstate(invalid="ignore"):
        return np.where(p > 0, p * (lp - lq), 0.0)


def _logaddexp(a, b):
    return np.logaddexp(a, b)


def _lg(x: float) -> float:
    return np.log(x) if x > 0 else -np.inf


# Each entry: (value, dvalue/dp_s) of D(p_t || p_s) for one row, from the
# definition, on float64 probability vectors (pt, ps) and their logs.
def _fkl(pt, ps, lt, ls, a, b):
    return _xlogy_ratio(pt, lt, ls).sum(), -pt / ps


def _rkl(pt, ps, lt, ls, a, b):
    return _xlogy_ratio(ps, ls, lt).sum(), (ls - lt) + 1.0


def _sym(pt, ps, lt, ls, a, b):
    v1, g1 = _fkl(pt, ps, lt, ls, a, b)
    v2, g2 = _rkl(pt, ps, lt, ls, a, b)
    return v1 + v2, g1 + g2


def _soft(pt, ps, lt, ls, a, b):
    return -(pt * ls).sum(), -pt / ps


def _hell(pt, ps, lt, ls, a, b):
    r = np.exp(0.5 * (lt + ls))
    return 1.0 - r.sum(), -0.5 * np.exp(0.5 * (lt - ls))


def _bhat(pt, ps, lt, ls, a, b):
    bc = np.exp(0.5 * (lt + ls)).sum()
    return -np.log(bc), -0.5 * np.exp(0.5 * (lt - ls)) / bc


def _renyi(pt, ps, lt, ls, a, b):
    s = np.exp(a * lt + (1 - a) * ls).sum()
    return np.log(s) / (a - 1.0), (1 - a) * np.exp(a * lt - a * ls) / s / (a - 1.0)


def _amari(pt, ps, lt, ls, a, b):
    s = np.exp(a * lt + (1 - a) * ls).sum()
    return (1.0 - s) / (a * (1 - a)), -(1 - a) * np.exp(a * lt - a * ls) / (a * (1 - a))


def _chi2(pt, ps, lt, ls, a, b):
    return ((pt - ps) ** 2 / ps).sum(), 1.0 - (pt / ps) ** 2


def _l2(pt, ps, lt, ls, a, b):
    return ((pt - ps) ** 2).sum(), 2.0 * (ps - pt)


def _ab(pt, ps, lt, ls, a, b):
    s = a + b
    terms = np.exp(a * lt + b * ls) - a / s * np.exp(s * lt) - b / s * np.exp(s * ls)
    grad = -(b * np.exp(a * lt + (b - 1) * ls) - b * np.exp((s - 1) * ls)) / (a * b)
    return -terms.sum() / (a * b), grad


def _jsd(pt, ps, lt, ls, a, b):
    lm = _logaddexp(_lg(b) + lt, _lg(1 - b) + ls)
    v = b * _xlogy_ratio(pt, lt, lm).sum() + (1 - b) * _xlogy_ratio(ps, ls, lm).sum()
    return v, (1 - b) * (ls - lm)


def _skew_f(pt, ps, lt, ls, a, b):
    lm = _logaddexp(_lg(a) + lt, _lg(1 - a) + ls)
    return _xlogy_ratio(pt, lt, lm).sum(), -(1 - a) * np.exp(lt - lm)


def _skew_r(pt, ps, lt, ls, a, b):
    lm = _logaddexp(_lg(a) + ls, _lg(1 - a) + lt)
    return _xlogy_ratio(ps, ls, lm).sum(), (ls - lm) + 1.0 - a * np.exp(ls - lm)


def _tvd(pt, ps, lt, ls, a, b):
    return 0.5 * np.abs(pt - ps).sum(), 0.5 * np.sign(ps - pt)


# name -> (function, default alpha, default beta)
DIVERGENCE_DEFS = {
    "forward_kl": (_fkl, None, None),
    "reverse_kl": (_rkl, None, None),
    "symmetric_kl": (_sym, None, None),
    "soft_target_ce": (_soft, None, None),
    "hellinger": (_hell, None, None),
    "bhattacharyya": (_bhat, None, None),
    "renyi": (_renyi, 0.5, None),
    "amari_alpha": (_amari, 0.5, None),
    "chi_squared": (_chi2, None, None),
    "squared_l2": (_l2, None, None),
    "ab": (_ab, 0.5, 0.5),
    "jsd": (_jsd, None, 0.5),
    "skew_forward_kl": (_skew_f, 0.1, None),
    "skew_reverse_kl": (_skew_r, 0.1, None),
    "tvd": (_tvd, None, None),
}


def divergence_value_and_grad(z_t: np.ndarray, z_s: np.ndarray, name: str, alpha=None, beta=None):
    """Per-row D(softmax(z_t) || softmax(z_s)) and dD/dz_s for [rows, V]
    float64 arrays (z already divided by the temperature)."""
    fn, da, db = DIVERGENCE_DEFS[name]
    a = da if alpha is None else float(alpha)
    b = db if beta is None else float(beta)
    lt, ls = log_softmax(z_t), log_softmax(z_s)
    pt, ps = np.exp(lt), np.exp(ls)
    vals = np.empty(z_t.shape[0])
    grads = np.empty_like(z_s)
    for i in range(z_t.shape[0]):
        v, g = fn(pt[i], ps[i], lt[i], ls[i], a, b)
        vals[i] = v
        grads[i] = ps[i] * (g - (ps[i] * g).sum())  # softmax Jacobian
    return vals, grads


def distillation_loss_oracle(
    mode: str,
    student_hidden: np.ndarray,
    weight: np.ndarray,
    labels: np.ndarray,
    *,
    teacher_hidden: np.ndarray | None = None,
    teacher_weight: np.ndarray | None = None,
    teacher_logits: np.ndarray | None = None,
    student_ce_weight: float = 1.0,
    teacher_ce_weight: float | None = None,
    kl_weight: float = 0.0,
    kl_temperature: float = 1.0,
    ignore_index: int = -100,
    reduction: str = "mean",
    divergence: str = "forward_kl",
    alpha: float | None = None,
    beta: float | None = None,
    kernel_semantics: bool = True,
    grad_output: float = 1.0,
    teacher_grads: bool = True,
    grad_logits_dtype: str | None = None,
    student_norm_weight: np.ndarray | None = None,
    norm_eps: float = 1e-6,
    normed_dtype: str | None = None,
    fp8_operands: bool = False,
) -> dict:
    """Loss components and gradients, float64.

    ``mode`` is ``tied``, ``separate`` or ``precomputed``.  Returns a dict
    with ``loss``, ``student_ce``, ``teacher_ce``, ``kl`` (floats) and
    ``grad_student_hidden``, ``grad_weight`` and, where they exist,
    ``grad_teacher_hidden`` / ``grad_teacher_weight`` (teacher CE path only;
    pass ``teacher_grads=False`` for the separate student-only mode).
    """
    hs = np.asarray(student_hidden, dtype=np.float64)
    W = np.asarray(weight, dtype=np.float64)
    x_in = r_norm = g_norm = None
    if student_norm_weight is not None:
        # the student's RMSNorm (reference test/benchmark/src/core.py:13-14);
        # y optionally rounded to the dtype the kernels store it in
        x_in = hs
        g_norm = np.asarray(student_norm_weight, dtype=np.float64)
        r_norm = 1.0 / np.sqrt((x_in * x_in).mean(axis=1) + float(norm_eps))
        hs = round_to(x_in * r_norm[:, None] * g_norm[None, :], normed_dtype)
    y = np.asarray(labels, dtype=np.int64)
    N, V = hs.shape[0], W.shape[0]
    w_t = (1.0 if mode == "tied" else 0.0) if teacher_ce_weight is None else float(teacher_ce_weight)
    if mode == "tied":
        ht = np.asarray(teacher_hidden, dtype=np.float64)
        Wt = W
    elif mode == "separate":
        ht = np.asarray(teacher_hidden, dtype=np.float64)
        Wt = np.asarray(teacher_weight, dtype=np.float64)
    elif teacher_logits is not None:
        ht = Wt = None
    else:
        ht = np.asarray(teacher_hidden, dtype=np.float64)
        Wt = np.asarray(teacher_weight, dtype=np.float64)
    if fp8_operands:
        # the fp8 logits GEMM: its operands rounded per row to E4M3 (the
        # student's, and the tied teacher's, which shares W); the gradient
        # GEMMs keep the unrounded operands
        W8, hs8 = quantize_rows_e4m3(W), quantize_rows_e4m3(hs)
        x_s = hs8 @ W8.T
        if mode == "tied":
            x_t = quantize_rows_e4m3(ht) @ W8.T
        elif ht is None:
            x_t = np.asarray(teacher_logits, dtype=np.float64)
        else:
            x_t = ht @ Wt.T
    else:
        x_s = hs @ W.T
        x_t = np.asarray(teacher_logits, dtype=np.float64) if (ht is None) else ht @ Wt.T

    ignored = y == ignore_index
    y_eff = np.where((y >= 0) & (y < V), y, 0)
    onehot = np.zeros((N, V))
    onehot[np.arange(N), y_eff] = 1.0
    lse_s = np.log(np.exp(x_s - x_s.max(1, keepdims=True)).sum(1)) + x_s.max(1)
    lse_t = np.log(np.exp(x_t - x_t.max(1, keepdims=True)).sum(1)) + x_t.max(1)
    ce_s_rows = np.where(ignored, 0.0, lse_s - x_s[np.arange(N), y_eff])
    ce_t_rows = np.where(ignored, 0.0, lse_t - x_t[np.arange(N), y_eff])

    T = float(kl_temperature)
    d_rows, dz = divergence_value_and_grad(x_t / T, x_s / T, divergence, alpha, beta)
    div_on = (kl_weight != 0.0) or not kernel_semantics
    d_rows = np.where(ignored | (not div_on), 0.0, T * T * d_rows)

    count = int((~ignored).sum())
    scale = 1.0 / max(count, 1) if reduction == "mean" else 1.0
    ce_s = ce_s_rows.sum() * scale
    ce_t = ce_t_rows.sum() * scale if w_t != 0.0 else 0.0
    kl = d_rows.sum() * scale
    loss = student_ce_weight * ce_s + w_t * ce_t + kl_weight * kl

    g = grad_output * scale
    keep = (~ignored)[:, None].astype(np.float64)
    if grad_logits_dtype is not None:
        x_s = round_to(x_s, grad_logits_dtype)
        if ht is not None:  # given teacher logits are used as they come
            x_t = round_to(x_t, grad_logits_dtype)
        lse_s = np.log(np.exp(x_s - x_s.max(1, keepdims=True)).sum(1)) + x_s.max(1)
        lse_t = np.log(np.exp(x_t - x_t.max(1, keepdims=True)).sum(1)) + x_t.max(1)
        _, dz = divergence_value_and_grad(x_t / T, x_s / T, divergence, alpha, beta)
    p_s = np.exp(x_s - lse_s[:, None])
    p_t = np.exp(x_t - lse_t[:, None])
    dl_s = g * keep * (student_ce_weight * (p_s - onehot) + kl_weight * T * dz)
    dl_t = g * keep * (w_t * (p_t - onehot))
    out = {
        "loss": float(loss), "student_ce": float(ce_s), "teacher_ce": float(ce_t), "kl": float(kl),
        "count": count, "dlogits_student": dl_s, "dlogits_teacher": dl_t,
        "grad_student_hidden": dl_s @ W,
    }
    if mode == "tied":
        out["grad_weight"] = dl_s.T @ hs + dl_t.T @ ht
        out["grad_teacher_hidden"] = dl_t @ W
    else:
        out["grad_weight"] = dl_s.T @ hs
        if mode == "separate" and teacher_grads:
            out["grad_teacher_hidden"] = dl_t @ Wt
            out["grad_teacher_weight"] = dl_t.T @ ht
    if x_in is not None:
        # through the RMSNorm: dy -> dw = sum_t dy x r, dx = r (w dy) - x r^3 <w dy, x> / H
        dy = out["grad_student_hidden"]
        out["grad_student_norm_weight"] = (dy * x_in * r_norm[:, None]).sum(axis=0)
        gdy = dy * g_norm[None, :]
        c = (gdy * x_in).sum(axis=1)
        out["grad_student_hidden"] = (r_norm[:, None] * gdy
                                      - x_in * (r_norm ** 3 * c / x_in.shape[1])[:, None])
    return out
