"""Divergences for the distillation term.

The reference implements one: forward KL, ``T^2 * sum p_t (log p_t - log p_s)``
(reference ``ops/tied_teacher.py:182,189``, ``api.py:317-322``).  This module
adds fourteen more behind the ``divergence=`` keyword, whose default keeps
forward KL.  Every divergence D(p_t || p_s) is computed on the
temperature-scaled distributions ``p = softmax(logits / T)``, multiplied by
``T^2`` like the reference's KL, masked on ignored rows and reduced like the
reference's ``kl`` component.  Gradients flow to the student only; the
teacher distribution is detached, as in the reference.

=================  =========================================================  ==========
name               D(p_t || p_s)                                              parameters
=================  =========================================================  ==========
forward_kl         sum p_t log(p_t / p_s)                                     --
reverse_kl         sum p_s log(p_s / p_t)                                     --
symmetric_kl       forward_kl + reverse_kl (Jeffreys)                         --
soft_target_ce     -sum p_t log p_s                                           --
hellinger          1 - sum sqrt(p_t p_s)   (squared Hellinger)                --
bhattacharyya      -log sum sqrt(p_t p_s)                                     --
renyi              log(sum p_t^a p_s^(1-a)) / (a - 1)                         alpha (0.5)
amari_alpha        (1 - sum p_t^a p_s^(1-a)) / (a (1 - a))                    alpha (0.5)
chi_squared        sum (p_t - p_s)^2 / p_s   (Pearson)                        --
squared_l2         sum (p_t - p_s)^2                                          --
ab                 -1/(ab) sum(p_t^a p_s^b - a/(a+b) p_t^(a+b)                alpha, beta (0.5, 0.5)
                   - b/(a+b) p_s^(a+b))   (Cichocki-Cruces-Amari 2011)
jsd                b KL(p_t||m) + (1-b) KL(p_s||m), m = b p_t + (1-b) p_s      beta (0.5)
                   (generalized JSD of Agarwal et al. 2024; b = 0.5 is JSD)
skew_forward_kl    KL(p_t || a p_t + (1-a) p_s)   (DistiLLM, Ko et al. 2024)  alpha (0.1)
skew_reverse_kl    KL(p_s || a p_s + (1-a) p_t)   (DistiLLM)                  alpha (0.1)
tvd                1/2 sum |p_t - p_s|                                        --
=================  =========================================================  ==========
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

__all__ = ["DIVERGENCES", "Divergence", "resolve_divergence", "divergence_rows_torch"]

# name -> (ABI code, default alpha, default beta)
DIVERGENCES: dict[str, tuple[int, float | None, float | None]] = {
    "forward_kl": (0, None, None),
    "reverse_kl": (1, None, None),
    "symmetric_kl": (2, None, None),
    "soft_target_ce": (3, None, None),
    "hellinger": (4, None, None),
    "bhattacharyya": (5, None, None),
    "renyi": (6, 0.5, None),
    "amari_alpha": (7, 0.5, None),
    "chi_squared": (8, None, None),
    "squared_l2": (9, None, None),
    "ab": (10, 0.5, 0.5),
    "jsd": (11, None, 0.5),
    "skew_forward_kl": (12, 0.1, None),
    "skew_reverse_kl": (13, 0.1, None),
    "tvd": (14, None, None),
}

# Divergences whose value needs normalised per-element probabilities, so the
# fused kernels make a second pass over the logits for them.
TWO_PASS = frozenset({"jsd", "skew_forward_kl", "skew_reverse_kl", "tvd"})


@dataclass(frozen=True)
class Divergence:
    """A divergence name with its parameters (``None`` = the default)."""

    name: str = "forward_kl"
    alpha: float | None = None
    beta: float | None = None

    @property
    def code(self) -> int:
        return DIVERGENCES[self.name][0]


def resolve_divergence(divergence) -> Divergence:
    """Normalise ``divergence`` (a name, a :class:`Divergence` or None) and
    check its parameters; raises ``ValueError`` on a bad name or value."""
    if divergence is None:
        return Divergence()
    if isinstance(divergence, str):
        divergence = Divergence(divergence)
    if not isinstance(divergence, Divergence):
        raise ValueError(f"divergence must be a name or a Divergence, got {type(divergence).__name__}")
    if divergence.name not in DIVERGENCES:
        raise ValueError(f"divergence must be one of {sorted(DIVERGENCES)}, got {divergence.name!r}")
    _, da, db = DIVERGENCES[divergence.name]
    alpha = da if divergence.alpha is None else float(divergence.alpha)
    beta = db if divergence.beta is None else float(divergence.beta)
    name = divergence.name
    if name == "renyi" and not (alpha > 0.0 and alpha != 1.0):
        raise ValueError(f"renyi divergence needs alpha > 0 and alpha != 1, got {alpha}")
    if name == "amari_alpha" and alpha in (0.0, 1.0):
        raise ValueError(f"amari_alpha divergence needs alpha not in (0, 1) endpoints, got {alpha}")
    if name == "ab" and (alpha == 0.0 or beta == 0.0 or alpha + beta == 0.0):
        raise ValueError(f"ab divergence needs alpha, beta and alpha + beta nonzero, got {alpha}, {beta}")
    if name == "jsd" and not (0.0 < beta < 1.0):
        raise ValueError(f"jsd divergence needs 0 < beta < 1, got {beta}")
    if name in ("skew_forward_kl", "skew_reverse_kl") and not (0.0 <= alpha < 1.0):
        raise ValueError(f"{name} needs 0 <= alpha < 1, got {alpha}")
    return Divergence(name, alpha, beta)


def _log(x: float) -> float:
    return math.log(x) if x > 0.0 else float("-inf")


def divergence_rows_torch(log_p_s: torch.Tensor, log_p_t: torch.Tensor, div: Divergence) -> torch.Tensor:
    """Per-row D(p_t || p_s) from row-normalised log-probabilities
    (``[rows, V]`` -> ``[rows]``), differentiable in ``log_p_s``."""
    name, a, b = div.name, div.alpha, div.beta
    p_s, p_t = log_p_s.exp(), log_p_t.exp()
    if name == "forward_kl":
        return (p_t * (log_p_t - log_p_s)).sum(-1)
    if name == "reverse_kl":
        return (p_s * (log_p_s - log_p_t)).sum(-1)
    if name == "symmetric_kl":
        return ((p_t - p_s) * (log_p_t - log_p_s)).sum(-1)
    if name == "soft_target_ce":
        return -(p_t * log_p_s).sum(-1)
    if name == "hellinger":
        return 1.0 - (0.5 * (log_p_t + log_p_s)).exp().sum(-1)
    if name == "bhattacharyya":
        return -torch.logsumexp(0.5 * (log_p_t + log_p_s), dim=-1)
    if name == "renyi":
        return torch.logsumexp(a * log_p_t + (1.0 - a) * log_p_s, dim=-1) / (a - 1.0)
    if name == "amari_alpha":
        return (1.0 - (a * log_p_t + (1.0 - a) * log_p_s).exp().sum(-1)) / (a * (1.0 - a))
    if name == "chi_squared":
        return (2.0 * log_p_t - log_p_s).exp().sum(-1) - 1.0
    if name == "squared_l2":
        return ((p_t - p_s) ** 2).sum(-1)
    if name == "ab":
        s = a + b
        terms = (
            (a * log_p_t + b * log_p_s).exp()
            - (a / s) * (s * log_p_t).exp()
            - (b / s) * (s * log_p_s).exp()
        )
        return -terms.sum(-1) / (a * b)
    if name == "jsd":
        log_m = torch.logaddexp(_log(b) + log_p_t, _log(1.0 - b) + log_p_s)
        return b * (p_t * (log_p_t - log_m)).sum(-1) + (1.0 - b) * (p_s * (log_p_s - log_m)).sum(-1)
    if name == "skew_forward_kl":
        log_m = torch.logaddexp(_log(a) + log_p_t, _log(1.0 - a) + log_p_s)
        return (p_t * (log_p_t - log_m)).sum(-1)
    if name == "skew_reverse_kl":
        log_m = torch.logaddexp(_log(a) + log_p_s, _log(1.0 - a) + log_p_t)
        return (p_s * (log_p_s - log_m)).sum(-1)
    if name == "tvd":
        return 0.5 * (p_t - p_s).abs().sum(-1)
    raise ValueError(f"unknown divergence {name!r}")
