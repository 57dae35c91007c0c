"""orda_ce_kernel for MI355X: fused LM-head cross-entropy + knowledge
distillation loss on hand-written CDNA4 (gfx950) HIP kernels.

Drop-in for the reference package of the same name: same public names,
signatures, defaults and errors.  The compute path is ``liborda_ce.so``
(C ABI in ``include/orda_ce.h``) loaded through ctypes.
"""
import torch

from ._runtime import HAS_NATIVE
from .api import (
    DistillationLoss,
    DistillationLossOutput,
    KernelConfig,
    PrecomputedTeacher,
    SeparateTeacher,
    StudentRMSNorm,
    TiedTeacher,
    TopKTeacher,
    distillation_loss,
)


from . import compiled  # noqa: E402,F401  (torch.compile-friendly entry; not in __all__)

# TopKTeacher (a top-k precomputed teacher) and StudentRMSNorm (the student's
# final RMSNorm fused in front of the loss) are importable from here but kept
# out of __all__, which stays the reference's public surface.


def is_available() -> bool:
    """True when the HIP kernels can be selected (library loaded and a HIP
    device present)."""
    return bool(HAS_NATIVE and torch.cuda.is_available())


__all__ = [
    "DistillationLoss",
    "DistillationLossOutput",
    "KernelConfig",
    "PrecomputedTeacher",
    "SeparateTeacher",
    "TiedTeacher",
    "distillation_loss",
    "is_available",
]
