"""Runtime policy: native-library probe and compute-dtype selection.

``default_compute_dtype`` follows the reference (``_runtime.py:41-80``):
an active autocast dtype wins; otherwise bf16 if any input is bf16, then
fp16, then fp32; with no floating input, bf16 on HIP.
"""
from __future__ import annotations

import torch

__all__ = ["HAS_NATIVE", "default_compute_dtype", "is_hip", "native_error", "supports_bfloat16"]


def _probe_native():
    try:
        from . import _native

        _native.library()
        return True, None
    except Exception as exc:  # noqa: BLE001 - the message is surfaced on use
        return False, str(exc)


HAS_NATIVE, _NATIVE_ERROR = _probe_native()


def native_error() -> str | None:
    """Why liborda_ce.so could not be loaded (None when it loaded)."""
    return _NATIVE_ERROR


def is_hip() -> bool:
    return getattr(torch.version, "hip", None) is not None


def supports_bfloat16(device: torch.device | None = None) -> bool:
    """bf16 is native on every HIP device; elsewhere ask torch."""
    if is_hip():
        return True
    if device is not None and device.type != "cuda":
        return False
    if not torch.cuda.is_available():
        return False
    try:
        return bool(torch.cuda.is_bf16_supported())
    except (AttributeError, RuntimeError):
        return False


def _autocast_dtype(device: torch.device | None) -> torch.dtype | None:
    device_type = device.type if device is not None else "cuda"
    try:
        enabled = torch.is_autocast_enabled(device_type)
    except TypeError:
        enabled = torch.is_autocast_enabled()
    if not enabled:
        return None
    try:
        dtype = torch.get_autocast_dtype(device_type)
    except (AttributeError, TypeError):
        dtype = torch.get_autocast_gpu_dtype()
    if dtype == torch.bfloat16 and supports_bfloat16(device):
        return torch.bfloat16
    if dtype == torch.float16:
        return torch.float16
    return None


def default_compute_dtype(*tensors: torch.Tensor) -> torch.dtype:
    tensors = [t for t in tensors if isinstance(t, torch.Tensor)]
    device = tensors[0].device if tensors else None
    autocast = _autocast_dtype(device)
    if autocast is not None:
        return autocast
    floats = {t.dtype for t in tensors if t.is_floating_point()}
    if torch.bfloat16 in floats:
        return torch.bfloat16 if supports_bfloat16(device) else torch.float16
    if torch.float16 in floats:
        return torch.float16
    if torch.float32 in floats:
        return torch.float32
    return torch.bfloat16 if is_hip() else torch.float16
