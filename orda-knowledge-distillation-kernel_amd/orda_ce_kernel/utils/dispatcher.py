"""Chunk dispatcher with out-of-memory retry (reference ``utils/dispatcher.py``).

Behaviour kept from the reference because callers and tests depend on it:

* an explicit ``num_chunks`` or ``chunk_size`` makes one call
  (``:187-216``);
* otherwise the chunk count starts from :func:`resolve_chunk_size` (or a
  larger cached count for the same problem signature) and doubles after each
  device OOM, up to ``min(BT, max_chunks)`` with ``max_chunks`` defaulting to
  ``2 * max(1, BT // 512)`` (``:218-293``);
* the successful count is cached under a thread-safe, bounded cache keyed by
  shapes, dtypes, devices and mode (``:33-80``).
"""
from __future__ import annotations

import threading

import torch

from ._autotune import _is_oom_error
from .resolver import DEFAULT_MAX_FUSED_SIZE

__all__ = ["clear_chunk_cache", "dynamic_chunk", "get_chunk_cache"]


def _chunk_size_from_num_chunks(BT: int, num_chunks: int) -> int:
    return -(-int(BT) // int(num_chunks))


def _tensor_sig(tensor):
    if tensor is None:
        return None
    return (tuple(tensor.shape), tensor.dtype, tensor.device.type, tensor.device.index)


def _cache_key(
    BT: int,
    V: int,
    H: int,
    student_hidden: torch.Tensor,
    weight: torch.Tensor,
    teacher_mode: str = "tied",
    max_fused_size: int = DEFAULT_MAX_FUSED_SIZE,
    max_chunks: int | None = None,
    teacher_hidden: torch.Tensor | None = None,
    teacher_weight: torch.Tensor | None = None,
    logits_teacher: torch.Tensor | None = None,
    compute_kl: bool = True,
):
    """Signature of a problem for the chunk-count cache."""
    dev = student_hidden.device
    return (
        int(BT), int(V), int(H), dev.type, dev.index,
        student_hidden.dtype, weight.dtype, teacher_mode,
        int(max_fused_size), max_chunks, bool(compute_kl),
        _tensor_sig(teacher_hidden), _tensor_sig(teacher_weight), _tensor_sig(logits_teacher),
    )


_CACHE_LOCK = threading.Lock()
_MAX_CHUNK_CACHE_SIZE = 1024
_cached_num_chunks: dict = {}


def clear_chunk_cache() -> None:
    with _CACHE_LOCK:
        _cached_num_chunks.clear()


def get_chunk_cache() -> dict:
    """A copy of the cache (mutating it does not touch the cache)."""
    with _CACHE_LOCK:
        return dict(_cached_num_chunks)


def _resolve_kernel_fn(teacher_mode: str):
    if teacher_mode == "tied":
        from ..ops.tied_teacher import tied_distillation_loss

        return tied_distillation_loss
    if teacher_mode == "separate":
        from ..ops.separate_teacher import separate_distillation_loss

        return separate_distillation_loss
    if teacher_mode == "precomputed":
        from ..ops.precomputed_teacher import precomputed_distillation_loss

        return precomputed_distillation_loss
    raise ValueError(f"teacher_mode must be 'tied', 'separate', or 'precomputed', got {teacher_mode!r}")


def _call_kernel_fn(
    kernel_fn,
    teacher_mode: str,
    student_hidden,
    teacher_hidden,
    weight,
    labels,
    *,
    student_ce_weight,
    ignore_index,
    reduction,
    chunk_size,
    use_fp32_accum,
    kl_weight,
    kl_temperature,
    max_chunks,
    max_fused_size,
    autotune,
    teacher_weight,
    logits_teacher,
    teacher_ce_weight,
    validate_labels,
    divergence=None,
):
    """Call a mode entry point with its own positional layout
    (reference ``utils/dispatcher.py:99-152``)."""
    kwargs = dict(
        student_ce_weight=student_ce_weight,
        ignore_index=ignore_index,
        reduction=reduction,
        chunk_size=chunk_size,
        use_fp32_accum=use_fp32_accum,
        kl_weight=kl_weight,
        kl_temperature=kl_temperature,
        teacher_ce_weight=teacher_ce_weight,
        max_chunks=max_chunks,
        max_fused_size=max_fused_size,
        autotune=autotune,
        validate_labels=validate_labels,
    )
    if divergence is not None:
        kwargs["divergence"] = divergence
    if teacher_mode == "tied":
        return kernel_fn(student_hidden, teacher_hidden, weight, labels, **kwargs)
    if teacher_mode == "separate":
        return kernel_fn(student_hidden, teacher_hidden, weight, teacher_weight, labels, **kwargs)
    return kernel_fn(
        student_hidden, weight, logits_teacher, labels,
        teacher_hidden=teacher_hidden, teacher_weight=teacher_weight, **kwargs,
    )


@torch._dynamo.disable
def dynamic_chunk(
    student_hidden: torch.Tensor,
    teacher_hidden: torch.Tensor | None,
    weight: torch.Tensor,
    labels: torch.Tensor,
    student_ce_weight: float = 1.0,
    ignore_index: int = -100,
    reduction: str = "mean",
    chunk_size=None,
    num_chunks: int | None = None,
    use_fp32_accum: bool | None = None,
    kl_weight: float = 0.0,
    kl_temperature: float = 1.0,
    max_chunks: int | None = None,
    max_fused_size: int = DEFAULT_MAX_FUSED_SIZE,
    autotune: bool = False,
    teacher_mode: str | None = None,
    teacher_weight: torch.Tensor | None = None,
    logits_teacher: torch.Tensor | None = None,
    teacher_ce_weight: float | None = None,
    validate_labels: bool = True,
    divergence=None,
):
    """Run one mode entry point, retrying with more chunks after an OOM."""
    from .resolver import _is_auto_chunk_size, resolve_chunk_size

    BT, H = student_hidden.shape
    V = weight.shape[0]
    mode = "tied" if teacher_mode is None else teacher_mode
    kernel_fn = _resolve_kernel_fn(mode)

    def call(cs):
        return _call_kernel_fn(
            kernel_fn, mode, student_hidden, teacher_hidden, weight, labels,
            student_ce_weight=student_ce_weight, ignore_index=ignore_index, reduction=reduction,
            chunk_size=cs, use_fp32_accum=use_fp32_accum, kl_weight=kl_weight,
            kl_temperature=kl_temperature, max_chunks=max_chunks, max_fused_size=max_fused_size,
            autotune=autotune, teacher_weight=teacher_weight, logits_teacher=logits_teacher,
            teacher_ce_weight=teacher_ce_weight, validate_labels=validate_labels, divergence=divergence,
        )

    if num_chunks is not None or not _is_auto_chunk_size(chunk_size):
        cs, _ = resolve_chunk_size(BT, chunk_size, max_chunks=max_chunks, num_chunks=num_chunks)
        return call(cs)

    limit = max_chunks if max_chunks is not None else 2 * max(1, BT // 512)
    _, start = resolve_chunk_size(BT, chunk_size, V=V, max_chunks=limit)
    key = _cache_key(
        BT, V, H, student_hidden, weight, mode, max_fused_size, limit,
        teacher_hidden, teacher_weight, logits_teacher, compute_kl=float(kl_weight) != 0.0,
    )
    with _CACHE_LOCK:
        cached = _cached_num_chunks.get(key)
    n = min(max(cached or start, start), BT, limit)

    while True:
        try:
            result = call(_chunk_size_from_num_chunks(BT, n))
        except Exception as exc:
            if not _is_oom_error(exc):
                raise
            torch.cuda.empty_cache()
            if n >= BT or n >= limit:
                accum = "enabled" if use_fp32_accum else "disabled"
                raise RuntimeError(
                    f"Out of memory with max_chunks={limit}, fp32_accum={accum}\n"
                    f"BT={BT}, V={V}, H={H}\n"
                    f"Options:\n"
                    f"  - Increase max_chunks to {limit * 2}\n"
                    f"  - Enable fp32 grad-weight accumulation if numerical stability is required\n"
                    f"  - Reduce batch size or sequence length"
                ) from exc
            n = min(n * 2, BT, limit)
            continue
        with _CACHE_LOCK:
            if key not in _cached_num_chunks and len(_cached_num_chunks) >= _MAX_CHUNK_CACHE_SIZE:
                _cached_num_chunks.clear()
            _cached_num_chunks[key] = n
        return result
