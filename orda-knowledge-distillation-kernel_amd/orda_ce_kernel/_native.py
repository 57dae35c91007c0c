"""ctypes binding of liborda_ce.so (the C ABI in include/orda_ce.h).

The library is built in-tree by ``csrc/Makefile`` into ``_lib/liborda_ce.so``.
``ORDA_CE_LIBRARY`` may point at another build.  Nothing here falls back to
another implementation: if the library is missing, :func:`library` raises and
the HIP path reports it.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

__all__ = [
    "ABI_VERSION", "PlanInfo", "Problem", "Tensors", "library", "plan_info", "library_path", "forward", "forward_static", "backward",
    "saved_bytes", "forward_workspace_bytes", "backward_workspace_bytes", "gemm_abt", "gemm",
    "MODE", "DTYPE", "FLAG", "KERNEL_CLASSES", "timing_enable", "timing_collect",
]

ABI_VERSION = 4

MODE = {"tied": 0, "separate": 1, "precomputed_logits": 2, "precomputed_hidden": 3, "topk": 4}
DTYPE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
FLAG = {
    "need_grad_student_hidden": 1 << 0,
    "need_grad_weight": 1 << 1,
    "need_grad_teacher_hidden": 1 << 2,
    "need_grad_teacher_weight": 1 << 3,
    "compute_teacher_ce": 1 << 4,
    "compute_divergence": 1 << 5,
    "reduction_sum": 1 << 6,
    "grads_in_forward": 1 << 7,
    "student_rmsnorm": 1 << 8,
    "need_grad_student_norm_weight": 1 << 9,
    "fp8_logits": 1 << 10,
}


class Problem(ctypes.Structure):
    """orda_problem_t"""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("logits_dtype", ctypes.c_int32),
        ("n_rows", ctypes.c_int64),
        ("vocab", ctypes.c_int64),
        ("hidden", ctypes.c_int64),
        ("teacher_hidden", ctypes.c_int64),
        ("ignore_index", ctypes.c_int64),
        ("vocab_chunk", ctypes.c_int64),
        ("flags", ctypes.c_uint32),
        ("divergence", ctypes.c_int32),
        ("temperature", ctypes.c_float),
        ("student_ce_weight", ctypes.c_float),
        ("teacher_ce_weight", ctypes.c_float),
        ("kl_weight", ctypes.c_float),
        ("div_alpha", ctypes.c_float),
        ("div_beta", ctypes.c_float),
        ("grad_hidden_splits", ctypes.c_int32),
        ("token_chunk", ctypes.c_int64),
        ("topk", ctypes.c_int64),
        ("norm_dim", ctypes.c_int64),
        ("norm_eps", ctypes.c_float),
    ]


class PlanInfo(ctypes.Structure):
    """orda_plan_info_t"""

    _fields_ = [
        ("grads_in_forward", ctypes.c_int32),
        ("table_entry", ctypes.c_int32),
        ("teacher_class", ctypes.c_int32),
        ("scan_engine", ctypes.c_int32),
        ("token_chunk", ctypes.c_int64),
        ("n_token_chunks", ctypes.c_int64),
        ("chunk_scale", ctypes.c_int32),
        ("scan_tokens_per_tile", ctypes.c_int32),
        ("scan_workgroups", ctypes.c_int32),
        ("grad_hidden_splits", ctypes.c_int32),
        ("grad_teacher_hidden_splits", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("vocab_rows_per_split", ctypes.c_int64),
        ("vocab_chunk", ctypes.c_int64),
        ("forward_workspace_bytes", ctypes.c_uint64),
        ("backward_workspace_bytes", ctypes.c_uint64),
    ]


KERNEL_CLASSES = ("scan", "rows", "dlogits", "gemm_w", "gemm_h", "aux")


class Timing(ctypes.Structure):
    """orda_timing_t"""

    _fields_ = [
        ("launches", ctypes.c_int32 * 6),
        ("milliseconds", ctypes.c_double * 6),
        ("algorithmic_flops", ctypes.c_double * 6),
        ("executed_flops", ctypes.c_double * 6),
    ]


class Tensors(ctypes.Structure):
    """orda_tensors_t"""

    _fields_ = [
        (name, ctypes.c_void_p)
        for name in (
            "student_hidden", "weight", "teacher_hidden", "teacher_weight", "teacher_logits", "labels",
            "out_loss", "out_student_ce", "out_teacher_ce", "out_kl", "saved", "grad_output",
            "grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight",
            "teacher_topk_indices", "teacher_topk_logprobs",
            "student_norm_weight", "grad_student_norm_weight",
        )
    ]


_LOCK = threading.Lock()
_LIB = None


def library_path() -> Path:
    env = os.environ.get("ORDA_CE_LIBRARY")
    if env:
        return Path(env)
    return Path(__file__).resolve().parent / "_lib" / "liborda_ce.so"


def library() -> ctypes.CDLL:
    """Load (once) and return liborda_ce.so; raise RuntimeError if missing."""
    global _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"liborda_ce.so not found at {path}; build it with `make -C csrc` "
                "(or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(path))
        P, T = ctypes.POINTER(Problem), ctypes.POINTER(Tensors)
        lib.orda_abi_version.restype = ctypes.c_int
        lib.orda_abi_version.argtypes = []
        lib.orda_last_error.restype = ctypes.c_char_p
        lib.orda_last_error.argtypes = []
        for name in ("orda_saved_bytes", "orda_forward_workspace_bytes", "orda_backward_workspace_bytes"):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_size_t
            fn.argtypes = [P]
        for name in ("orda_forward", "orda_backward"):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [P, T, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.orda_plan_info.restype = ctypes.c_int
        lib.orda_plan_info.argtypes = [P, ctypes.POINTER(PlanInfo)]
        lib.orda_forward_static.restype = ctypes.c_int
        lib.orda_forward_static.argtypes = [P, T, ctypes.c_void_p]
        lib.orda_gemm_abt.restype = ctypes.c_int
        lib.orda_gemm_abt.argtypes = [
            ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ]
        lib.orda_gemm.restype = ctypes.c_int
        lib.orda_gemm.argtypes = [
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
            ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.orda_scale_gradient.restype = ctypes.c_int
        lib.orda_scale_gradient.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                            ctypes.c_void_p]
        lib.orda_timing_enable.restype = ctypes.c_int
        lib.orda_timing_enable.argtypes = [ctypes.c_int]
        lib.orda_timing_collect.restype = ctypes.c_int
        lib.orda_timing_collect.argtypes = [ctypes.POINTER(Timing)]
        version = lib.orda_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"liborda_ce.so ABI version {version}, expected {ABI_VERSION}")
        _LIB = lib
        return lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = library().orda_last_error().decode("utf-8", "replace")
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def _size(fn_name: str, problem: Problem) -> int:
    n = getattr(library(), fn_name)(ctypes.byref(problem))
    if n == 0:
        _check(-1, fn_name)
    return int(n)


def saved_bytes(problem: Problem) -> int:
    return _size("orda_saved_bytes", problem)


def forward_workspace_bytes(problem: Problem) -> int:
    return _size("orda_forward_workspace_bytes", problem)


def backward_workspace_bytes(problem: Problem) -> int:
    return _size("orda_backward_workspace_bytes", problem)


def plan_info(problem: Problem) -> dict:
    """The launch plan orda_forward would use for ``problem`` (host only)."""
    info = PlanInfo()
    _check(library().orda_plan_info(ctypes.byref(problem), ctypes.byref(info)), "orda_plan_info")
    return {name: getattr(info, name) for name, _ in PlanInfo._fields_ if name != "reserved"}


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def forward(problem: Problem, tensors: Tensors, workspace: torch.Tensor) -> None:
    rc = library().orda_forward(
        ctypes.byref(problem), ctypes.byref(tensors), workspace.data_ptr(), workspace.numel(),
        _stream(workspace.device),
    )
    _check(rc, "orda_forward")


def forward_static(problem: Problem, tensors: Tensors, device: torch.device) -> None:
    """orda_forward on the library's static scratch (no workspace, no
    allocation); raises RuntimeError when the problem does not fit it."""
    with torch.cuda.device(device):
        rc = library().orda_forward_static(ctypes.byref(problem), ctypes.byref(tensors), _stream(device))
    _check(rc, "orda_forward_static")


STATIC_SCRATCH_BYTES = 64 << 20  # ORDA_STATIC_SCRATCH_BYTES


def backward(problem: Problem, tensors: Tensors, workspace: torch.Tensor | None, device: torch.device) -> None:
    ptr = workspace.data_ptr() if workspace is not None else None
    size = workspace.numel() if workspace is not None else 0
    rc = library().orda_backward(ctypes.byref(problem), ctypes.byref(tensors), ptr, size, _stream(device))
    _check(rc, "orda_backward")


def scale_gradient_(grad: torch.Tensor, factor: torch.Tensor) -> None:
    """``grad *= factor`` in place on the library's scaling kernel (``factor``
    a 1-element fp32 tensor on grad's device, read there: no host
    synchronisation, and factor 1 leaves ``grad`` untouched)."""
    if grad.dtype not in DTYPE or not grad.is_contiguous():
        raise ValueError("grad must be a contiguous bf16, fp16 or fp32 tensor")
    if factor.dtype != torch.float32 or factor.numel() != 1 or factor.device != grad.device:
        raise ValueError("factor must be a 1-element float32 tensor on grad's device")
    rc = library().orda_scale_gradient(DTYPE[grad.dtype], grad.data_ptr(), grad.numel(), factor.data_ptr(),
                                       _stream(grad.device))
    _check(rc, "orda_scale_gradient")


def gemm_abt(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """C = a @ b.T on the library's MFMA engine (a [M, K], b [N, K])."""
    if a.dtype != b.dtype or a.dtype not in DTYPE:
        raise ValueError("a and b must share a dtype among bf16, fp16, fp32")
    a = a.contiguous()
    b = b.contiguous()
    M, K = a.shape
    N = b.shape[0]
    c = torch.empty((M, N), dtype=a.dtype, device=a.device)
    rc = library().orda_gemm_abt(DTYPE[a.dtype], M, N, K, a.data_ptr(), b.data_ptr(), c.data_ptr(), _stream(a.device))
    _check(rc, "orda_gemm_abt")
    return c


def gemm(a: torch.Tensor, b: torch.Tensor, *, a_mn: bool = False, b_mn: bool = False, splits: int = 1) -> torch.Tensor:
    """C = op(a) @ op(b).T on the library's general GEMM.

    ``a`` is [M, K] (``a_mn=False``) or stored [K, M] (``a_mn=True``: the
    operand is read MN-major, i.e. C = a.T @ ...); likewise ``b`` is [N, K]
    or stored [K, N].  ``splits`` > 1 splits K into fp32 partials summed in a
    fixed order (MN-major a and b only)."""
    if a.dtype != b.dtype or a.dtype not in DTYPE:
        raise ValueError("a and b must share a dtype among bf16, fp16, fp32")
    a = a.contiguous()
    b = b.contiguous()
    M, K = (a.shape[1], a.shape[0]) if a_mn else (a.shape[0], a.shape[1])
    N, Kb = (b.shape[1], b.shape[0]) if b_mn else (b.shape[0], b.shape[1])
    if Kb != K:
        raise ValueError(f"inner dimensions differ: {K} vs {Kb}")
    c = torch.empty((M, N), dtype=a.dtype, device=a.device)
    ws = None
    if splits > 1:
        ws = torch.empty(splits * M * N * 4 + 512, dtype=torch.uint8, device=a.device)
    rc = library().orda_gemm(
        DTYPE[a.dtype], int(a_mn), int(b_mn), M, N, K, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
        c.data_ptr(), N, int(splits), ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        _stream(a.device),
    )
    _check(rc, "orda_gemm")
    return c


def timing_enable(enable: bool = True) -> None:
    """Start/stop per-launch hipEvent timing inside the library (this thread)."""
    library().orda_timing_enable(1 if enable else 0)


def timing_collect() -> dict:
    """Per kernel class: launches, ms, algorithmic and executed GEMM flops
    since the last enable/collect (waits for the recorded events)."""
    t = Timing()
    _check(library().orda_timing_collect(ctypes.byref(t)), "orda_timing_collect")
    return {
        name: {
            "launches": int(t.launches[i]),
            "ms": float(t.milliseconds[i]),
            "algorithmic_flops": float(t.algorithmic_flops[i]),
            "executed_flops": float(t.executed_flops[i]),
        }
        for i, name in enumerate(KERNEL_CLASSES)
    }
