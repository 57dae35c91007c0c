"""C ABI of liborda_ce.so on the CPU: the library loads, exports every
function include/orda_ce.h declares, its struct layouts match the ctypes
mirror (checked against a gcc-compiled probe of the header), and argument
validation fails with the documented codes -- no kernel is launched."""
from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from orda_ce_kernel import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "orda_ce.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(orda_[a-z_]+)\s*\(", text)))


def test_library_loads_with_matching_abi():
    lib = _native.library()
    assert lib.orda_abi_version() == _native.ABI_VERSION == 2


def test_every_declared_function_is_exported():
    names = _declared_functions()
    assert "orda_forward" in names and "orda_backward" in names
    lib = _native.library()
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", str(_native.library_path())], capture_output=True,
                             text=True, check=True).stdout
        exported = set(re.findall(r" T (orda_[a-z_]+)", out))
        assert set(names) <= exported


PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "orda_ce.h"
#define F(T, m) printf(#T "." #m " %zu\n", offsetof(T, m));
int main(void) {
  printf("orda_problem_t %zu\n", sizeof(orda_problem_t));
  printf("orda_tensors_t %zu\n", sizeof(orda_tensors_t));
  printf("orda_timing_t %zu\n", sizeof(orda_timing_t));
  F(orda_problem_t, n_rows) F(orda_problem_t, vocab_chunk) F(orda_problem_t, flags) F(orda_problem_t, divergence)
  F(orda_problem_t, temperature) F(orda_problem_t, div_beta) F(orda_problem_t, token_chunk)
  F(orda_tensors_t, labels) F(orda_tensors_t, saved) F(orda_tensors_t, grad_output)
  F(orda_tensors_t, grad_teacher_weight)
  F(orda_timing_t, milliseconds) F(orda_timing_t, executed_flops)
  printf("ORDA_DIV_COUNT %d\n", (int)ORDA_DIV_COUNT);
  printf("ORDA_K_COUNT %d\n", (int)ORDA_K_COUNT);
  return 0;
}
"""


def test_struct_layout_matches_the_header(tmp_path):
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not available")
    src = tmp_path / "probe.c"
    src.write_text(PROBE)
    exe = tmp_path / "probe"
    subprocess.run([gcc, "-std=c11", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                               check=True).stdout.splitlines())
    P, T, Ti = _native.Problem, _native.Tensors, _native.Timing
    assert int(got["orda_problem_t"]) == ctypes.sizeof(P)
    assert int(got["orda_tensors_t"]) == ctypes.sizeof(T)
    assert int(got["orda_timing_t"]) == ctypes.sizeof(Ti)
    for key, value in got.items():
        if "." not in key:
            continue
        struct, field = key.split(".")
        cls = {"orda_problem_t": P, "orda_tensors_t": T, "orda_timing_t": Ti}[struct]
        assert getattr(cls, field).offset == int(value), key
    assert int(got["ORDA_DIV_COUNT"]) == 15
    assert int(got["ORDA_K_COUNT"]) == len(_native.KERNEL_CLASSES)


def _problem(**kw):
    p = _native.Problem()
    p.abi_version = _native.ABI_VERSION
    p.mode = 0
    p.dtype = 0
    p.n_rows, p.vocab, p.hidden, p.teacher_hidden = 8192, 128256, 4096, 4096
    p.ignore_index = -100
    p.flags = 0x33
    p.temperature = 1.0
    p.student_ce_weight = p.teacher_ce_weight = p.kl_weight = 1.0
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_workspace_queries_for_the_headline_shape():
    p = _problem()
    saved = _native.saved_bytes(p)
    fwd = _native.forward_workspace_bytes(p)
    bwd = _native.backward_workspace_bytes(p)
    assert saved == 64 * 4 + 8 * 8192 * 4
    assert 0 < fwd < 64 << 20
    # backward staging is bounded: no [N x V] tensor (that alone is 2.1 GB)
    assert 0 < bwd < 1 << 30
    p.vocab_chunk = 2048
    assert _native.backward_workspace_bytes(p) < bwd


@pytest.mark.parametrize(
    "field, value, message",
    [
        ("abi_version", 1, "abi_version"),
        ("mode", 9, "unknown mode"),
        ("dtype", 7, "unknown dtype"),
        ("n_rows", 0, "must be > 0"),
        ("temperature", 0.0, "temperature"),
        ("kl_weight", -1.0, "weights"),
        ("divergence", 15, "unknown divergence"),
        ("hidden", 4100, "multiple of 8"),
    ],
)
def test_invalid_problems_are_rejected(field, value, message):
    p = _problem(**{field: value})
    with pytest.raises(ValueError, match=message):
        _native.forward_workspace_bytes(p)


def test_divergence_parameters_are_validated_by_the_library():
    for div, alpha, beta in ((6, 1.0, 0.0), (11, 0.0, 1.0), (10, 0.5, -0.5), (12, 1.0, 0.0)):
        with pytest.raises(ValueError):
            _native.forward_workspace_bytes(_problem(divergence=div, div_alpha=alpha, div_beta=beta))


def test_forward_rejects_missing_operands_without_launching():
    lib = _native.library()
    p = _problem()
    t = _native.Tensors()
    ws = ctypes.create_string_buffer(16)
    rc = lib.orda_forward(ctypes.byref(p), ctypes.byref(t), ctypes.addressof(ws), 16, None)
    assert rc == -1
    assert b"required" in lib.orda_last_error()


def test_gemm_entry_validates_shapes():
    lib = _native.library()
    assert lib.orda_gemm_abt(0, 0, 4, 8, None, None, None, None) == -1
    assert lib.orda_gemm_abt(0, 4, 4, 12, 16, 16, 16, None) == -1  # K not a multiple of 8 (bf16)
    # general entry: MN-major A needs M a multiple of 8; K-major needs K; splits in range
    assert lib.orda_gemm(0, 1, 0, 12, 16, 16, 16, 16, 16, 16, 16, 16, 1, None, 0, None) == -1
    assert lib.orda_gemm(0, 0, 0, 16, 16, 12, 16, 16, 16, 16, 16, 16, 1, None, 0, None) == -1
    assert lib.orda_gemm(0, 0, 0, 16, 16, 16, 16, 16, 16, 16, 16, 16, 0, None, 0, None) == -1
    assert lib.orda_gemm(0, 2, 0, 16, 16, 16, 16, 16, 16, 16, 16, 16, 1, None, 0, None) == -1
    assert b"a_mn" in lib.orda_last_error()


GIF = _native.FLAG["grads_in_forward"]


def test_grads_in_forward_plan_for_the_headline_shape():
    p = _problem(flags=0x33 | GIF)
    ws = _native.forward_workspace_bytes(p)
    # one token chunk of student + teacher logits (1024 tokens x V x 2 x bf16)
    # plus split-K partials and row state; far below an [N x V] tensor
    assert 1024 * 128256 * 2 * 2 < ws < 900 << 20
    p.token_chunk = 512
    assert _native.forward_workspace_bytes(p) < ws
    # the backward only scales the gradients: no workspace
    assert lib_backward_bytes(p) == 0


def lib_backward_bytes(p):
    return _native.library().orda_backward_workspace_bytes(ctypes.byref(p))


@pytest.mark.parametrize("divergence", [11, 12, 13, 14])
def test_grads_in_forward_plans_two_pass_divergences(divergence):
    """JSD, the skew KLs and TVD take the schedule too (their second pass
    reads the chunk's stored logits): the same one-chunk workspace."""
    p = _problem(flags=0x33 | GIF, div_alpha=0.1, div_beta=0.5, divergence=divergence)
    ws = _native.forward_workspace_bytes(p)
    assert 1024 * 128256 * 2 * 2 < ws < 900 << 20
    assert lib_backward_bytes(p) == 0


@pytest.mark.parametrize("mode", [2, 3])
def test_grads_in_forward_plans_precomputed_teachers(mode):
    """Precomputed teachers (logits in memory / frozen hidden + W) take the
    schedule too: one chunk of student and teacher logits, no teacher grads."""
    p = _problem(mode=mode, flags=0x23 | GIF, teacher_ce_weight=0.0, logits_dtype=0)
    ws = _native.forward_workspace_bytes(p)
    assert 1024 * 128256 * 2 * 2 < ws < 900 << 20
    assert lib_backward_bytes(p) == 0


def test_timing_hook_without_launches_reports_zeros():
    _native.timing_enable(True)
    rows = _native.timing_collect()
    _native.timing_enable(False)
    assert set(rows) == set(_native.KERNEL_CLASSES)
    assert all(r["launches"] == 0 for r in rows.values())
