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
    assert lib.orda_abi_version() == _native.ABI_VERSION == 4


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
  printf("orda_plan_info_t %zu\n", sizeof(orda_plan_info_t));
  F(orda_problem_t, n_rows) F(orda_problem_t, vocab_chunk) F(orda_problem_t, flags) F(orda_problem_t, divergence)
  F(orda_problem_t, temperature) F(orda_problem_t, div_beta) F(orda_problem_t, grad_hidden_splits)
  F(orda_problem_t, token_chunk) F(orda_problem_t, topk) F(orda_problem_t, norm_dim) F(orda_problem_t, norm_eps)
  F(orda_plan_info_t, token_chunk) F(orda_plan_info_t, grad_hidden_splits) F(orda_plan_info_t, vocab_rows_per_split)
  F(orda_plan_info_t, backward_workspace_bytes)
  F(orda_tensors_t, labels) F(orda_tensors_t, saved) F(orda_tensors_t, grad_output)
  F(orda_tensors_t, grad_teacher_weight) F(orda_tensors_t, teacher_topk_indices)
  F(orda_tensors_t, teacher_topk_logprobs) F(orda_tensors_t, student_norm_weight)
  F(orda_tensors_t, grad_student_norm_weight)
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
    P, T, Ti, Pi = _native.Problem, _native.Tensors, _native.Timing, _native.PlanInfo
    assert int(got["orda_plan_info_t"]) == ctypes.sizeof(Pi)
    assert int(got["orda_problem_t"]) == ctypes.sizeof(P)
    assert int(got["orda_tensors_t"]) == ctypes.sizeof(T)
    assert int(got["orda_timing_t"]) == ctypes.sizeof(Ti)
    for key, value in got.items():
        if "." not in key:
            continue
        struct, field = key.split(".")
        cls = {"orda_problem_t": P, "orda_tensors_t": T, "orda_timing_t": Ti, "orda_plan_info_t": Pi}[struct]
        assert getattr(cls, field).offset == int(value), key
    assert int(got["ORDA_DIV_COUNT"]) == 15
    assert int(got["ORDA_K_COUNT"]) == len(_native.KERNEL_CLASSES)


def _integration_structs():
    """The ctypes structs of INTEGRATION.md's reference-side binding: the
    class definitions of its first python block, executed alone (nothing in
    the block is loaded or called)."""
    import ast

    text = (ROOT / "INTEGRATION.md").read_text()
    section = text.split("### Binding a maintainer would add", 1)[1]
    code = section.split("```python", 1)[1].split("```", 1)[0]
    tree = ast.parse(code)
    keep = [n for n in tree.body if isinstance(n, ast.ClassDef)]
    ns = {"ctypes": ctypes}
    exec(compile(ast.Module(body=keep, type_ignores=[]), "INTEGRATION.md", "exec"), ns)  # noqa: S102
    return ns["Problem"], ns["Tensors"]


def test_integration_binding_matches_the_header(tmp_path):
    """Every field of the documented binding's Problem / Tensors sits at the
    header's offset, and both structs have the header's size (so a caller
    copying the snippet passes the whole struct the library reads)."""
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not available")
    P, T = _integration_structs()
    lines = []
    for cname, cls in (("orda_problem_t", P), ("orda_tensors_t", T)):
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{cname}.{field} %zu\\n", offsetof({cname}, {field}));')
    src = tmp_path / "probe_doc.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "orda_ce.h"\nint main(void) {\n'
                   + "\n".join(lines) + "\nreturn 0;\n}\n")
    exe = tmp_path / "probe_doc"
    subprocess.run([gcc, "-std=c11", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                               check=True).stdout.splitlines())
    assert int(got["orda_problem_t"]) == ctypes.sizeof(P)
    assert int(got["orda_tensors_t"]) == ctypes.sizeof(T)
    for cname, cls in (("orda_problem_t", P), ("orda_tensors_t", T)):
        for field, _ in cls._fields_:
            assert getattr(cls, field).offset == int(got[f"{cname}.{field}"]), f"{cname}.{field}"
    # and the package's own binding is the same layout
    for doc, pkg in ((P, _native.Problem), (T, _native.Tensors)):
        assert [f for f, _ in doc._fields_] == [f for f, _ in pkg._fields_]


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


_TOPK_FLAGS = 0x3 | 0x20 | 0x80  # both student gradients, divergence, gradients in forward


@pytest.mark.parametrize(
    "kw, message",
    [
        (dict(topk=0), "topk must be in"),
        (dict(topk=128257), "topk must be in"),
        (dict(flags=_TOPK_FLAGS | 0x10), "no teacher CE"),
        (dict(flags=_TOPK_FLAGS & ~0x80), "ORDA_GRADS_IN_FORWARD"),
        (dict(divergence=1), "forward KL and soft-target CE"),
    ],
)
def test_invalid_topk_problems_are_rejected(kw, message):
    p = _problem(mode=_native.MODE["topk"], flags=_TOPK_FLAGS, topk=64, teacher_ce_weight=0.0)
    for k, v in kw.items():
        setattr(p, k, v)
    with pytest.raises(ValueError, match=message):
        _native.forward_workspace_bytes(p)


def test_topk_plan_runs_the_student_ring_scan():
    """A top-k teacher's scan sees the student alone: the ring engine with
    256-token tiles; the workspace holds the ids' dlogits share ([chunk x k]
    fp32) and a row of log-sum-exps."""
    p = _problem(mode=_native.MODE["topk"], flags=_TOPK_FLAGS, topk=64, teacher_ce_weight=0.0, token_chunk=512)
    info = _native.plan_info(p)
    assert info["grads_in_forward"] == 1 and info["scan_engine"] == 1
    assert info["scan_tokens_per_tile"] == 256
    p.topk = 1
    small = _native.forward_workspace_bytes(p)
    p.topk = 65
    assert _native.forward_workspace_bytes(p) - small >= 64 * 4 * info["token_chunk"]


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
    p.token_chunk = 256  # requested chunk x 2 = 512 tokens
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


# ------------------------------------------------------------ launch table
def _cfg_problem(cfg):
    """orda_problem_t of a benchmark configuration, as the Python layer builds
    it for the default call (the dispatcher's auto chunk: 512 tokens)."""
    if cfg == "c2":
        return _problem(flags=0x33 | GIF, token_chunk=512)
    if cfg == "c3":  # separate, student-only Function (teacher CE off), reverse KL
        return _problem(mode=1, hidden=2048, teacher_hidden=4096, flags=0x23 | GIF, teacher_ce_weight=0.0,
                        divergence=1, temperature=2.0, token_chunk=512)
    if cfg == "c4":  # precomputed bf16 logits read in place
        return _problem(mode=2, flags=0x23 | GIF, teacher_ce_weight=0.0, logits_dtype=0, token_chunk=512)
    if cfg == "c5":
        return _problem(n_rows=32768, hidden=5120, teacher_hidden=5120, vocab=152064, flags=0x33 | GIF,
                        token_chunk=512)
    if cfg.endswith("f16"):  # the configuration in fp16
        q = _cfg_problem(cfg[:-3])
        q.dtype = q.logits_dtype = 1
        return q
    if cfg == "h8192":
        return _problem(hidden=8192, teacher_hidden=8192, flags=0x33 | GIF, token_chunk=512)
    if cfg == "h3584":
        return _problem(hidden=3584, teacher_hidden=3584, vocab=152064, flags=0x33 | GIF, token_chunk=512)
    raise ValueError(cfg)


@pytest.mark.parametrize("cfg, entry, chunk, splits, tclass", [
    ("c2", 0, 1024, 4, 0), ("c3", 1, 2048, 4, 1), ("c4", 2, 2048, 2, 2), ("c5", 3, 2048, 8, 0),
    ("c2f16", 4, 1024, 4, 0), ("c3f16", 5, 2048, 4, 1), ("c4f16", 6, 2048, 2, 2), ("c5f16", 7, 2048, 8, 0),
    ("h8192", 8, 2048, 2, 0), ("h3584", 9, 1024, 9, 0)])
def test_launch_table_drives_the_benchmark_configurations(cfg, entry, chunk, splits, tclass):
    """Each benchmark configuration finds its row of the gfx950 launch table
    (csrc/launch_table.hpp) and takes its chunk scale and split count."""
    info = _native.plan_info(_cfg_problem(cfg))
    assert info["grads_in_forward"] == 1
    assert info["table_entry"] == entry
    assert info["teacher_class"] == tclass
    assert info["token_chunk"] == chunk and info["chunk_scale"] == chunk // 512
    assert info["grad_hidden_splits"] == splits
    assert info["scan_engine"] == 1  # the ring engine
    assert info["scan_workgroups"] <= 256
    # the plan's workspace is the one orda_forward_workspace_bytes reports
    assert info["forward_workspace_bytes"] == _native.forward_workspace_bytes(_cfg_problem(cfg))


@pytest.mark.parametrize("token_chunk, tokens_per_tile", [(640, 128), (600, 128), (320, 128), (1000, 128)])
def test_scan_grid_fits_one_wave_when_token_tiles_do_not_divide_it(token_chunk, tokens_per_tile):
    """A chunk whose token-tile count does not divide the 256 persistent
    workgroups (1280 tokens: 10 tiles of 128) gets floor(256 / tiles)
    vocabulary ranges, not the ceiling: 260 workgroups would run 4 of them in
    a second wave behind the first and double the scan."""
    info = _native.plan_info(_problem(flags=0x33 | GIF, token_chunk=token_chunk))
    assert info["table_entry"] == 0 and info["scan_tokens_per_tile"] == tokens_per_tile
    ntt = -(-info["token_chunk"] // tokens_per_tile)
    assert info["scan_workgroups"] <= 256
    # every vocabulary tile (501 of 256 rows) is still covered by the ranges
    ranges = info["scan_workgroups"] // ntt
    assert ranges * ntt == info["scan_workgroups"]
    assert ranges >= 256 // ntt - 1 and ranges * -(-501 // ranges) >= 501


# divergence codes of include/orda_ce.h
_HELLINGER, _RENYI, _CHI2, _L2, _AB = 4, 6, 8, 9, 10


@pytest.mark.parametrize("cfg, div, alpha, ring", [
    ("c3", _HELLINGER, 0.5, True),  # separate teacher: staged logits, ring scan
    ("c3", _RENYI, 0.5, True),
    ("c3", _RENYI, 2.0, False),     # negative student exponent over bf16-staged logits
    ("c3", _CHI2, 0.5, False),
    ("c3", _L2, 0.5, True),         # three power terms: two passes on the ring scan
    ("c3", _AB, 0.5, True),
    ("c3", _AB, -1.0, False),       # alpha + beta < 0: negative student exponent
    ("c4", _CHI2, 0.5, True),       # precomputed logits read in place: not rounded again
    ("c4", _AB, 0.5, True),
    ("c4", _AB, -1.0, True),
])
def test_power_family_scan_engine(cfg, div, alpha, ring):
    """The one-term power family runs the ring scan with a staged or in-place
    teacher, and so do the three-term divergences (squared L2, AB), as
    two-pass divergences; a negative student exponent over a computed
    teacher's logits (staged in bf16) keeps the two-stage scan."""
    p = _cfg_problem(cfg)
    p.divergence, p.div_alpha, p.div_beta = div, alpha, 0.5
    info = _native.plan_info(p)
    assert info["scan_engine"] == (1 if ring else 0)
    assert info["scan_tokens_per_tile"] == (256 if ring else 128)


def test_launch_overrides_and_rule_for_unlisted_shapes():
    p = _cfg_problem("c2")
    p.grad_hidden_splits = 12
    assert _native.plan_info(p)["grad_hidden_splits"] == 12
    # a shape the table does not list takes the rule (round-filling split count)
    q = _problem(hidden=3072, teacher_hidden=3072, flags=0x33 | GIF, token_chunk=512)
    info = _native.plan_info(q)
    assert info["table_entry"] == -1 and info["chunk_scale"] == 2
    tiles = (1024 // 256) * (3072 // 256)
    s = info["grad_hidden_splits"]
    assert (tiles * s) % 256 == 0 or tiles * s < 256
    # the two-phase schedule has no token chunks
    r = _problem(flags=0x33)
    assert _native.plan_info(r)["grads_in_forward"] == 0


@pytest.mark.parametrize("name, kw, scale", [
    # (the launch table's swept shapes with the vocabulary moved off its rows,
    # so the rule decides; the table's measured choice in parentheses)
    ("tied, hidden 4096", dict(flags=0x33 | GIF), 2),                                   # (c2: 2)
    ("separate, hidden 2048", dict(mode=1, hidden=2048, teacher_hidden=4096, flags=0x23 | GIF,
                                   teacher_ce_weight=0.0, divergence=1, temperature=2.0), 4),  # (c3: 4)
    ("separate, hidden 2048, fp16", dict(mode=1, dtype=1, hidden=2048, teacher_hidden=4096, flags=0x23 | GIF,
                                         teacher_ce_weight=0.0, divergence=1, temperature=2.0), 4),  # (c3f16: 4)
    ("tied, hidden 8192", dict(hidden=8192, teacher_hidden=8192, flags=0x33 | GIF), 4),  # (h8192: 4)
    ("tied, hidden 3584", dict(hidden=3584, teacher_hidden=3584, flags=0x33 | GIF), 2),  # (h3584: 2)
    # (c5: 4; gradients 1.89 GB, so no chunk keeps the budget)
    ("tied, hidden 5120, 32768 tokens", dict(n_rows=32768, hidden=5120, teacher_hidden=5120, flags=0x33 | GIF), 4),
])
def test_chunk_rule_keeps_the_memory_budget(name, kw, scale):
    """Shapes the table does not list (vocabulary 128000) take the rule: the
    chunk scale rises from 2 to 4 when the step's extra memory at 4 stays
    under 2 GB (a separate teacher with a small student hidden) or when no
    chunk keeps 2 GB (hidden 8192, whose gradients alone pass it; 32768
    tokens at hidden 5120), and stays at 2 otherwise."""
    p = _problem(vocab=128000, token_chunk=512, **kw)
    info = _native.plan_info(p)
    assert info["table_entry"] == -1, name
    assert info["chunk_scale"] == scale, name
    # a small problem keeps the plain rule
    small = _problem(n_rows=96, hidden=64, teacher_hidden=64, vocab=1000, flags=0x33 | GIF, token_chunk=20)
    assert _native.plan_info(small)["token_chunk"] == 40


def test_grad_hidden_splits_keep_each_split_inside_a_buffer_resource():
    """H = 8192, V = 262144, 4096-token chunks: the whole W (4 GiB of bf16)
    exceeds one 32-bit buffer resource, so the grad-hidden GEMM is split at
    least until each split's K range of W and of the chunk's logits fits,
    whatever the requested split count."""
    for requested in (0, 1):
        p = _problem(hidden=8192, teacher_hidden=8192, vocab=262144, flags=0x33 | GIF, token_chunk=2048,
                     grad_hidden_splits=requested)
        info = _native.plan_info(p)
        assert info["token_chunk"] == 4096
        ld_bytes = max(8192, 2 * 4096) * 2
        assert info["vocab_rows_per_split"] * ld_bytes < 2 ** 31
        assert info["grad_hidden_splits"] >= 3
    with pytest.raises(ValueError, match="shape too large"):
        _native.plan_info(_problem(hidden=1 << 23, teacher_hidden=1 << 23))
    with pytest.raises(ValueError, match="grad_hidden_splits"):
        _native.plan_info(_problem(grad_hidden_splits=65))
