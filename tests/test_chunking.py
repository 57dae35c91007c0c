"""Chunk resolver and OOM-retry dispatcher (CPU): the known answers of the
reference's test/unit/test_resolver.py and test_dispatcher.py, plus the
vocabulary-chunk mapping of this build."""
from __future__ import annotations

import ast
from pathlib import Path

import pytest
import torch

from orda_ce_kernel.ops._engine import vocab_chunk_for
from orda_ce_kernel.utils import dispatcher
from orda_ce_kernel.utils._autotune import _is_oom_error
from orda_ce_kernel.utils.resolver import resolve_chunk_size


def test_resolver_rejects_empty_batch():
    with pytest.raises(ValueError, match="BT"):
        resolve_chunk_size(0, None, V=128)


def test_resolver_explicit_chunk_size_is_clamped():
    assert resolve_chunk_size(128, 512, V=32768) == (128, 1)
    assert resolve_chunk_size(128, 64, V=32768) == (64, 2)


def test_resolver_num_chunks_rounds_up():
    assert resolve_chunk_size(10, None, V=32768, num_chunks=3) == (4, 3)
    assert resolve_chunk_size(10, "dynamic", V=32768, num_chunks=20) == (1, 10)


def test_resolver_rejects_ambiguous_controls():
    with pytest.raises(ValueError, match="mutually exclusive"):
        resolve_chunk_size(10, 4, V=32768, num_chunks=3)


def test_resolver_dynamic_partition_covers_batch():
    cs, n = resolve_chunk_size(8192, "dynamic", V=32768)
    assert cs > 0 and n > 0 and cs * n >= 8192


@pytest.mark.parametrize("auto", [None, "dynamic", "auto", -2, 0, -1.0])
def test_resolver_auto_without_vocab_is_one_chunk(auto):
    assert resolve_chunk_size(128, auto, V=None) == (128, 1)


def test_resolver_respects_max_chunks_and_default_cap():
    assert resolve_chunk_size(32768, "dynamic", V=131072, max_chunks=2)[1] <= 2
    assert resolve_chunk_size(32768, "dynamic", V=131072)[1] == 64


def test_resolver_baseline_shapes():
    # C2/C3/C4 -> 16 x 512 rows, C5 -> 64 x 512, C1 -> 1 x 512
    assert resolve_chunk_size(8192, None, V=128256) == (512, 16)
    assert resolve_chunk_size(32768, None, V=152064) == (512, 64)
    assert resolve_chunk_size(512, None, V=4096) == (512, 1)


def test_vocab_chunk_maps_token_chunks_to_vocab_chunks():
    assert vocab_chunk_for(8192, 128256, None, None) == 8016
    assert vocab_chunk_for(16, 257, 7, None) == 86
    # doubling the chunk count halves the staging
    assert vocab_chunk_for(8192, 128256, 256, None) == 4008


def test_chunk_size_from_num_chunks():
    assert dispatcher._chunk_size_from_num_chunks(10, 3) == 4
    assert dispatcher._chunk_size_from_num_chunks(10, 5) == 2


def test_chunk_cache_is_a_copy_and_clears():
    dispatcher.clear_chunk_cache()
    c = dispatcher.get_chunk_cache()
    c[("fake",)] = 1
    assert dispatcher.get_chunk_cache() == {}


def test_oom_classifier():
    assert _is_oom_error(torch.cuda.OutOfMemoryError("boom"))
    assert _is_oom_error(RuntimeError("CUDA out of memory"))
    assert _is_oom_error(RuntimeError("HIP out of memory. Tried to allocate"))
    assert not _is_oom_error(RuntimeError("CPU out of memory"))
    assert not _is_oom_error(RuntimeError("shape mismatch"))


def test_cache_key_separates_modes_tensors_and_contract_fields():
    hs = torch.randn(8, 2, dtype=torch.float16)
    ht = torch.randn(8, 2, dtype=torch.float16)
    w = torch.randn(4, 2, dtype=torch.float16)
    wt = torch.randn(4, 2, dtype=torch.float16)
    lt = torch.randn(8, 4, dtype=torch.float32)
    k = dispatcher._cache_key
    tied = k(8, 4, 2, hs, w, "tied", teacher_hidden=ht)
    sep = k(8, 4, 2, hs, w, "separate", teacher_hidden=ht, teacher_weight=wt)
    pre = k(8, 4, 2, hs, w, "precomputed", logits_teacher=lt)
    assert len({tied, sep, pre}) == 3
    base = k(8, 4, 2, hs, w, "precomputed", max_fused_size=64, max_chunks=8, logits_teacher=lt)
    assert base != k(8, 4, 2, hs, w, "precomputed", max_fused_size=128, max_chunks=8, logits_teacher=lt)
    assert base != k(8, 4, 2, hs, w, "precomputed", max_fused_size=64, max_chunks=8, logits_teacher=lt.half())
    on = k(8, 4, 2, hs, w, "separate", teacher_hidden=ht, teacher_weight=wt, compute_kl=True)
    off = k(8, 4, 2, hs, w, "separate", teacher_hidden=ht, teacher_weight=wt, compute_kl=False)
    assert on != off


def test_dynamic_chunk_retries_after_oom_and_caches(monkeypatch):
    dispatcher.clear_chunk_cache()
    calls = []

    def fake(*args, chunk_size=None, **kwargs):
        calls.append(chunk_size)
        if len(calls) == 1:
            raise torch.cuda.OutOfMemoryError("synthetic out of memory")
        one = torch.tensor(1.0)
        return one, one, one, one

    monkeypatch.setattr(dispatcher, "_resolve_kernel_fn", lambda _mode: object())
    monkeypatch.setattr(dispatcher, "_call_kernel_fn", fake)
    out = dispatcher.dynamic_chunk(torch.randn(4, 2), torch.randn(4, 2), torch.randn(4, 2),
                                   torch.randint(0, 4, (4,)), chunk_size="dynamic")
    assert len(out) == 4
    assert calls == [4, 2]
    assert list(dispatcher.get_chunk_cache().values()) == [2]
    dispatcher.clear_chunk_cache()


def test_dynamic_chunk_gives_up_with_advice(monkeypatch):
    dispatcher.clear_chunk_cache()

    def always_oom(*args, **kwargs):
        raise torch.cuda.OutOfMemoryError("synthetic")

    monkeypatch.setattr(dispatcher, "_resolve_kernel_fn", lambda _mode: object())
    monkeypatch.setattr(dispatcher, "_call_kernel_fn", always_oom)
    with pytest.raises(RuntimeError, match="Increase max_chunks"):
        dispatcher.dynamic_chunk(torch.randn(4, 2), torch.randn(4, 2), torch.randn(4, 2),
                                 torch.randint(0, 4, (4,)), chunk_size="dynamic")


def test_dynamic_chunk_fixed_path_makes_one_call(monkeypatch):
    calls = []

    def fake(*args, chunk_size=None, **kwargs):
        calls.append(chunk_size)
        one = torch.tensor(1.0)
        return one, one, one, one

    monkeypatch.setattr(dispatcher, "_resolve_kernel_fn", lambda _mode: object())
    monkeypatch.setattr(dispatcher, "_call_kernel_fn", fake)
    dispatcher.dynamic_chunk(torch.randn(10, 2), torch.randn(10, 2), torch.randn(4, 2),
                             torch.randint(0, 4, (10,)), num_chunks=3)
    assert calls == [4]


def test_non_oom_errors_propagate(monkeypatch):
    def boom(*args, **kwargs):
        raise ValueError("not an OOM")

    monkeypatch.setattr(dispatcher, "_resolve_kernel_fn", lambda _mode: object())
    monkeypatch.setattr(dispatcher, "_call_kernel_fn", boom)
    with pytest.raises(ValueError, match="not an OOM"):
        dispatcher.dynamic_chunk(torch.randn(4, 2), torch.randn(4, 2), torch.randn(4, 2),
                                 torch.randint(0, 4, (4,)))


PKG = Path(__file__).resolve().parents[1] / "orda-knowledge-distillation-kernel_amd" / "orda_ce_kernel"


def test_runtime_options_are_not_file_backed():
    """Reference test/unit/test_no_config_dependency.py: no yaml / config
    module imports in the core files, no config file."""
    offenders = []
    for path in PKG.rglob("*.py"):
        tree = ast.parse(path.read_text(encoding="utf-8"))
        for node in ast.walk(tree):
            names = []
            if isinstance(node, ast.Import):
                names = [a.name for a in node.names]
            elif isinstance(node, ast.ImportFrom) and node.module:
                names = [node.module]
            offenders += [f"{path.name}: {n}" for n in names if n == "yaml" or n.endswith(".config")]
    assert offenders == []
    assert not (PKG / "config.py").exists()


def test_product_never_imports_the_oracle():
    for path in PKG.rglob("*.py"):
        text = path.read_text(encoding="utf-8")
        assert "from oracle" not in text and "import oracle" not in text, path
