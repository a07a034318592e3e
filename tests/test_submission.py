"""The drop-in's contract and the stack's host logic (CPU only).

Mirrors the reference's `tests/test_submission.py` (strict weight copy, announced and
sticky fallback, CPU output) and the arithmetic half of `tests/test_streaming.py`
(memory-budget batch slicing decisions, which need no GPU).
"""
from __future__ import annotations

import pytest
import torch

from techjam2026_amd import harness, shapes
from techjam2026_amd.model import BaselineTransformer, TransformerConfig
from techjam2026_amd.optimized import LADDER, FusedTransformer, Plan
from techjam2026_amd.submission import UserOptimizedTransformer


def _cfg(**kw):
    base = dict(batch_size=2, seq_len=16, d_model=32, num_heads=4, ffn_dim=32, num_layers=2,
                causal=True)
    base.update(kw)
    return TransformerConfig(**base)


def test_is_a_baseline_subclass_so_strict_weight_copy_works():
    cfg = _cfg()
    assert issubclass(UserOptimizedTransformer, BaselineTransformer)
    ours, ref = UserOptimizedTransformer(cfg), BaselineTransformer(cfg)
    assert set(ours.state_dict()) == set(ref.state_dict())
    harness.copy_model_weights(ref, ours, strict=True)
    keys = set(ref.state_dict())
    assert "layers.0.attention.q_proj.weight" in keys and "final_norm.bias" in keys
    assert set(FusedTransformer(cfg).state_dict()) == keys


def test_forward_falls_back_to_the_reference_when_the_fused_path_raises(capsys, monkeypatch):
    monkeypatch.setenv("KF950_STRICT", "0")
    cfg = _cfg()
    ours = UserOptimizedTransformer(cfg).eval()
    ref = BaselineTransformer(cfg).eval()
    ref.load_state_dict(ours.state_dict(), strict=True)

    class Exploding(torch.nn.Module):
        def forward(self, *a, **kw):
            raise RuntimeError("simulated kernel failure")

    ours._impl, ours._failed = Exploding(), False
    x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model)
    with torch.inference_mode():
        got, want = ours(x, None), ref(x, None)
    assert torch.equal(got, want)
    out = capsys.readouterr().out
    assert "kernelforge" in out and "reference forward" in out


def test_the_fallback_is_sticky(monkeypatch):
    monkeypatch.setenv("KF950_STRICT", "0")
    cfg = _cfg()
    ours = UserOptimizedTransformer(cfg).eval()
    calls = {"n": 0}

    class Exploding(torch.nn.Module):
        def forward(self, *a, **kw):
            calls["n"] += 1
            raise RuntimeError("boom")

    ours._impl, ours._failed = Exploding(), False
    x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model)
    with torch.inference_mode():
        for _ in range(4):
            ours(x, None)
    assert calls["n"] == 1


def test_strict_mode_raises_instead_of_falling_back(monkeypatch):
    monkeypatch.setenv("KF950_STRICT", "1")
    cfg = _cfg()
    ours = UserOptimizedTransformer(cfg).eval()

    class Exploding(torch.nn.Module):
        def forward(self, *a, **kw):
            raise RuntimeError("boom")

    ours._impl, ours._failed = Exploding(), False
    with pytest.raises(RuntimeError, match="boom"):
        ours(torch.randn(2, 16, 32), None)


def test_output_shape_and_dtype_on_cpu(monkeypatch, capsys):
    """No GPU: selection fails (no device) and the announced fallback answers."""
    monkeypatch.setenv("KF950_STRICT", "0")
    cfg = _cfg()
    ours = UserOptimizedTransformer(cfg).eval()
    x, mask = harness.generate_random_case(cfg, "cpu", torch.float32, 3, 0.4)
    with torch.inference_mode():
        out = ours(x, mask)
    assert out.shape == x.shape and out.dtype == x.dtype and torch.isfinite(out).all()
    assert torch.count_nonzero(out[~mask]) == 0
    if not torch.cuda.is_available():
        assert ours._failed and "reference forward" in capsys.readouterr().out


def test_fused_transformer_refuses_cpu_tensors():
    m = FusedTransformer(_cfg(), LADDER["f16x3"])
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.randn(2, 16, 32), None)


def test_plan_stage_precisions():
    p = Plan(compute_dtype="f16x3").with_override("ffn1", "float16")
    assert p.stage_precision("attn", torch.float32) == "f16x3"
    assert p.stage_precision("ffn1", torch.float32) == "float16"
    assert Plan(compute_dtype="auto").stage_precision("attn", torch.float32) == "float32"
    with pytest.raises(ValueError):
        Plan(compute_dtype="int8").stage_precision("attn", torch.float32)
    assert "ffn1:float16" in p.name


# (shape, GPU memory free in GB, expected decision) -- `tests/test_streaming.py:71-84`
BUDGETS = [
    ("B64-S128-d128-H4-F128-L4-causal", 8, "whole"),
    ("B64-S1024-d128-H4-F128-L4-causal", 8, "whole"),
    ("B10000-S128-d128-H4-F128-L4-causal", 79, "whole"),
    ("B10000-S128-d128-H4-F128-L4-causal", 6, "slice"),
    ("B32-S100000-d1024-H16-F1024-L2-causal", 79, "slice"),
    ("B32-S100000-d1024-H16-F1024-L2-causal", 288, "slice"),
    ("B4-S65536-d1024-H16-F1024-L2-causal", 288, "whole"),      # config C5 on one MI355X
]


@pytest.mark.parametrize("spec,free_gb,expect", BUDGETS)
def test_chunk_decision(spec, free_gb, expect):
    cfg = shapes.parse_spec(spec).to_config()
    m = FusedTransformer(cfg, LADDER["f16x3"])
    chunk = m._chunk_for_budget(cfg.batch_size, cfg.seq_len, torch.float32, free_gb * 2**30)
    if expect == "whole":
        assert chunk == cfg.batch_size
    else:
        assert 1 <= chunk < cfg.batch_size


def test_peak_memory_adapts_to_the_budget():
    cfg = shapes.parse_spec("B32-S100000-d1024-H16-F1024-L2-causal").to_config()
    m = FusedTransformer(cfg, LADDER["f16x3"])
    budgets = [288, 200, 160, 120, 93, 79, 60, 48]
    chunks = [m._chunk_for_budget(cfg.batch_size, cfg.seq_len, torch.float32, gb * 2**30)
              for gb in budgets]
    assert chunks == sorted(chunks, reverse=True) and chunks[0] > chunks[-1] >= 1
    assert m._chunk_for_budget(cfg.batch_size, cfg.seq_len, torch.float32, 4 * 2**30) == 1
    assert m.set_memory_budget(60 * 2**30) is m and m.memory_budget_bytes == 60 * 2**30
    with pytest.raises(ValueError):
        m.set_memory_budget(0)


def test_memory_model_arithmetic():
    """One pass may take `headroom` of what is left after the whole output, in units of one
    sequence's modelled working set (LIVE_TENSORS widest-row tensors)."""
    from techjam2026_amd.optimized import MemoryModel
    mm = MemoryModel(widest=1024, d_model=512)
    one = 1 * 100 * 1024 * 32 * 4
    assert mm.working_set(1, 100, 4) == one and mm.working_set(3, 100, 4) == 3 * one
    out = 8 * 100 * 512 * 4
    for k in (1, 2, 5, 7):
        free = int((k * one) / 0.55) + out + 64
        assert mm.sequences_per_pass(8, 100, 4, free) == k
    assert mm.sequences_per_pass(8, 100, 4, 10**15) == 8      # never more than the batch
    assert mm.sequences_per_pass(8, 100, 4, out // 2) == 1     # nothing left: one at a time
    assert mm.sequences_per_pass(1, 100, 4, 0) == 1


class _OomAbove:
    """Stands in for `_eager_forward`: raises OutOfMemoryError for passes of more than
    `limit` sequences, otherwise returns its input + 1 and records the pass."""

    def __init__(self, limit):
        self.limit, self.passes = limit, []

    def __call__(self, x, keep):
        if x.shape[0] > self.limit:
            raise torch.cuda.OutOfMemoryError("test: pass too large")
        self.passes.append(x.shape[0])
        return x + 1


@pytest.mark.parametrize("B,chunk,limit", [(8, 8, 3), (7, 4, 1), (5, 5, 5), (9, 2, 2)])
def test_sliced_forward_splits_passes_that_run_out_of_memory(monkeypatch, B, chunk, limit):
    cfg = _cfg(batch_size=B)
    m = FusedTransformer(cfg, LADDER["f16x3"])
    fake = _OomAbove(limit)
    monkeypatch.setattr(m, "_eager_forward", fake)
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: None)
    x = torch.arange(B * 2 * 3, dtype=torch.float32).view(B, 2, 3)
    keep = torch.ones(B, 2, dtype=torch.bool)
    out = m._chunked_forward(x, keep, chunk)
    assert torch.equal(out, x + 1)                       # every row written, once each
    assert sum(fake.passes) == B and max(fake.passes) <= limit
    # after the first split, later passes are planned at the size that succeeded
    assert len(fake.passes) <= 2 * ((B + limit - 1) // limit) + 1


def test_sliced_forward_reraises_when_one_sequence_does_not_fit(monkeypatch):
    m = FusedTransformer(_cfg(batch_size=4), LADDER["f16x3"])
    monkeypatch.setattr(m, "_eager_forward", _OomAbove(0))
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: None)
    with pytest.raises(torch.cuda.OutOfMemoryError):
        m._chunked_forward(torch.zeros(4, 2, 3), None, 4)
