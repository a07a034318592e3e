"""Dispatch-table policy, hardware probe strings, shapes, roofline (CPU only).

Mirrors the reference's `tests/test_dispatch.py` for the parts that carry over to a
gfx950 table: keying, collision rules, JSON round trip, lookup order, the device overlay,
device slugs, plus the gfx950-specific default rules and arch parsing (the reference's
`_arch_major` would read "gfx950" as major 95).
"""
from __future__ import annotations

import dataclasses

import pytest
import torch

from techjam2026_amd import dispatch as D
from techjam2026_amd import hw, roofline, shapes
from techjam2026_amd.dispatch import (DispatchTable, Entry, _aggressiveness, default_plan,
                                      shape_signature)
from techjam2026_amd.model import TransformerConfig
from techjam2026_amd.optimized import LADDER, Plan

SAFE_G = dataclasses.replace(D.SAFE, cuda_graph=True, name="safe+graph")
MILD = Plan(name="f16[attn]", overrides=(("attn", "float16"),))
MILD_G = dataclasses.replace(MILD, cuda_graph=True, name="f16[attn]+graph")
BOLD = Plan(name="f16[attn,out,ffn2]", overrides=(("attn", "float16"), ("out_proj", "float16"),
                                                  ("ffn2", "float16")))
CFG = TransformerConfig(8, 128, 512, 8, 2048, 6, False)


def entry(plan, case, speedup=2.0, util=0.6, dtype="float32", arch="gfx950", sig="SIG"):
    return Entry(sig, dtype, arch, "gemm", plan, util, speedup, 1.0, case)


def test_risk_ordering_is_monotone_in_narrowing():
    assert _aggressiveness(D.SAFE) < _aggressiveness(MILD) < _aggressiveness(BOLD)
    assert _aggressiveness(Plan(compute_dtype="f16x3")) < _aggressiveness(Plan(compute_dtype="bf16x3"))
    assert _aggressiveness(Plan(compute_dtype="bf16x3")) < _aggressiveness(Plan(compute_dtype="float16"))


def test_graph_capture_carries_no_risk():
    assert _aggressiveness(MILD) == _aggressiveness(MILD_G)


def test_different_variants_resolve_to_the_safer_plan():
    for order in ([("default", BOLD), ("default_pad", SAFE_G)],
                  [("default_pad", SAFE_G), ("default", BOLD)]):
        table = DispatchTable()
        for case, plan in order:
            table.add(entry(plan, case))
        assert table.entries[0].plan.name == SAFE_G.name


def test_re_measuring_the_same_case_supersedes():
    table = DispatchTable()
    table.add(entry(MILD, "default"))
    table.add(entry(BOLD, "default"))
    assert table.entries[0].plan.name == BOLD.name


def test_ties_prefer_the_faster_plan_and_keep_the_tighter_envelope():
    table = DispatchTable()
    table.add(entry(MILD, "default_pad", speedup=1.5, util=0.3))
    table.add(entry(MILD_G, "default", speedup=2.7, util=0.7))
    assert table.entries[0].plan.cuda_graph
    assert table.entries[0].utilization == 0.7


def test_round_trip_through_json(tmp_path, monkeypatch):
    monkeypatch.setattr(D, "TABLE_DIR", str(tmp_path))
    table = DispatchTable()
    plan = dataclasses.replace(BOLD, flash_block=(128, 64, 4, 2))
    table.add(entry(plan, "default"))
    table.save("gfx950")
    again = DispatchTable.load("gfx950")
    got = again.entries[0]
    assert got.plan.overrides == plan.overrides and got.plan.flash_block == (128, 64, 4, 2)
    assert got.case == "default"


def test_reference_schema_entries_load(tmp_path, monkeypatch):
    """Plan JSON written with the reference's field set (e.g. torch_compile) loads."""
    import json
    monkeypatch.setattr(D, "TABLE_DIR", str(tmp_path))
    blob = {"arch": "gfx950", "entries": [{
        "signature": shape_signature(CFG), "dtype": "float32", "arch": "gfx950",
        "regime": "gemm", "utilization": 0.1, "speedup": 3.0, "speedup_vs_compile": 1.2,
        "case": "c", "plan": {"name": "x", "compute_dtype": "f16x3", "residual_dtype": "float32",
                              "fuse_qkv": True, "attention": "flash", "fused_norm": True,
                              "cuda_graph": True, "torch_compile": None, "flash_block": None,
                              "smem_kb": 160.0, "overrides": [], "match_score_rounding": False,
                              "some_future_field": 1}}]}
    (tmp_path / "dispatch_gfx950.json").write_text(json.dumps(blob))
    plan, source = DispatchTable.load("gfx950").lookup("gfx950", torch.float32, CFG)
    assert source == "exact" and plan.name == "x"


def test_lookup_falls_back_in_order():
    _, source = DispatchTable().lookup("gfx950", torch.float32, CFG)
    assert source == "default"
    table = DispatchTable()
    table.add(Entry(shape_signature(CFG), "float32", "gfx950", "gemm", MILD_G, 0.6, 2.5, 1.2, "d"))
    plan, source = table.lookup("gfx950", torch.float32, CFG)
    assert source == "exact" and plan.name == MILD_G.name
    other = TransformerConfig(8, 129, 512, 8, 2048, 6, False)
    plan, source = table.lookup("gfx950", torch.float32, other)
    assert source == "nearest"
    # a neighbour's precision choices must not transfer: the conservative default answers
    assert plan.overrides == default_plan(torch.float32, conservative=True).overrides
    assert plan.overrides != MILD_G.overrides


def test_causal_and_layers_are_part_of_the_signature():
    a = TransformerConfig(8, 128, 512, 8, 2048, 6, False)
    assert shape_signature(a) != shape_signature(dataclasses.replace(a, causal=True))
    assert shape_signature(a) != shape_signature(dataclasses.replace(a, num_layers=12))
    assert shape_signature(a) == "B8-S128-d512-H8-F2048-L6"


def test_gfx950_float32_default_is_split_precision_with_graph():
    plan = default_plan(torch.float32, arch="gfx950")
    assert plan.compute_dtype == "f16x3" and dict(plan.overrides) == {"attn": "f16x3p"}
    assert plan.residual_dtype == "float32" and plan.cuda_graph and plan.attention == "flash"
    assert default_plan(torch.float32, conservative=True, arch="gfx950") == plan


def test_narrow_io_dtypes_take_the_reference_forward_graph_captured():
    for dt in (torch.float16, torch.bfloat16):
        plan = default_plan(dt, arch="gfx950")
        assert plan.attention == "baseline" and plan.cuda_graph
        assert plan.compute_dtype == "auto" and plan.residual_dtype == "auto"


def test_unmaterialisable_scores_never_get_a_score_matrix_plan():
    big = TransformerConfig(4, 65536, 1024, 16, 1024, 2, True)
    assert D.score_matrix_bytes(big) > 8 * 2**30
    table = DispatchTable([Entry(shape_signature(big), "float32", "gfx950", "attention",
                                 LADDER["baseline"], 0.0, 1.0, 1.0, "c")])
    plan, source = table.lookup("gfx950", torch.float32, big)
    assert plan.attention == "flash" and source == "exact"


def test_device_table_overlays_the_architecture_table(tmp_path, monkeypatch):
    monkeypatch.setattr(D, "TABLE_DIR", str(tmp_path))
    sig = shape_signature(CFG)
    p = lambda n: dataclasses.replace(SAFE_G, name=n)  # noqa: E731
    DispatchTable([Entry(sig, "float32", "gfx950", "gemm", p("ARCH"), 0.5, 2.0, 1.1, "c"),
                   Entry("ONLY", "float32", "gfx950", "gemm", p("ARCH_ONLY"), 0.5, 2.0, 1.1, "c"),
                   ]).save("gfx950")
    DispatchTable([Entry(sig, "float32", "gfx950", "gemm", p("DEVICE"), 0.9, 1.0, 1.0, "c")]
                  ).save("gfx950", "mi355x-288gb_gfx950")
    merged = DispatchTable.load("gfx950", "mi355x-288gb_gfx950")
    plan, source = merged.lookup("gfx950", torch.float32, CFG)
    assert plan.name == "DEVICE" and source == "exact"
    assert any(e.plan.name == "ARCH_ONLY" for e in merged.entries)
    keys = [(e.arch, e.dtype, e.signature) for e in merged.entries]
    assert len(keys) == len(set(keys))
    assert DispatchTable.load("gfx950").lookup("gfx950", torch.float32, CFG)[0].name == "ARCH"
    path = merged.save("gfx950", "mi355x-288gb_gfx950")
    assert len(DispatchTable.load("gfx950", "mi355x-288gb_gfx950").entries) == 2
    assert "__mi355x-288gb_gfx950" in path


def test_arch_string_and_device_slugs():
    assert hw.arch_of("gfx950:sramecc+:xnack-") == "gfx950"
    assert hw.arch_of("gfx942") == "gfx942"

    class Spec:
        def __init__(self, name, arch, mem):
            self.name, self.arch, self.total_mem_gb = name, arch, mem

    cards = [("AMD Instinct MI355X", "gfx950", 287.98), ("AMD Instinct MI350X", "gfx950", 287.98),
             ("AMD Instinct MI300X", "gfx942", 191.98), ("AMD Instinct MI325X", "gfx942", 255.98)]
    slugs = [hw.device_slug(Spec(*c)) for c in cards]
    assert slugs[0] == "mi355x-288gb_gfx950"
    assert len(set(slugs)) == len(slugs)
    for s in slugs:
        assert "--" not in s and s == s.lower() and " " not in s

    class Generic(Spec):
        cu_count = 256
    # a host without the driver's name table reports a generic name for every card
    assert hw.device_slug(Generic("AMD Radeon Graphics", "gfx950", 287.98)) == "256cu-288gb_gfx950"


def test_shape_grammar_and_configs():
    c = shapes.parse_spec("B8-S128-d512-H8-F2048-L6-causal-pad0.4-scale64-float16")
    assert (c.batch_size, c.seq_len, c.d_model, c.num_heads, c.ffn_dim, c.num_layers) == \
        (8, 128, 512, 8, 2048, 6)
    assert c.causal and c.padding_ratio == 0.4 and c.input_scale == 64 and c.dtype == "float16"
    assert shapes.parse_spec("B2xS2048xd512xH8xF2048").num_layers == 6
    with pytest.raises(ValueError):
        shapes.parse_spec("B2-S16-d30-H4-F8")
    with pytest.raises(ValueError):
        shapes.parse_spec("nonsense")
    names = [c.name for c in shapes.CONFIGS]
    assert names == ["C1", "C2", "C3", "C4", "C5"]
    c3 = shapes.config("C3")
    assert c3.head_dim == 8 and c3.padding_ratio == 0.875
    # valid-length ranges stated in BASELINE.json
    for name, lo in (("C1", 64), ("C2", 64), ("C3", 128), ("C4", 1024), ("C5", 32768)):
        c = shapes.config(name)
        assert max(1, int(round(c.seq_len * (1 - c.padding_ratio)))) == lo


def test_roofline_units_and_work_formulas():
    c = shapes.config("C2")
    g = roofline.gemm_flops(c.batch_size, c.seq_len, c.d_model, c.ffn_dim, c.num_layers)
    assert abs(g / 1e9 - 309.2) < 0.1      # 2*M*(3d*d + d*d + 2*d*F) per layer, x L
    a = roofline.attention_flops(c.batch_size, c.seq_len, c.d_model, c.num_heads, 1, True)
    assert abs(a / 1e9 - 4.295) < 0.01
    # padding-aware count equals the mask-agnostic one when nothing is padded (up to the
    # diagonal: S(S+1)/2 pairs vs S^2/2)
    full = roofline.attention_flops_padded([c.seq_len] * c.batch_size, c.seq_len, c.d_model,
                                           c.num_heads, 1, True)
    assert full == 4 * c.num_heads * (c.d_model // c.num_heads) * c.batch_size * \
        c.seq_len * (c.seq_len + 1) // 2
    r = roofline.analyse(c, 2.0, "f16x3")
    assert r.achieved_tflops == pytest.approx(roofline.stack_flops(
        c.batch_size, c.seq_len, c.d_model, c.num_heads, c.ffn_dim, c.num_layers, True) / 2e-3 / 1e12)
    assert 0 < r.utilization <= 1.0
    assert roofline.useful_peak_tflops("f16x3") == pytest.approx(2500 / 3)
    assert roofline.ln_bytes(262144, 1024) == 262144 * 1024 * 16 + 262144 + 8 * 1024
