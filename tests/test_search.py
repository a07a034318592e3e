"""Plan search, table verification and spread logic (CPU only; the gate is faked).

Mirrors the reference's search behaviour (`kernelforge/search.py:131-351`) and
`verify --demote` (`kernelforge/cli.py:149-260`): stages are narrowed cheapest measured
cost first while the margin holds, only gate-passing plans are timed, the fastest wins;
verification demotes entries that re-measure above the demotion threshold to the safe
plan and leaves the rest alone.
"""
from __future__ import annotations

import dataclasses

import pytest
import torch

from techjam2026_amd import search as S
from techjam2026_amd.dispatch import DispatchTable, Entry, shape_signature
from techjam2026_amd.hw import GPUSpec
from techjam2026_amd.numerics import CheckResult
from techjam2026_amd.shapes import config
from techjam2026_amd.timing import Timing

# envelope of narrowing one stage alone (a C2-like budget: attention the most expensive)
ALONE = {"attn": 0.97, "out_proj": 0.68, "ffn1": 0.63, "ffn2": 0.64}
# the same with the activation alone rounded to fp16 (f16x2; for attention its QKV GEMM)
HALF = {"attn": 0.30, "out_proj": 0.25, "ffn1": 0.22, "ffn2": 0.24}
P16 = 0.05              # attention with single-plane probabilities
SINGLE_ATTN = 0.62      # f16x3 QKV GEMM feeding the single-pass fp16 attention
CONTROL_ENV = 0.003


def fake_envelope(plan) -> float:
    o = plan.overrides
    narrowed = [s for s, p in o if p == "float16"]
    half = [s for s, p in o if p in ("f16x2", "f16x2p")]
    p16 = [s for s, p in o if p in ("f16x3p", "f16x2p")]
    single = [s for s, p in o if p == "f16x3s"]
    # errors of independent stages add in quadrature
    return (CONTROL_ENV ** 2 + sum(ALONE[s] ** 2 for s in narrowed)
            + sum(HALF[s] ** 2 for s in half) + len(p16) * P16 ** 2
            + len(single) * SINGLE_ATTN ** 2) ** 0.5


def fake_evaluate(case, plan, device, trials=3, base=None, **_):
    u = fake_envelope(plan)
    return CheckResult(u < 1.0, u * 2e-3, 0.0, 0.0, 0, 1, None, 0.0, 0.0, u)


def fake_compare(runnable, warmup=0, repeats=0, rounds=0):
    def ms(name):
        if name == "reference":
            return 10.0
        # faster with every narrowed stage (a comma or a bracket opens one)
        return 2.0 - 0.2 * (name.count(",") + name.count("[")) - 0.1 * ("f16x2p[" in name)
    return {n: Timing([ms(n)]) for n in runnable}


def test_greedy_narrowing_cheapest_first_and_skips_what_breaks_the_margin():
    tried = []

    def gate(plan):
        tried.append(plan.overrides)
        u = fake_envelope(plan)
        return S.Candidate(plan, u, u <= 0.8)

    cost = {k: v - CONTROL_ENV for k, v in ALONE.items()}
    cands = S.narrow_greedy(S.CONTROL, CONTROL_ENV, cost, 0.8, gate)
    # ffn1 (cheapest) joins in fp16; ffn2 in fp16 exceeds 0.8, its f16x2 option joins;
    # out_proj likewise; attention in fp16 alone already exceeds the margin and is never
    # tried; its f16x3s option is tried and exceeds the margin, its f16x2p option joins
    # (f16x3p is then not needed)
    assert tried[0] == (("ffn1", "float16"),)
    assert [c.passed for c in cands] == [True, False, True, False, True, False, True]
    assert dict(cands[-2].plan.overrides)["attn"] == "f16x3s"
    assert all(dict(t).get("attn") != "float16" for t in tried)
    assert dict(cands[-1].plan.overrides) == {"ffn1": "float16", "ffn2": "f16x2",
                                              "out_proj": "f16x2", "attn": "f16x2p"}
    assert cands[0].plan.name == "fp16[ffn1]"
    assert cands[-1].plan.name == "fp16[ffn1]+f16x2[ffn2,out_proj]+f16x2p[attn]"
    assert all(c.utilization <= 0.8 for c in cands if c.passed)


def test_margin_is_a_hard_bound_on_what_passes():
    def gate(plan):
        u = fake_envelope(plan)
        return S.Candidate(plan, u, u <= 0.5)

    cost = {k: v - CONTROL_ENV for k, v in ALONE.items()}
    cands = S.narrow_greedy(S.CONTROL, CONTROL_ENV, cost, 0.5, gate)
    # every single-pass stage alone exceeds 0.5 and is never tried: the GEMM stages join
    # as f16x2; attention's f16x3s and f16x2p then exceed 0.5 and its f16x3p option joins
    assert [(dict(c.plan.overrides), c.passed) for c in cands] == [
        ({"ffn1": "f16x2"}, True),
        ({"ffn1": "f16x2", "ffn2": "f16x2"}, True),
        ({"ffn1": "f16x2", "ffn2": "f16x2", "out_proj": "f16x2"}, True),
        ({"ffn1": "f16x2", "ffn2": "f16x2", "out_proj": "f16x2", "attn": "f16x3s"}, False),
        ({"ffn1": "f16x2", "ffn2": "f16x2", "out_proj": "f16x2", "attn": "f16x2p"}, False),
        ({"ffn1": "f16x2", "ffn2": "f16x2", "out_proj": "f16x2", "attn": "f16x3p"}, True)]
    assert all(c.utilization <= 0.5 for c in cands if c.passed)


def test_search_picks_the_fastest_passing_plan():
    case = dataclasses.replace(config("C1"), num_layers=1)
    r = S.search(case, torch.device("cpu"), margin=0.8, trials=1, verbose=False,
                 evaluate=fake_evaluate, compare=fake_compare)
    assert r.best is not None and r.best.passed
    assert r.best.plan.cuda_graph
    assert dict(r.best.plan.overrides) == {"ffn1": "float16", "ffn2": "f16x2",
                                           "out_proj": "f16x2", "attn": "f16x2p"}
    assert r.best.utilization <= 0.8
    assert r.baseline_ms == 10.0 and r.best.speedup == pytest.approx(10.0 / r.best.median_ms)
    rec = r.record()
    assert rec["best"]["plan"] == r.best.plan.name
    assert all(c["envelope"] <= 0.8 for c in rec["candidates"] if c["passed"])


SPEC = GPUSpec(name="test", arch="gfx950", cu_count=256, total_mem_gb=288.0,
               shared_mem_per_block_kb=160.0, warp_size=64, l2_cache_mb=4.0)


def _table_with(plan, case):
    t = DispatchTable()
    t.add(Entry(signature=shape_signature(case), dtype=case.dtype, arch="gfx950",
                regime=case.regime, plan=plan, utilization=0.6, speedup=5.0,
                speedup_vs_compile=float("nan"), case=case.name))
    return t


def test_verify_demotes_drifted_entries_only():
    case = config("C2")
    narrow = S.CONTROL.with_override("attn", "float16")          # 0.97: passes, drifted
    table = _table_with(narrow, case)
    recs, demoted, failures = S.verify_table(table, SPEC, [case], "cpu", 1, 0.941, True,
                                             evaluate=fake_evaluate)
    assert recs[0]["envelope"] == pytest.approx(fake_envelope(narrow))
    assert demoted and demoted[0][0] == "C2" and not failures
    plan, source = table.lookup("gfx950", torch.float32, case.to_config())
    assert source == "exact" and plan.compute_dtype == "f16x3" and not plan.overrides

    kept = S.CONTROL.with_override("ffn1", "float16")
    table = _table_with(kept, case)
    _, demoted, _ = S.verify_table(table, SPEC, [case], "cpu", 1, 0.941, True,
                                   evaluate=fake_evaluate)
    assert not demoted
    plan, _ = table.lookup("gfx950", torch.float32, case.to_config())
    assert dict(plan.overrides) == {"ffn1": "float16"}


def test_verify_without_demote_changes_nothing():
    case = config("C2")
    narrow = S.CONTROL.with_override("attn", "float16").with_override("ffn2", "float16")
    table = _table_with(narrow, case)
    _, demoted, failures = S.verify_table(table, SPEC, [case], "cpu", 1, 0.941, False,
                                          evaluate=fake_evaluate)
    assert not demoted and failures       # 1.17 > 1: a gate failure is reported
    plan, _ = table.lookup("gfx950", torch.float32, case.to_config())
    assert dict(plan.overrides) == {"attn": "float16", "ffn2": "float16"}


def test_spread_is_the_largest_difference_per_case():
    runs = [[{"case": "C1", "envelope": 0.50}, {"case": "C2", "envelope": 0.60}],
            [{"case": "C1", "envelope": 0.52}, {"case": "C2", "envelope": 0.55}],
            [{"case": "C1", "envelope": 0.49}, {"case": "C2", "checked": False}]]
    s = S.spread_of(runs)
    assert s["C1"] == pytest.approx(0.03) and s["C2"] == pytest.approx(0.05)


def test_admission_and_verification_include_the_timing_input():
    """Every gate call of the search and of verify sees the organizer's timing input
    (seed 1234 + 100000) beside the accuracy seeds, so bench's checked output was admitted."""
    seen = []

    def recording_evaluate(case, plan, device, trials=3, base=None, extra_seeds=(), **_):
        seen.append(tuple(extra_seeds))
        return fake_evaluate(case, plan, device, trials, base)

    case = dataclasses.replace(config("C1"), num_layers=1)
    S.search(case, torch.device("cpu"), margin=0.8, trials=1, verbose=False,
             evaluate=recording_evaluate, compare=fake_compare)
    gate_calls = [s for s in seen if s]
    assert gate_calls and all(s == (1234 + 100000,) for s in gate_calls)
    seen.clear()
    S.verify_table(DispatchTable(), SPEC, [case], "cpu", 1, 0.941, False,
                   evaluate=recording_evaluate)
    assert seen == [(1234 + 100000,)]


def test_time_order_lets_the_dominant_stage_narrow_first():
    """Where attention dominates the forward (long S), narrowing the cheap GEMM stages
    first would spend the budget attention needs; the time-ordered pass keeps a plan with
    attention in fp16, and the fastest passing plan wins."""
    alone = {"attn": 0.66, "out_proj": 0.30, "ffn1": 0.25, "ffn2": 0.28}

    def env(plan):
        o = dict(plan.overrides)
        return (CONTROL_ENV ** 2 + sum(alone[s] ** 2 for s, p in o.items() if p == "float16")
                + sum((0.5 * alone[s]) ** 2 for s, p in o.items() if p in ("f16x2", "f16x2p"))
                + sum(P16 ** 2 for s, p in o.items() if p in ("f16x3p", "f16x2p"))) ** 0.5

    def evaluate(case, plan, device, trials=3, base=None, **_):
        u = env(plan)
        return CheckResult(u < 1.0, u * 2e-3, 0.0, 0.0, 0, 1, None, 0.0, 0.0, u)

    def compare(runnable, warmup=0, repeats=0, rounds=0):
        def ms(name):      # attention in fp16 halves the forward; other stages save little
            t = 10.0 - (4.0 if "fp16[attn" in name or ",attn" in name and "fp16[" in name else 0.0)
            return t - 0.1 * name.count("[")
        return {n: Timing([ms(n)]) for n in runnable}

    case = dataclasses.replace(config("C1"), num_layers=1)
    r = S.search(case, torch.device("cpu"), margin=0.8, trials=1, verbose=False,
                 evaluate=evaluate, compare=compare)
    assert dict(r.best.plan.overrides).get("attn") == "float16", r.best.plan.name
    assert r.best.utilization <= 0.8
