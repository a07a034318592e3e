"""Budget-guided plan search and table verification on gfx950.

Mirrors `kernelforge/search.py:131-351` (the search), `kernelforge/cli.py:353-446`
(`sweep`: search each case, write the device's dispatch table) and
`kernelforge/cli.py:149-260` (`verify [--demote]`: re-measure the frozen table, replace
drifted entries with the safe plan).

    python -m techjam2026_amd.search sweep  --configs C1 C2 C3 C4 C5 [--margin 0.74]
    python -m techjam2026_amd.search verify [--demote] [--margin 0.80] [--json-out F]
    python -m techjam2026_amd.search spread --configs C1 C2 --processes 3

Search, per case:

1. the control plan (split fp32, "f16x3", every stage) and the per-stage cost of
   narrowing each stage alone to single-pass fp16 (`measure_stage_cost`);
2. stages narrowed greedily, cheapest measured cost first: a stage takes the first of its
   options (single-pass fp16, then "f16x2"; for attention fp16, "f16x3s", "f16x2p", "f16x3p")
   that keeps the running plan
   inside the gate at `margin` over `trials` seeds (default the organizer's five) and the
   organizer's timing input; fp16 is not tried for a stage whose
   own cost already exceeds the margin (the reference walks the same cumulative chain and
   keeps the passing prefix; skipping a failing stage instead of stopping lets a cheaper
   later stage still join);
3. every gate-passing plan is timed with hipGraph capture (capture changes no arithmetic,
   so it inherits the plan's envelope), interleaved with the reference forward; the
   fastest passing plan is the case's entry.

There is no `torch.compile` competitor (no tracing compiler on this path) and no tile
search: the kernels pick their tiles per shape from measured sweeps. The gate is the
organizer's rule, worst case over the seeds and the Xavier weight draws
`budget.WEIGHT_DRAWS`; the admission margin (0.74: the 0.80 target less the measured
sensitivity of a worst per-seed envelope) and the demotion threshold (the target plus the
run-to-run spread) are `numerics.ADMISSION_MARGIN` / `numerics.DEMOTION_MARGIN`.
"""
from __future__ import annotations

import dataclasses
import json
import os
import subprocess
import sys
import time
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch

from . import budget, harness, timing
from .dispatch import DispatchTable, Entry, SAFE, shape_signature
from .numerics import ADMISSION_MARGIN, DEMOTION_MARGIN
from .optimized import STAGES, Plan, build_shared
from .shapes import Case

CONTROL = Plan(name="f16x3", compute_dtype="f16x3", residual_dtype="float32")
# Admission and verification use the organizer's five accuracy seeds (1234..1238: seed +
# trial, `torch_transformer_benchmark.py:382-390, 617`): a plan admitted on fewer seeds has
# been seen to reach 0.84 of the tolerance on another input. The organizer's timing input
# (seed 1234 + 100000, `torch_transformer_benchmark.py:533`), whose output bench.py checks,
# is admitted beside them: a plan admitted at 0.76 over the five read 0.84 on it.
TRIALS = 5
TIMING_SEEDS = (1234 + 100000,)
NARROW = "float16"
# Cheaper precisions tried per stage, fastest first, when a stage is narrowed. After
# single-pass fp16, a GEMM stage has "f16x2" (the activation as one fp16 plane, the weight
# split: 2 of 3 MFMAs); attention has "f16x3s" (an f16x3 QKV GEMM feeding the single-pass
# fp16 attention: the fast attention kernel without the rounding of h and W in the
# projection, where most of single-pass fp16's budget goes), "f16x2p" (an f16x2 QKV GEMM,
# and the probabilities as one fp16 plane in P.V) and then "f16x3p" (the probabilities
# alone), which costs almost nothing of the budget where single-pass fp16 costs most.
OPTIONS = {"attn": ("float16", "f16x3s", "f16x2p", "f16x3p"), "out_proj": ("float16", "f16x2"),
           "ffn1": ("float16", "f16x2"), "ffn2": ("float16", "f16x2")}


@dataclasses.dataclass
class Candidate:
    plan: Plan
    utilization: float
    passed: bool
    median_ms: float = float("nan")
    speedup: float = float("nan")
    error: str = ""

    def row(self) -> str:
        status = "pass" if self.passed else "FAIL"
        return (f"{self.plan.name:<48} env={self.utilization:6.3f} {status}  "
                f"{self.median_ms:9.4f} ms  {self.speedup:7.3f}x"
                + (f"  {self.error}" if self.error else ""))


@dataclasses.dataclass
class SearchResult:
    case: Case
    best: Optional[Candidate]
    candidates: List[Candidate]
    baseline_ms: float
    stage_cost: Dict[str, float]
    seconds: float

    def summary(self) -> str:
        lines = [f"### {self.case.name}: {self.case.label()}",
                 f"    reference forward {self.baseline_ms:.4f} ms",
                 "    stage cost (fp16 alone): " + ", ".join(
                     f"{k}={v:+.3f}" for k, v in sorted(self.stage_cost.items(),
                                                        key=lambda kv: kv[1]))]
        lines += ["      " + c.row() for c in self.candidates]
        if self.best:
            lines.append(f"    -> BEST {self.best.plan.name} {self.best.median_ms:.4f} ms, "
                         f"{self.best.speedup:.3f}x vs the reference forward, "
                         f"envelope {self.best.utilization:.3f}")
        return "\n".join(lines)

    def record(self) -> dict:
        return {"case": self.case.name, "shape": self.case.label(),
                "baseline_ms": self.baseline_ms, "stage_cost": self.stage_cost,
                "seconds": round(self.seconds, 1),
                "candidates": [{"plan": c.plan.name, "describe": c.plan.describe(),
                                "envelope": c.utilization, "passed": c.passed,
                                "median_ms": c.median_ms, "speedup": c.speedup,
                                "error": c.error} for c in self.candidates],
                "best": None if self.best is None else {
                    "plan": self.best.plan.name, "utilization": self.best.utilization,
                    "median_ms": self.best.median_ms, "speedup": self.best.speedup}}


def measure_stage_cost(case: Case, device, control: Plan, trials: int = 2,
                       base=None, evaluate: Callable = budget.evaluate,
                       ) -> Tuple[float, Dict[str, float]]:
    """Envelope of the control plan and the marginal cost of narrowing each stage alone
    (`kernelforge/search.py:108-121`)."""
    base_util = evaluate(case, control, device, trials, base=base).envelope_utilization
    cost: Dict[str, float] = {}
    for stage in STAGES:
        try:
            u = evaluate(case, control.with_override(stage, NARROW), device, trials,
                         base=base).envelope_utilization
            cost[stage] = u - base_util
        except Exception:
            cost[stage] = float("inf")
    return base_util, cost


def _plan_name(plan: Plan) -> str:
    parts = []
    for prec in dict.fromkeys(p for _, p in plan.overrides):
        tag = "fp16" if prec == NARROW else prec
        parts.append(tag + "[" + ",".join(s for s, p in plan.overrides if p == prec) + "]")
    return "+".join(parts) or plan.name


def narrow_greedy(control: Plan, base_util: float, cost: Dict[str, float], margin: float,
                  gate: Callable[[Plan], Candidate],
                  order: Optional[Sequence[str]] = None) -> List[Candidate]:
    """Step 2 of the search: the gated candidates, in the order they were tried. Stages go
    cheapest measured fp16 cost first (or in `order`); each takes the first of its options
    (fastest first) that keeps the running plan inside the margin. Single-pass fp16 is not
    tried where its own cost already exceeds the margin."""
    out: List[Candidate] = []
    running = control
    if order is None:
        order = sorted(STAGES, key=lambda s: cost.get(s, float("inf")))
    for stage in order:
        for prec in OPTIONS.get(stage, (NARROW,)):
            if prec == NARROW:
                c = cost.get(stage, float("inf"))
                if c == float("inf") or base_util + c > margin:
                    continue
            trial = running.with_override(stage, prec)
            trial = dataclasses.replace(trial, name=_plan_name(trial))
            cand = gate(trial)
            out.append(cand)
            if cand.passed:
                running = trial
                break
    return out


def stage_time_saving(cfg, base, x, m, compare: Callable, heavy: bool) -> Dict[str, float]:
    """Milliseconds saved by narrowing each stage alone to single-pass fp16, from graph
    replays of the control plan and the four one-stage plans (interleaved timing)."""
    plans = {"(control)": dataclasses.replace(CONTROL, cuda_graph=True, name="control+graph")}
    for stage in STAGES:
        plans[stage] = dataclasses.replace(CONTROL.with_override(stage, NARROW),
                                           cuda_graph=True, name=f"fp16[{stage}]+graph")
    runnable = {}
    for plan in plans.values():
        mdl = build_shared(cfg, plan, base)
        runnable[plan.name] = (lambda mm=mdl: mm(x, m))
    t = compare(runnable, warmup=3 if heavy else 10, repeats=5 if heavy else 20, rounds=2)
    ctl = t[plans["(control)"].name].median_ms
    return {s: ctl - t[plans[s].name].median_ms for s in STAGES}


def search(case: Case, device, margin: float = ADMISSION_MARGIN, trials: int = TRIALS,
           time_budget_s: float = 600.0, verbose: bool = True,
           evaluate: Callable = budget.evaluate,
           compare: Callable = timing.compare) -> SearchResult:
    started = time.time()
    cfg = case.to_config()
    bases = budget.reference_models(case, device)
    base = bases[0]                     # stage costs and timing use the first draw
    x, m = harness.generate_random_case(cfg, device, case.torch_dtype, 1234,
                                        case.padding_ratio, case.input_scale)

    gated: Dict[frozenset, Candidate] = {}

    def gate(plan: Plan) -> Candidate:
        key = frozenset(plan.overrides)
        if key in gated:                 # the same stage precisions reached in another order
            return dataclasses.replace(gated[key], plan=plan)
        try:
            r = evaluate(case, plan, device, trials, bases=bases, extra_seeds=TIMING_SEEDS)
            c = Candidate(plan, r.envelope_utilization,
                          bool(r.passed) and r.envelope_utilization <= margin)
        except Exception as e:
            c = Candidate(plan, float("nan"), False,
                          error=f"{type(e).__name__}: {str(e)[:100]}")
        if verbose:
            print(f"  [{case.name}] gate {c.row()}", flush=True)
        gated[key] = c
        return c

    candidates: List[Candidate] = [gate(CONTROL)]
    base_util, cost = measure_stage_cost(case, device, CONTROL, trials=2, base=base,
                                         evaluate=evaluate)
    if verbose:
        print(f"  [{case.name}] control envelope {base_util:.3f}; stage cost " +
              ", ".join(f"{k}{v:+.3f}" for k, v in cost.items()), flush=True)
    # Two narrowing orders: the reference's (cheapest error cost first), and most time
    # saved first -- where one stage dominates the forward (attention at long S), narrowing
    # the cheap stages first can spend the budget that stage needed.
    heavy = cfg.batch_size * cfg.seq_len * cfg.d_model >= (1 << 24)
    orders = [sorted(STAGES, key=lambda s: cost.get(s, float("inf")))]
    if time.time() - started < time_budget_s:
        saved = stage_time_saving(cfg, base, x, m, compare, heavy)
        if verbose:
            print(f"  [{case.name}] ms saved by fp16 alone: " +
                  ", ".join(f"{k} {v:+.3f}" for k, v in saved.items()), flush=True)
        by_time = sorted(STAGES, key=lambda s: -saved[s])
        if by_time != orders[0]:
            orders.append(by_time)
    seen = set()
    for order in orders:
        if time.time() - started >= time_budget_s:
            break
        for cand in narrow_greedy(CONTROL, base_util, cost, margin, gate, order=order):
            if cand.plan.name not in seen:
                seen.add(cand.plan.name)
                candidates.append(cand)

    # 3. graph-capture every passing plan and time them against the reference forward
    timed: List[Candidate] = []
    for c in candidates:
        if c.passed:
            g = dataclasses.replace(c.plan, cuda_graph=True, name=c.plan.name + "+graph")
            timed.append(Candidate(g, c.utilization, True))
    # the reference forward is timed beside the candidates, except where its score tensor
    # cannot be formed (then no speedup is claimed; the candidates are ranked by time)
    streamed = budget.must_stream(cfg)
    runnable: Dict[str, Callable[[], object]] = {} if streamed else {
        "reference": lambda: base(x, m)}
    for c in timed:
        try:
            mdl = build_shared(cfg, c.plan, base)
            runnable[c.plan.name] = (lambda mm=mdl: mm(x, m))
        except Exception as e:
            c.passed, c.error = False, f"build: {type(e).__name__}: {str(e)[:80]}"
    t = compare(runnable, warmup=5 if heavy else 20, repeats=10 if heavy else 30,
                rounds=3)
    baseline_ms = t["reference"].median_ms if "reference" in t else float("nan")
    for c in timed:
        if c.plan.name in t:
            c.median_ms = t[c.plan.name].median_ms
            c.speedup = baseline_ms / c.median_ms
    candidates += timed
    ranked = sorted((c for c in timed if c.passed and c.median_ms == c.median_ms),
                    key=lambda c: c.median_ms)
    best = ranked[0] if ranked else None
    del runnable, base, bases
    torch.cuda.empty_cache()
    return SearchResult(case, best, candidates, baseline_ms, cost, time.time() - started)


# ----------------------------------------------------------------------------- CLI

def _spec_and_table(untuned: bool = False):
    from .hw import probe
    spec = probe(measure=False)
    return spec, (DispatchTable() if untuned else DispatchTable.load_for(spec))


def cmd_sweep(args) -> int:
    from .hw import device_slug
    from .shapes import resolve
    dev = torch.device("cuda")
    spec, table = _spec_and_table()
    slug = device_slug(spec)
    print(f"# {spec.summary()}\n# margin {args.margin}, {args.trials} seeds + timing input",
          flush=True)
    path = os.path.join(os.path.dirname(DispatchTable.path_for(spec.arch)), f"sweep_{slug}.json")
    records = []
    if os.path.exists(path):
        with open(path, encoding="utf-8") as f:
            records = json.load(f).get("records", [])
    for case in resolve(args.configs):
        print(f"[sweep] {case.name} {case.label()}", flush=True)
        r = search(case, dev, margin=args.margin, trials=args.trials,
                   time_budget_s=args.case_budget)
        print(r.summary(), flush=True)
        if r.best is not None:
            table.add(Entry(signature=shape_signature(case), dtype=case.dtype, arch=spec.arch,
                            regime=case.regime, plan=r.best.plan,
                            utilization=r.best.utilization, speedup=r.best.speedup,
                            speedup_vs_compile=float("nan"), case=case.name))
            print(f"[sweep] table -> {table.save(spec.arch, slug)}", flush=True)
        records = [x for x in records if x.get("case") != case.name] + [r.record()]
        with open(path, "w", encoding="utf-8") as f:
            json.dump({"gpu": spec.summary(), "arch": spec.arch, "device": slug,
                       "margin": args.margin, "trials": args.trials,
                       "extra_seeds": list(TIMING_SEEDS), "records": records}, f, indent=2)
    return 0


def verify_table(table: DispatchTable, spec, cases: Sequence[Case], device, trials: int,
                 margin: float, demote: bool, evaluate: Callable = budget.evaluate,
                 ) -> Tuple[List[dict], List[tuple], List[tuple]]:
    """(records, demoted, failures) of re-measuring `table` on `cases`
    (`kernelforge/cli.py:149-260`), worst case over `trials` seeds, the timing input and
    the weight draws `budget.WEIGHT_DRAWS`. With `demote`, an exact entry that fails the
    gate or re-measures above `margin` becomes the safe plan + graph."""
    records, demoted, failures = [], [], []
    for case in cases:
        plan, source = table.lookup(spec.arch, case.torch_dtype, case.to_config(),
                                    spec.shared_mem_per_block_kb)
        try:
            r = evaluate(case, plan, device, trials, extra_seeds=TIMING_SEEDS,
                         bases=budget.reference_models(case, device))
        except torch.cuda.OutOfMemoryError:
            records.append({"case": case.name, "plan": plan.name, "source": source,
                            "checked": False, "reason": "OutOfMemoryError"})
            continue
        except Exception as e:
            failures.append((case.name, plan.name, f"{type(e).__name__}: {e}"))
            records.append({"case": case.name, "plan": plan.name, "source": source,
                            "passed": False, "error": f"{type(e).__name__}: {str(e)[:160]}"})
            continue
        over = r.envelope_utilization > margin
        records.append({"case": case.name, "plan": plan.name, "source": source,
                        "passed": bool(r.passed), "envelope": r.envelope_utilization,
                        "worst_at": r.note, "max_abs": r.max_abs_error,
                        "failed_elements": r.failed_elements,
                        "total_elements": r.total_elements})
        if (not r.passed or over) and demote and source == "exact":
            safe = dataclasses.replace(SAFE, cuda_graph=True, name="safe(f16x3)+graph",
                                       smem_kb=spec.shared_mem_per_block_kb)
            table.add(Entry(signature=shape_signature(case), dtype=case.dtype, arch=spec.arch,
                            regime=case.regime, plan=safe, utilization=0.0,
                            speedup=float("nan"), speedup_vs_compile=float("nan"),
                            case=case.name))
            demoted.append((case.name, plan.name, r.envelope_utilization))
        if not r.passed:
            failures.append((case.name, plan.name, str(r)))
    return records, demoted, failures


def cmd_verify(args) -> int:
    from .hw import device_slug
    from .shapes import resolve
    dev = torch.device("cuda")
    spec, table = _spec_and_table(args.untuned)
    cases = resolve(args.configs)
    records, demoted, failures = verify_table(table, spec, cases, dev, args.trials,
                                              args.margin, args.demote)
    print(f"{'case':<8} {'plan':<40} {'envelope':>9} verdict")
    for rec in records:
        env = rec.get("envelope")
        verdict = ("SKIP (" + rec["reason"] + ")" if rec.get("checked") is False else
                   "ERR " + rec["error"] if "error" in rec else
                   ("PASS" if rec["passed"] else "FAIL")
                   + (f" but > margin {args.margin}" if env is not None and env > args.margin
                      else ""))
        print(f"{rec['case']:<8} {rec['plan']:<40} "
              f"{'-' if env is None else f'{env:9.4f}':>9} {verdict} ({rec['source']})",
              flush=True)
    if args.json_out:
        with open(args.json_out, "w", encoding="utf-8") as f:
            json.dump({"gpu": spec.summary(), "arch": spec.arch, "untuned": args.untuned,
                       "margin": args.margin, "records": records}, f, indent=2)
    if demoted:
        table.save(spec.arch, table.device or device_slug(spec))
        for c, p, u in demoted:
            print(f"demoted {c} {p} (re-measured {u:.3f}) to the safe plan")
    if failures:
        print(f"{len(failures)} FAILURE(S)")
        return 1
    print("all cases pass the organizer's tolerance")
    return 0


def spread_of(runs: Sequence[Sequence[dict]]) -> Dict[str, float]:
    """Largest envelope difference per case over verify records of separate processes."""
    seen: Dict[str, List[float]] = {}
    for recs in runs:
        for r in recs:
            if r.get("envelope") is not None:
                seen.setdefault(r["case"], []).append(float(r["envelope"]))
    return {k: max(v) - min(v) for k, v in seen.items() if len(v) > 1}


def cmd_spread(args) -> int:
    """Re-measure the run-to-run envelope spread: `verify` over the table in several fresh
    processes (`kernelforge/numerics.py:48-68` derives the demotion margin from it)."""
    runs = []
    workdir = os.path.abspath(args.workdir)
    os.makedirs(workdir, exist_ok=True)
    for i in range(args.processes):
        out = os.path.join(workdir, f"spread_{i}.json")
        cmd = [sys.executable, "-u", "-m", "techjam2026_amd.search", "verify", "--configs",
               *args.configs, "--trials", str(args.trials), "--json-out", out]
        proc = subprocess.run(cmd, cwd=os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                              timeout=args.timeout)
        if proc.returncode not in (0, 1) or not os.path.exists(out):
            print(f"[spread] process {i} exited {proc.returncode}", flush=True)
            return 1
        with open(out, encoding="utf-8") as f:
            runs.append(json.load(f)["records"])
    s = spread_of(runs)
    for k, v in sorted(s.items()):
        print(f"[spread] {k}: {v:.4f}")
    print(f"[spread] max {max(s.values()) if s else float('nan'):.4f} over "
          f"{args.processes} processes", flush=True)
    return 0


def main(argv: Optional[Sequence[str]] = None) -> int:
    import argparse
    ap = argparse.ArgumentParser(prog="python -m techjam2026_amd.search")
    sub = ap.add_subparsers(dest="cmd", required=True)
    sp = sub.add_parser("sweep", help="search each case and write the device table")
    sp.add_argument("--configs", nargs="+", default=["C1", "C2", "C3", "C4"])
    sp.add_argument("--margin", type=float, default=ADMISSION_MARGIN)
    sp.add_argument("--trials", type=int, default=TRIALS)
    sp.add_argument("--case-budget", type=float, default=600.0)
    sp.set_defaults(func=cmd_sweep)
    sp = sub.add_parser("verify", help="re-measure the frozen table")
    sp.add_argument("--configs", nargs="+", default=["C1", "C2", "C3", "C4"])
    sp.add_argument("--margin", type=float, default=DEMOTION_MARGIN)
    sp.add_argument("--trials", type=int, default=TRIALS)
    sp.add_argument("--demote", action="store_true")
    sp.add_argument("--untuned", action="store_true", help="ignore the table (default plans)")
    sp.add_argument("--json-out", default=None)
    sp.set_defaults(func=cmd_verify)
    sp = sub.add_parser("spread", help="run-to-run envelope spread over fresh processes")
    sp.add_argument("--configs", nargs="+", default=["C1", "C2", "C3", "C4"])
    sp.add_argument("--processes", type=int, default=3)
    sp.add_argument("--trials", type=int, default=TRIALS)
    sp.add_argument("--workdir", default=".")
    sp.add_argument("--timeout", type=float, default=600.0)
    sp.set_defaults(func=cmd_spread)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("search: no GPU visible", flush=True)
        return 2
    return args.func(args)


if __name__ == "__main__":
    raise SystemExit(main())
