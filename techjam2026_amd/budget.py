"""Per-stage precision error budget (`kernelforge/budget.py:66-167`).

Envelope utilisation = max |e| / max(atol, rtol*|ref|) over every output element,
worst over several seeds (1234, 1235, ...). `stage_budget` runs a control plan with every
stage at the control precision, then narrows one stage at a time to each candidate
precision, then all stages together, then all stages plus the residual stream (16-bit
candidates), so that each stage's share of the tolerance is measured rather than
guessed. The reference here is the reference layer itself (the
`BaselineTransformer` forward) in float32 on the same device: on gfx950 that is true
fp32 arithmetic (there is no TF32-like matrix mode), which is what the north-star gate
compares against. Where its [B, H, S, S] score tensor cannot be formed (> 8 GiB), the same
forward is evaluated streamed (`model.streamed_reference_forward`).
"""
from __future__ import annotations

import dataclasses
import weakref
from typing import List, Optional, Sequence

import torch

from . import harness
from .model import BaselineTransformer, streamed_reference_forward
from .numerics import ATOL, RTOL, CheckResult, check
from .optimized import STAGES, Plan, build_shared
from .shapes import Case

CANDIDATES = ("float16", "bfloat16", "bf16x3", "float32", "f16x3p", "f16x2", "f16x2p", "f16x3s")
# Xavier weight draws a plan is admitted and verified on (the benchmark's weights are the
# first); worst case over all of them
WEIGHT_DRAWS = (7, 8, 9)
ATTN_ONLY = ("f16x3p", "f16x2p", "f16x3s")   # precisions that differ from another only in attention


@dataclasses.dataclass
class BudgetRow:
    case: str
    stage: str
    dtype: str
    utilization: float
    max_abs: float
    passed: bool
    error: str = ""

    def verdict(self) -> str:
        if self.error:
            return "ERROR"
        if not self.passed:
            return "FAIL"
        return "tight" if self.utilization > 0.5 else "ok"


def reference_model(case: Case, device, weight_seed: int = 7) -> BaselineTransformer:
    cfg = case.to_config()
    model = BaselineTransformer(cfg)
    harness.init_weights_(model, weight_seed)
    return model.to(device, case.torch_dtype).eval()


def must_stream(cfg) -> bool:
    """The reference layer's fp32 [B, H, S, S] score tensor would exceed 8 GiB
    (`kernelforge/dispatch.py:291-298`): its reference answer is then streamed."""
    return cfg.batch_size * cfg.num_heads * cfg.seq_len ** 2 * 4 > 8 * 2 ** 30


# Reference outputs per reference module and input: the reference does not depend on the
# plan under test, so a search computes it once per seed. Keyed weakly on the module, so
# the entries (device tensors) go when the module does.
_REF_CACHE: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()


def reference_output(case: Case, base: BaselineTransformer, seed: int, x, m):
    per = _REF_CACHE.setdefault(base, {})
    key = (case.label(), seed)
    hit = per.get(key)
    if hit is None:
        with torch.inference_mode():
            if must_stream(case.to_config()):
                hit = streamed_reference_forward(base, x, m)
            else:
                hit = base(x, m)
        per[key] = hit
    return hit


def reference_models(case: Case, device, draws: Sequence[int] = WEIGHT_DRAWS
                     ) -> List[BaselineTransformer]:
    """One reference module per weight draw (keep them for the duration of a search or a
    verification: their reference outputs are cached on them)."""
    return [reference_model(case, device, w) for w in draws]


def evaluate(case: Case, plan: Plan, device, trials: int = 3, rtol: float = RTOL,
             atol: float = ATOL, base: Optional[BaselineTransformer] = None,
             extra_seeds: Sequence[int] = (),
             bases: Optional[Sequence[BaselineTransformer]] = None) -> CheckResult:
    """Worst check over `trials` seeded inputs (seeds 1234 + t), then `extra_seeds`, for
    each reference module of `bases` (one per weight draw; default: `base`, else the first
    draw). The reference is the reference layer on the same device, streamed where its
    score tensor cannot be formed. The worst result's note names its draw and seed."""
    if not bases:
        bases = [base if base is not None else reference_model(case, device)]
    worst = None
    for d, ref_model in enumerate(bases):
        opt = build_shared(case.to_config(), plan, ref_model)
        for seed in [1234 + t for t in range(trials)] + list(extra_seeds):
            x, m = harness.generate_random_case(case.to_config(), device, case.torch_dtype,
                                                seed, case.padding_ratio, case.input_scale)
            ref = reference_output(case, ref_model, seed, x, m)
            with torch.inference_mode():
                out = opt(x, m)
            res = check(ref, out, rtol=rtol, atol=atol)
            del out
            if worst is None or res.envelope_utilization > worst.envelope_utilization:
                worst = dataclasses.replace(res, note=f"weight draw {d}, seed {seed}")
        del opt
    return worst


def stage_budget(case: Case, device, control: Optional[Plan] = None, trials: int = 3,
                 candidates: Sequence[str] = CANDIDATES) -> List[BudgetRow]:
    control = control or Plan(name="control", compute_dtype="f16x3")
    base = reference_model(case, device)
    rows: List[BudgetRow] = []

    def run(stage: str, dtype: str, plan: Plan) -> None:
        try:
            r = evaluate(case, plan, device, trials, base=base)
            rows.append(BudgetRow(case.name, stage, dtype, r.envelope_utilization,
                                  r.max_abs_error, r.passed))
        except Exception as e:   # a precision the kernels refuse is a row, not a crash
            rows.append(BudgetRow(case.name, stage, dtype, float("nan"), float("nan"),
                                  False, f"{type(e).__name__}: {str(e)[:80]}"))

    run("(control)", control.compute_dtype, control)
    for stage in STAGES:
        for dt in candidates:
            if dt in ATTN_ONLY and stage != "attn":
                continue
            run(stage, dt, control.with_override(stage, dt))
    for dt in (c for c in candidates if c not in ATTN_ONLY):
        plan = control
        for stage in STAGES:
            plan = plan.with_override(stage, dt)
        run("(all stages)", dt, dataclasses.replace(plan, name=f"all:{dt}"))
    # the residual stream accumulates over 2L sublayers: narrow storage compounds there
    # rather than merely rounding (`kernelforge/budget.py:146-167`)
    for dt in (c for c in candidates if c in ("float16", "bfloat16")):
        plan = control
        for stage in STAGES:
            plan = plan.with_override(stage, dt)
        run("(all + residual)", dt, dataclasses.replace(plan, residual_dtype=dt,
                                                        name=f"all+res:{dt}"))
    return rows


def format_rows(rows: List[BudgetRow]) -> str:
    out = [f"{'case':<8} {'stage':<14} {'dtype':<9} {'envelope':>9} {'max_abs':>10}  verdict",
           "-" * 64]
    for r in rows:
        u = "nan" if r.utilization != r.utilization else f"{r.utilization:9.4f}"
        a = "nan" if r.max_abs != r.max_abs else f"{r.max_abs:10.3e}"
        out.append(f"{r.case:<8} {r.stage:<14} {r.dtype:<9} {u:>9} {a:>10}  {r.verdict()}"
                   + (f"  {r.error}" if r.error else ""))
    return "\n".join(out)


def main(argv: Optional[Sequence[str]] = None) -> int:
    """`python -m techjam2026_amd.budget --configs C2 C3`: measure the per-stage budget on
    this GPU and write it next to the dispatch tables (kernelforge/budget.py:170-214)."""
    import argparse
    import os

    from . import hw
    from .dispatch import TABLE_DIR
    from .shapes import resolve

    ap = argparse.ArgumentParser(description=main.__doc__)
    ap.add_argument("--configs", nargs="+", default=["C2"],
                    help="config names (C1..C5) or shape specs")
    ap.add_argument("--trials", type=int, default=3)
    ap.add_argument("--out", default=None, help="output file (default: results/error_budget_<device>.txt)")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("budget: no GPU visible", flush=True)
        return 2
    dev = torch.device("cuda")
    slug = hw.device_slug(hw.probe(0))
    out = args.out or os.path.join(TABLE_DIR, f"error_budget_{slug}.txt")
    lines = [f"# per-stage error budget on {slug}; control = f16x3 on every stage; "
             f"worst of {args.trials} seeds; reference = the fp32 reference layer on the same GPU",
             f"# command: python -m techjam2026_amd.budget --configs {' '.join(args.configs)}"
             f" --trials {args.trials}"]
    for case in resolve(args.configs):
        print(f"[budget] {case.name} {case.label()}", flush=True)
        rows = stage_budget(case, dev, trials=args.trials)
        text = format_rows(rows)
        print(text, flush=True)
        lines += ["", f"## {case.name}: {case.label()}", text]
    os.makedirs(os.path.dirname(out), exist_ok=True)
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"[budget] wrote {out}", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
