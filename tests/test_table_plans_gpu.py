"""The plans the gfx950 dispatch table actually serves, under oracle parity at full size.

The reference re-measures its frozen table before trusting it (`kernelforge/cli.py:149-260`,
verify --demote) and the organizer gates every shape on five seeded trials
(`torch_transformer_benchmark.py:382-393`). Here each BASELINE config is built the way
the organizer builds it -- `UserOptimizedTransformer`, weights copied with strict=True,
so the real table lookup picks the plan bench.py times -- and its output is checked
against the oracle over the organizer's five accuracy seeds (1234-1238) and its timing
input (seed 1234 + 100000), on each of the three Xavier weight draws the table was admitted
on, at the config's full batch. Bar: the organizer's OR rule with envelope utilisation
<= 0.8 (north star); the plans were admitted at <= 0.74 over the same draws and inputs.

Oracle: `oracle.reference` in fp32 -- on the CPU where it finishes in seconds (C1, C2),
otherwise on the GPU with query-chunked attention (C3 at B64, C4, C5), which is first
checked against the CPU oracle on a slice of the same input (batch rows are independent).
"""
from __future__ import annotations

import dataclasses
import json
import os

import pytest
import torch

from oracle import reference as R
from techjam2026_amd import harness
from techjam2026_amd.numerics import check
from techjam2026_amd.shapes import config

from conftest import make_model, params_of

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
ENVELOPE_TARGET = 0.8
ACCURACY_SEEDS = (1234, 1235, 1236, 1237, 1238)
TIMING_SEED = 1234 + 100000
TABLE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                     "techjam2026_amd", "results", "dispatch_gfx950__256cu-288gb_gfx950.json")


def _table_plan_name(case) -> str:
    with open(TABLE, encoding="utf-8") as f:
        entries = json.load(f)["entries"]
    from techjam2026_amd.dispatch import shape_signature
    sig = shape_signature(case)
    hit = [e for e in entries if e["signature"] == sig and e["dtype"] == "float32"]
    return hit[0]["plan"]["name"] if hit else None


def _drop_in(cfg, weight_seed):
    from techjam2026_amd.submission import UserOptimizedTransformer
    base = make_model(cfg, seed=weight_seed, device="cpu")
    opt = UserOptimizedTransformer(cfg)
    opt.load_state_dict(base.state_dict(), strict=True)
    return base, opt.to(DEV, torch.float32).eval()


def _oracle(p, x, m, cfg, on_gpu, chunk=1024):
    with torch.inference_mode():
        if on_gpu:
            pd = {k: v.to(DEV) for k, v in p.items()}
            return R.stack_forward_rows(pd, x.to(DEV), m.to(DEV), cfg.num_heads, cfg.causal,
                                        chunk=chunk)
        return R.stack_forward(p, x, m, cfg.num_heads, cfg.causal)


def _check_gpu_oracle_against_cpu(p, x, m, cfg, rows=2):
    """The GPU-run oracle agrees with the CPU one on a slice of the batch."""
    cpu = _oracle(p, x[:rows], m[:rows], cfg, False)
    gpu = _oracle(p, x[:rows], m[:rows], cfg, True).cpu()
    res = check(cpu, gpu)
    print(f"[oracle] GPU vs CPU oracle, {rows} rows: {res}", flush=True)
    assert res.passed and res.envelope_utilization < 0.05, str(res)


def _run(name, weight_seed, seeds, gpu_oracle, batch=None, expect_exact=True,
         cross_check=True, chunk=1024):
    case = config(name)
    if batch is not None:
        case = dataclasses.replace(case, batch_size=batch)
    cfg = case.to_config()
    base, opt = _drop_in(cfg, weight_seed)
    p = params_of(base)
    worst, envs = 0.0, []
    for i, seed in enumerate(seeds):
        x, m = harness.generate_random_case(cfg, "cpu", torch.float32, seed,
                                            case.padding_ratio, case.input_scale)
        if gpu_oracle and cross_check and i == 0:
            _check_gpu_oracle_against_cpu(p, x, m, cfg)
        with torch.inference_mode():
            out = opt(x.to(DEV), m.to(DEV))
        assert opt._impl is not None and not opt._failed, "native path must have run"
        ref = _oracle(p, x, m, cfg, gpu_oracle, chunk)
        res = check(ref, out)
        envs.append(round(res.envelope_utilization, 4))
        print(f"[table] {name} weights={weight_seed} seed={seed} plan={opt._plan.name} "
              f"({opt._source}): {res}", flush=True)
        assert res.passed, str(res)
        assert torch.count_nonzero(out[~m.to(DEV)]) == 0, "padded rows must be zero"
        worst = max(worst, res.envelope_utilization)
        del out, ref
    if expect_exact:
        assert opt._source == "exact", f"{name}: plan came from {opt._source}"
        assert opt._plan.name == _table_plan_name(case)
    print(f"[table] {name} weights={weight_seed}: per-seed envelopes {envs}, worst "
          f"{worst:.4f}", flush=True)
    assert worst <= ENVELOPE_TARGET, f"{name} plan {opt._plan.name}: envelope {worst:.3f}"
    return worst


WEIGHT_DRAWS = (7, 8, 9)       # budget.WEIGHT_DRAWS: the draws the table was admitted on


@pytest.mark.parametrize("weights", WEIGHT_DRAWS)
@pytest.mark.parametrize("name,gpu_oracle", [("C1", False), ("C2", False), ("C3", True),
                                             ("C4", True)])
def test_dispatched_plan_passes_over_the_organizer_seeds(name, gpu_oracle, weights):
    """C1-C4 through the drop-in at their full BASELINE shapes (C3 at batch 64), with the
    table's plan, over the five accuracy seeds and the timing input, on each of the three
    Xavier weight draws the plan was admitted on (admission 0.74, `numerics`)."""
    _run(name, weights, ACCURACY_SEEDS + (TIMING_SEED,), gpu_oracle,
         cross_check=weights == WEIGHT_DRAWS[0])


@pytest.mark.parametrize("weights", WEIGHT_DRAWS)
def test_c5_dispatched_plan_over_seeds_and_weight_draws(weights):
    """C5 (S = 65536): its table plan, every output element against the chunked oracle on
    the GPU, on the first accuracy seed and the timing input of each weight draw. (The GPU
    oracle's agreement with the CPU one is checked at C3 and C4; a CPU pass over two
    S = 65536 rows would take minutes.)"""
    _run("C5", weights, (1234, TIMING_SEED), True, cross_check=False, chunk=4096)
