"""Official shape 14 at full length (B32 S100000 d1024 H16, causal): the shape the
reference layer cannot run (its [B, H, S, S] score tensor is 18.6 TB).

The drop-in runs the whole batch; batch elements are independent in this model, so the
output of sampled sequences is checked against the chunked oracle run on the GPU for
those sequences alone, over every element of them, with the organizer's gate
(`scripts/shape14.py` reports the same shape; its accuracy claim in the reference rests
on sampled query rows against an exact reference).
"""
from __future__ import annotations

import pytest
import torch

from oracle import reference as R
from techjam2026_amd.dispatch import default_plan
from techjam2026_amd.model import TransformerConfig
from techjam2026_amd.numerics import check
from techjam2026_amd.official import LONG_SHAPE, official_shapes
from techjam2026_amd.optimized import build_shared

from conftest import make_model, params_of

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def test_official_shape14_full_length_sampled_sequences():
    cfg = TransformerConfig(32, 100000, 1024, 16, 1024, 2, True)
    base = make_model(cfg, device=DEV)
    ours = build_shared(cfg, default_plan(torch.float32), base)
    g = torch.Generator(device=DEV).manual_seed(1234)
    x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, device=DEV, generator=g)
    m = torch.ones(cfg.batch_size, cfg.seq_len, dtype=torch.bool, device=DEV)
    print("[shape14] drop-in forward, whole batch", flush=True)
    with torch.inference_mode():
        out = ours(x, m)
    torch.cuda.synchronize()
    p = {k: v.to(DEV) for k, v in params_of(base).items()}
    for b in (0, cfg.batch_size - 1):
        print(f"[shape14] chunked oracle, sequence {b}", flush=True)
        with torch.inference_mode():
            ref = R.stack_forward_rows(p, x[b:b + 1], m[b:b + 1], cfg.num_heads, cfg.causal,
                                       chunk=2048)
        res = check(ref, out[b:b + 1])
        print(f"[shape14] sequence {b}: {res}", flush=True)
        assert res.passed and res.envelope_utilization <= 0.8, str(res)
        del ref


def _official_args(spec):
    from techjam2026_amd.official import _flags, parser
    return parser().parse_args(_flags(spec))


@pytest.mark.parametrize("spec", [s for s in official_shapes() if s != LONG_SHAPE])
def test_official_shape_passes_the_organizer_accuracy_gate(spec):
    """The organizer's accuracy flow (`torch_transformer_benchmark.py:359-425`, run per
    shape by `scripts/official_all.py:98-102`): default-initialised weights from the
    seed, five seeded trials, the reference layer on the same GPU against the drop-in
    (through its dispatch table), the OR rule; here also envelope <= 0.8. Accuracy only."""
    from techjam2026_amd.official import _models, accuracy_trials
    args = _official_args(spec)
    cfg, baseline, optimized = _models(args, DEV, torch.float32)
    print(f"[official] {spec}", flush=True)
    acc = accuracy_trials(cfg, baseline, optimized, DEV, torch.float32, args.seed,
                          args.accuracy_trials, args.padding_ratio, args.input_scale)
    assert optimized._impl is not None and not optimized._failed, "native path must have run"
    print(f"[official] {spec}: plan {optimized._plan.name} ({optimized._source}), "
          f"envelopes {[round(e, 4) for e in acc['envelopes']]}", flush=True)
    assert acc["passed"] and acc["envelope"] <= 0.8, acc
    del baseline, optimized
    torch.cuda.empty_cache()
