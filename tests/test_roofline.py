"""Stack roofline floor (CPU): the per-config floor of the metric's reporting item --
sum over kernels of flops / MFMA peak and LayerNorm bytes / 8 TB/s -- against the
per-config figures derived independently for the benchmark's configs (GEMM floor at the
fp16 MFMA peak, causal attention at full length, 2L+1 LayerNorms of 16 B per element)."""
from __future__ import annotations

import pytest

from techjam2026_amd import roofline
from techjam2026_amd.shapes import config

# (GEMM fp16-peak floor, attention fp16 floor, LN floor) in ms, per config
DERIVED = {"C2": (0.124, 0.010, 0.109), "C3": (0.015, 0.021, 0.109),
           "C4": (0.660, 0.220, 0.336), "C5": (2.639, 28.148, 2.685)}


@pytest.mark.parametrize("name", sorted(DERIVED))
def test_floor_at_full_lengths_matches_the_derived_table(name):
    cfg = config(name).to_config()
    f = roofline.stack_floor_ms(cfg, [cfg.seq_len] * cfg.batch_size)
    assert f["floor_ms_fp16_peak"] == pytest.approx(sum(DERIVED[name]), rel=0.01, abs=2e-3)


def test_plan_floor_prices_each_stage_at_its_useful_peak():
    cfg = config("C2").to_config()
    lens = [cfg.seq_len] * cfg.batch_size
    prec = {"attn": "f16x3", "out_proj": "f16x3", "ffn1": "f16x3", "ffn2": "f16x3"}
    f = roofline.stack_floor_ms(cfg, lens, prec)
    ln = roofline.stack_floor_ms(cfg, lens)["floor_ms_fp16_peak"] - 0.124 - 0.010
    # every product at a third of the fp16 peak, LayerNorms unchanged
    assert f["floor_ms_plan"] == pytest.approx(3 * (0.124 + 0.010) + ln, rel=0.01)
    narrow = roofline.stack_floor_ms(cfg, lens, dict(prec, ffn1="float16"))
    assert narrow["floor_ms_plan"] < f["floor_ms_plan"]
