"""The official-shape harness: shape list, flags and output parsing (CPU only).

Mirrors the reference's `scripts/official_all.py` parsing of the organizer's printed
lines; the GPU run itself is `python -m techjam2026_amd.official all`.
"""
from __future__ import annotations

from techjam2026_amd import official as O
from techjam2026_amd.shapes import parse_spec


def test_fourteen_official_shapes_all_causal():
    specs = O.official_shapes()
    assert len(specs) == 14 and specs[-1] == O.LONG_SHAPE
    for s in specs:
        c = parse_spec(s)
        assert c.causal and c.ffn_dim == c.d_model and c.d_model % c.num_heads == 0
        assert c.num_layers == (2 if s == O.LONG_SHAPE else 4)


def test_flags_round_trip_the_spec():
    f = O._flags("B64-S1024-d128-H4-F128-L4-causal")
    args = O.parser().parse_args(f)
    assert (args.batch_size, args.seq_len, args.d_model, args.heads, args.ffn_dim,
            args.layers, args.causal) == (64, 1024, 128, 4, 128, 4, True)
    assert (args.warmup, args.repeats, args.benchmark_rounds, args.accuracy_trials) == (20, 100, 3, 5)
    assert (args.rtol, args.atol) == (0.02, 0.002)


def test_parse_reads_the_printed_record():
    text = "\n".join([
        "summary: PASS | max_abs=0.000123 | max_rel=0.5 | failed=0/100",
        "[kernelforge] gfx950 torch.float32 -> f16x3+graph (default)",
        "baseline : median=2.5000 ms | mean=2.6 ms | p90=2.7 ms | min=2.4 ms | throughput=1.00 token/s",
        "optimized: median=0.5000 ms | mean=0.6 ms | p90=0.7 ms | min=0.4 ms | throughput=5.00 token/s",
        "speedup  : 5.000x based on median latency"])
    got = O._parse(text)
    assert got == {"passed": True, "max_abs": 0.000123, "baseline_ms": 2.5, "ours_ms": 0.5,
                   "speedup": 5.0, "plan": "f16x3+graph", "plan_source": "default"}
    assert O._parse("summary: FAIL | max_abs=1.0 | max_rel=2 | failed=3/4")["passed"] is False
