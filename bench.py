#!/usr/bin/env python3
"""Benchmark of the native transformer-layer-stack forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C5]

A "step" is one forward of the layer stack over one batch of synthetic input, through
the drop-in `UserOptimizedTransformer` (dispatch table -> FusedTransformer, hipGraph
replay). Workload: BASELINE.json config C5 (2 layers, d_model 1024, 16 heads, FFN 1024,
batch 4, seq 65536, fp32, causal + key padding with valid lengths in [32768, 65536]).
BASELINE's metric is quoted per shape and names no single config, so the line is the
largest single-GPU configuration; the other configs are reported in `per_config`.
Inputs are drawn on a CPU generator (seed 1234 + 100000, the organizer's timing seed)
and copied to HBM before the timed region; weights are Xavier-uniform from seed 7.

Printed: one JSON line. `value` is the median per-step forward latency in ms
(BASELINE's metric is "median layer-stack forward ms"; lower is better).
`roofline` is for the dominant kernel of the forward (at C5 the attention), measured
live with HIP events on the launch stream during an instrumented pass of K eager
forwards: algorithmic FLOPs (padding-aware for attention, from the seeded lengths) or
bytes per launch / mean launch duration (raw event-pair time), against MI355X's published
dense peak; its `traffic` is the HBM bytes per launch from the committed rocprofv3
FETCH_SIZE / WRITE_SIZE measurement of that kernel (null when none is recorded).
`cpu_baseline` is the oracle (the reference layer restated in PyTorch, fp32) timed on
this host's cores on the same input, rank 0 only, on a bounded sample; the same leg
checks this run's output against the oracle (`envelope_vs_oracle`; on the GPU with
query-chunked attention where the sequence is long).
The plan is the measured gfx950 dispatch table's entry for the shape
(`config.stage_precision`); `control_f16x3_ms` is the all-split-fp32 plan on the same
weights and input.
`per_config` carries every BASELINE config (median forward ms, attention and LayerNorm
rates, roofline floor, CPU baseline), `attn_hd128` the attention target check at
head_dim 128, S = 8192.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "median layer-stack forward ms per shape; attn MFMA util %; LayerNorm HBM GB/s"


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C5")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="bound on the CPU-baseline sample's wall time")
    ap.add_argument("--no-per-config", action="store_true",
                    help="skip the medians of the other BASELINE configs and the hd128 check")
    ap.add_argument("--per-config-steps", type=int, default=50)
    ap.add_argument("--per-config-warmup", type=int, default=20)
    ap.add_argument("--label-log", default=None,
                    help="write the instrumented pass's [label, dispatches] sequence (JSON), "
                         "for attributing a profiler's per-dispatch counters to kernels")
    return ap.parse_args()


def build(name: str):
    """(case, cfg, model on cuda:0, x, mask, x_cpu, mask_cpu, reference params on CPU)."""
    import torch
    from techjam2026_amd import harness
    from techjam2026_amd.model import BaselineTransformer
    from techjam2026_amd.shapes import config as get_config
    from techjam2026_amd.submission import UserOptimizedTransformer
    case = get_config(name)
    cfg = case.to_config()
    dev = torch.device("cuda:0")
    base = BaselineTransformer(cfg)
    harness.init_weights_(base, 7)
    params_cpu = {k: v.detach().clone() for k, v in base.state_dict().items()}
    model = UserOptimizedTransformer(cfg)
    model.load_state_dict(base.state_dict(), strict=True)
    model = model.to(dev, torch.float32).eval()
    x_cpu, m_cpu = harness.generate_random_case(cfg, "cpu", torch.float32, 1234 + 100000,
                                                case.padding_ratio, case.input_scale)
    return case, cfg, model, x_cpu.to(dev), m_cpu.to(dev), x_cpu, m_cpu, params_cpu


def time_forward(model, x, m, steps: int, warmup: int):
    """(median ms, wall ms per step, last output) of `steps` event-timed forwards."""
    import torch
    with torch.inference_mode():
        for _ in range(max(1, warmup)):
            out = model(x, m)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    with torch.inference_mode():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            starts[i].record()
            out = model(x, m)
            ends[i].record()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    samples = [a.elapsed_time(b) for a, b in zip(starts, ends)]
    return statistics.median(samples), (t1 - t0) * 1e3 / steps, out


def control_median(model, x, m, steps: int, warmup: int) -> float:
    """Median forward ms of the all-f16x3 plan (hipGraph) on the same weights and input:
    the table's plan narrows stages to fp16 where the measured budget allows, and this
    number shows what the split-fp32 plan alone does."""
    import torch
    from techjam2026_amd.optimized import LADDER, FusedTransformer
    with torch.device("meta"):
        ctl = FusedTransformer(model.config, LADDER["graph"])
    # the drop-in's own parameters (its native module's copies are inference tensors)
    own = {k: v for k, v in model.state_dict().items() if not k.startswith("_impl.")}
    ctl.load_state_dict(own, assign=True)
    ctl.eval()
    med, _, _ = time_forward(ctl, x, m, steps, warmup)
    del ctl
    torch.cuda.empty_cache()
    return med


def instrumented(impl, x, m, passes: int, label_log: str = None) -> dict:
    """Per-kernel HIP-event timing of `passes` eager forwards (kernels.KernelTimer)."""
    import torch
    from techjam2026_amd import kernels
    kernels.TIMER = kernels.KernelTimer(pad_us=100.0)
    try:
        with torch.inference_mode():
            for _ in range(passes):
                impl._eager_forward(x, m)
        if label_log:
            with open(label_log, "w", encoding="utf-8") as f:
                json.dump({"note": "kf kernel dispatches of the instrumented pass, in order "
                                   "(the last ones of the run)",
                           "labels": kernels.TIMER.dispatch_labels()}, f)
        return kernels.TIMER.summary()
    finally:
        kernels.TIMER = None


def attention_and_ln(per_kernel: dict, lengths, cfg, precision: str):
    """Attention TFLOP/s (padding-aware and causal counts; MFMA share of the dense peak
    of the precision used) and LayerNorm bytes/s, from an instrumented pass."""
    from techjam2026_amd import roofline
    attn_flops = roofline.attention_flops_padded(lengths, cfg.seq_len, cfg.d_model,
                                                 cfg.num_heads, 1, cfg.causal)
    attn_causal = roofline.attention_flops(cfg.batch_size, cfg.seq_len, cfg.d_model,
                                           cfg.num_heads, 1, cfg.causal)
    attn = None
    for label, r in per_kernel.items():
        if label.startswith("flash"):
            r["flops"] = attn_flops
            r["tflops"] = attn_flops / (r["mean_ms"] / 1e3) / 1e12
            split = roofline.SPLIT_FACTOR.get(precision, 1)
            attn = {"kernel": label, "mean_ms": round(r["mean_ms"], 5),
                    "tflops_padding_aware": round(r["tflops"], 2),
                    "tflops_causal_count": round(attn_causal / (r["mean_ms"] / 1e3) / 1e12, 2),
                    "mfma_util_pct": round(100 * r["tflops"] * split
                                           / roofline.mfma_peak_tflops(precision), 2),
                    "precision": precision}
    ln = {k: v for k, v in per_kernel.items() if k.startswith("add_mask_ln")}
    ln_bytes = sum(v["bytes"] * v["launches"] for v in ln.values())
    ln_ms = sum(v["total_ms"] for v in ln.values())
    lnd = None
    if ln_ms:
        gbs = ln_bytes / (ln_ms / 1e3) / 1e9
        lnd = {"gbs": round(gbs, 1), "frac_of_hbm_peak": round(gbs / roofline.HBM_GBS, 4),
               "launches": sum(v["launches"] for v in ln.values())}
    return attn, lnd


def floor_of(cfg, lengths, plan, median_ms: float) -> dict:
    """The forward's roofline floor (fp16-peak convention and at the plan's precisions) and
    the fraction of it the measured median reaches."""
    import torch
    from techjam2026_amd import roofline
    from techjam2026_amd.optimized import STAGES
    floor = roofline.stack_floor_ms(cfg, lengths,
                                    {s: plan.stage_precision(s, torch.float32) for s in STAGES})
    floor["frac_fp16_peak"] = round(floor["floor_ms_fp16_peak"] / median_ms, 4)
    floor["frac_plan"] = round(floor["floor_ms_plan"] / median_ms, 4)
    return floor


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


# CPU-baseline protocol per config (`torch_transformer_benchmark.py:501-506`): warm-up
# forwards, timed repeats. A forward longer than CPU_LONG_MS is not warmed up again: the
# first call is the warm-up and one more is timed. C5's full forward is many minutes of CPU
# work, so it is sampled instead (`cpu_sampled_long`).
CPU_PROTOCOL = {"C1": (20, 100), "C2": (1, 3), "C3": (1, 3), "C4": (1, 3)}
CPU_LONG_MS = 4000.0
LONG_SEQ = 8192          # above this, the oracle's attention runs query-chunked
CPU_CHUNK = 1024         # query rows per oracle attention chunk on the CPU
CPU_SAMPLE_CHUNKS = 6    # attention chunks timed per sampled layer


def cpu_sampled_long(cfg, params_cpu, x_cpu, m_cpu) -> tuple:
    """(estimated ms of the whole forward, description) for a long-sequence config.

    Layer 1 of batch row 0 is timed in two parts with the oracle's own arithmetic: every
    operation except the attention core over the whole row (LayerNorms, projections,
    GELU; cost linear in the row), and the attention core for CPU_SAMPLE_CHUNKS query
    chunks spread evenly over the row's causal range. A chunk of rows [lo, hi) reads keys
    [0, hi), so its cost is proportional to hi: the sampled time is scaled by the row's
    total key reads over the sampled ones. Layers have one shape and batch rows are
    independent, so the sum is scaled by layers x batch rows."""
    import torch
    from oracle import reference as R
    S, H = cfg.seq_len, cfg.num_heads
    x, m = x_cpu[:1], m_cpu[:1]
    p, pre = params_cpu, "layers.0."
    at = pre + "attention."
    with torch.inference_mode():
        t0 = time.perf_counter_ns()
        n1 = R.layer_norm(x, p[pre + "norm1.weight"], p[pre + "norm1.bias"])
        q, k, v = (R._split_heads(R.linear(n1, p[at + f"{w}_proj.weight"], p[at + f"{w}_proj.bias"]),
                                  1, S, H) for w in ("q", "k", "v"))
        ctx = torch.zeros_like(q)     # stands in for the attention output below
        o = R.linear(ctx.transpose(1, 2).reshape(1, S, -1), p[at + "out_proj.weight"],
                     p[at + "out_proj.bias"])
        x1 = x + o.masked_fill(~m.bool()[..., None], 0)
        n2 = R.layer_norm(x1, p[pre + "norm2.weight"], p[pre + "norm2.bias"])
        hid = R.gelu_erf(R.linear(n2, p[pre + "ffn_in.weight"], p[pre + "ffn_in.bias"]))
        x2 = x1 + R.linear(hid, p[pre + "ffn_out.weight"], p[pre + "ffn_out.bias"])
        x2.masked_fill(~m.bool()[..., None], 0)
        dense_ms = (time.perf_counter_ns() - t0) / 1e6
        scale = q.shape[-1] ** -0.5
        starts = list(range(0, S, CPU_CHUNK))
        pick = sorted({starts[round(i * (len(starts) - 1) / max(CPU_SAMPLE_CHUNKS - 1, 1))]
                       for i in range(CPU_SAMPLE_CHUNKS)})
        n_keys = lambda lo: min(lo + CPU_CHUNK, S) if cfg.causal else S  # noqa: E731
        t0 = time.perf_counter_ns()
        for lo in pick:
            hi = min(lo + CPU_CHUNK, S)
            s = R._masked_scores(q[..., lo:hi, :], k, scale, m, cfg.causal, lo, n_keys(lo))
            pr = torch.softmax(s, dim=-1)
            torch.matmul(pr, v[..., :n_keys(lo), :])
        attn_ms = (time.perf_counter_ns() - t0) / 1e6
    ratio = sum(n_keys(lo) for lo in starts) / sum(n_keys(lo) for lo in pick)
    layer_ms = dense_ms + attn_ms * ratio
    rows_layers = cfg.batch_size * cfg.num_layers
    what = (f"oracle fp32, layer 1 of batch row 0: dense ops over the row {dense_ms / 1e3:.1f} s "
            f"+ attention core on {len(pick)} of {len(starts)} query chunks of {CPU_CHUNK} rows "
            f"{attn_ms / 1e3:.1f} s x {ratio:.2f} (key reads of the row / of the sample); "
            f"the layer estimate x{rows_layers} (layers x batch rows)")
    return layer_ms * rows_layers, what


def cpu_baseline_for(name: str, cfg, params_cpu, x_cpu, m_cpu) -> dict:
    """The oracle (the reference layer restated in PyTorch, fp32) on this host's CPU
    threads, on the same input as the GPU run, per CPU_PROTOCOL (sampled for long
    sequences)."""
    import torch
    from oracle import reference as R
    threads = torch.get_num_threads()
    base = {"unit": "ms", "cores": threads, "kind": "port",
            "host_cpu_count": os.cpu_count(), "cpu_model": cpu_model()}
    if cfg.seq_len > LONG_SEQ:
        est, what = cpu_sampled_long(cfg, params_cpu, x_cpu, m_cpu)
        return {"value": round(est, 2), **base, "sample": what}
    warm, reps = CPU_PROTOCOL.get(name, (1, 3))

    def fwd():
        return R.stack_forward(params_cpu, x_cpu, m_cpu, cfg.num_heads, cfg.causal)

    samples = []
    note = f"warm-up {warm}, {reps} timed"
    with torch.inference_mode():
        for i in range(warm):
            t0 = time.perf_counter_ns()
            fwd()
            first = (time.perf_counter_ns() - t0) / 1e6
            if i == 0 and first > CPU_LONG_MS:
                reps, note = 1, f"warm-up 1, 1 timed (a forward takes {first / 1e3:.1f} s)"
                break
        for _ in range(reps):
            t0 = time.perf_counter_ns()
            fwd()
            samples.append((time.perf_counter_ns() - t0) / 1e6)
    med = statistics.median(samples)
    return {"value": round(med, 2), **base,
            "sample": f"naive oracle.reference.stack_forward, fp32, {note}, median"}


def envelope_vs_oracle(cfg, params_cpu, x_cpu, m_cpu, out) -> float:
    """Envelope utilisation of `out` against the oracle's fp32 forward on the same input:
    on the CPU, or for long sequences on the GPU with query-chunked attention (every
    output element either way)."""
    import torch
    from oracle import reference as R
    from techjam2026_amd.numerics import check
    with torch.inference_mode():
        if cfg.seq_len > LONG_SEQ:
            dev = out.device
            pd = {k: v.to(dev) for k, v in params_cpu.items()}
            ref = R.stack_forward_rows(pd, x_cpu.to(dev), m_cpu.to(dev), cfg.num_heads,
                                       cfg.causal, chunk=4096)
            env = check(ref, out).envelope_utilization
            del ref, pd
            torch.cuda.empty_cache()
            return env
        ref = R.stack_forward(params_cpu, x_cpu, m_cpu, cfg.num_heads, cfg.causal)
        return check(ref, out.cpu()).envelope_utilization


def per_config_line(name: str, steps: int, warmup: int, cpu: bool = True) -> dict:
    """Median forward ms, tokens/s, attention and LayerNorm rates of one BASELINE config,
    with its CPU baseline beside it."""
    import torch
    from techjam2026_amd import roofline
    case, cfg, model, x, m, x_cpu, m_cpu, params_cpu = build(name)
    med, _, _ = time_forward(model, x, m, steps, warmup)
    plan = model._plan
    per_kernel = instrumented(model._impl, x, m, 3)
    attn, lnd = attention_and_ln(per_kernel, m_cpu.sum(1).tolist(), cfg,
                                 roofline.kernel_precision(
                                     plan.stage_precision("attn", torch.float32), True))
    floor = floor_of(cfg, m_cpu.sum(1).tolist(), plan, med)
    out = {"workload": case.label(), "median_ms": round(med, 4), "steps": steps,
           "warmup": warmup,
           "tokens_per_s": round(cfg.batch_size * cfg.seq_len * 1000.0 / med, 1),
           "plan": plan.name, "attn": attn, "layernorm": lnd, "roofline_floor": floor}
    del model, x, m
    torch.cuda.empty_cache()
    if cpu:
        print(f"[bench] CPU baseline {name}", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline_for(name, cfg, params_cpu, x_cpu, m_cpu)
        out["cpu_baseline"]["gpu_speedup"] = round(out["cpu_baseline"]["value"] / med, 1)
    return out


def attention_microbench(B: int = 2, H: int = 16, S: int = 8192, hd: int = 128) -> dict:
    """The attention target check at head_dim 128, S >= 4096 (no BASELINE config has it):
    causal, unpadded, operands already in the attention layout; the split-fp32 precision
    the stack uses and single-pass fp16."""
    import torch
    from techjam2026_amd import _lib as L, kernels as K, roofline
    torch.manual_seed(1234)
    q, k, v = (torch.randn(B, H, S, hd, device="cuda") for _ in range(3))
    res = {"shape": f"B{B}-H{H}-S{S}-d{hd}-causal"}
    for name, mode in (("f16x3", L.MMA_F16X3), ("f16x3p", L.MMA_F16X3), ("float16", L.MMA_F16)):
        p16 = name == "f16x3p"
        qq, kk, vv = (q, k, v) if mode == L.MMA_F16X3 else (q.half(), k.half(), v.half())
        k_hi, k_lo, vt_hi, vt_lo = K.attn_prep(kk, vv, mode)
        ops = K.AttnOperands(qq, k_hi, k_lo, vt_hi, vt_lo, mode)
        o = torch.empty_like(qq)
        for _ in range(2):
            K.flash_attention_ops(ops, causal=True, out=o, p16=p16)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 10
        a.record()
        for _ in range(n):
            K.flash_attention_ops(ops, causal=True, out=o, p16=p16)
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / n
        tf = roofline.attention_flops(B, S, H * hd, H, 1, True) / (ms / 1e3) / 1e12
        split = roofline.SPLIT_FACTOR.get(name, 1)
        res[name] = {"mean_ms": round(ms, 4), "tflops": round(tf, 1),
                     "mfma_util_pct": round(100 * tf * split / roofline.mfma_peak_tflops(name), 2)}
        del ops, o, k_hi, k_lo, vt_hi, vt_lo
    return res


def stage_of(label: str, cfg) -> str:
    """The plan stage a kernel label belongs to (its precision is that stage's)."""
    if label.startswith(("gemm_qkv", "flash")):
        return "attn"
    if label.startswith("gemm["):
        n, k = (int(v) for v in label[5:-1].split("x")[1:])
        if n == cfg.ffn_dim and k == cfg.d_model and n != k:
            return "ffn1"
        if k == cfg.ffn_dim and n == cfg.d_model and n != k:
            return "ffn2"
        return "out_proj" if n == k == cfg.d_model and cfg.ffn_dim != cfg.d_model else "ffn1"
    return "ffn1"


def traffic_for(label: str):
    """HBM bytes per launch of `label` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    measurement (techjam2026_amd/results/traffic_gfx950.json), or None."""
    path = os.path.join(ROOT, "techjam2026_amd", "results", "traffic_gfx950.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None
    rec = table.get("kernels", {}).get(label)
    return None if rec is None else rec.get("hbm_bytes_per_launch")


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(batch data-parallel sharding is designed, not built). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from techjam2026_amd import roofline

    os.environ.setdefault("KF950_STRICT", "1")
    case, cfg, model, x, m, x_cpu, m_cpu, params_cpu = build(args.config)
    lengths = m_cpu.sum(1).tolist()

    # ---- warm-up (first call selects the plan, prepares weights, captures the graph),
    # then exactly K timed steps
    median_ms, wall_ms, out = time_forward(model, x, m, args.steps, args.warmup)
    plan = model._plan
    from techjam2026_amd.optimized import STAGES
    stage_precision = {s: plan.stage_precision(s, torch.float32) for s in STAGES}
    control_ms = (control_median(model, x, m, args.steps, args.warmup)
                  if plan.overrides else median_ms)

    # ---- instrumented pass: per-kernel HIP-event timing of K eager forwards
    per_kernel = instrumented(model._impl, x, m, args.steps, args.label_log)
    attn, lnd = attention_and_ln(per_kernel, lengths, cfg, roofline.kernel_precision(
        plan.stage_precision("attn", torch.float32), True))
    dominant = max(per_kernel, key=lambda k: per_kernel[k]["total_ms"])
    dk = per_kernel[dominant]
    precision = roofline.kernel_precision(
        plan.stage_precision(stage_of(dominant, cfg), torch.float32), dominant.startswith("flash"))
    traffic = traffic_for(dominant)
    if dk["flops"]:
        peak = roofline.mfma_peak_tflops(precision)
        roof = {"bound": "mfma", "kernel": dominant, "achieved": round(dk["tflops"], 2),
                "peak": peak, "unit": "TFLOP/s", "frac": round(dk["tflops"] / peak, 4),
                "traffic": traffic, "precision": precision,
                "mfma_issued_frac": round(dk["tflops"] * roofline.SPLIT_FACTOR.get(precision, 1) / peak, 4),
                "vs_fp32_mfma_peak": round(dk["tflops"] / roofline.PEAK_TFLOPS["float32"], 3),
                "mean_launch_ms": round(dk["mean_ms"], 5),
                        "net_of_pair_overhead_ms": round(dk["net_ms"], 5),
                "event_bracket_ms": round(dk["bracket_ms"], 5), "launches": dk["launches"],
                "flops_per_launch": dk["flops"], "bytes_per_launch": dk["bytes"]}
    else:
        roof = {"bound": "hbm", "kernel": dominant, "achieved": round(dk["gbs"], 1),
                "peak": roofline.HBM_GBS, "unit": "GB/s", "frac": round(dk["gbs"] / roofline.HBM_GBS, 4),
                "traffic": traffic, "mean_launch_ms": round(dk["mean_ms"], 5),
                "net_of_pair_overhead_ms": round(dk["net_ms"], 5),
                "event_bracket_ms": round(dk["bracket_ms"], 5), "launches": dk["launches"],
                "bytes_per_launch": dk["bytes"]}
    kernels_out = {k: {"launches_per_step": v["launches"] // args.steps,
                       "mean_ms": round(v["mean_ms"], 5),
                       "tflops": None if v["tflops"] is None else round(v["tflops"], 2),
                       "gbs": None if v["gbs"] is None else round(v["gbs"], 1)}
                   for k, v in sorted(per_kernel.items(), key=lambda kv: -kv[1]["total_ms"])}

    # ---- CPU baseline (the oracle on the host's cores, bounded sample) + parity of this
    # very output against the oracle
    cpu = None
    envelope = None
    if not args.no_cpu_baseline:
        print(f"[bench] oracle check and CPU baseline {case.name}", file=sys.stderr, flush=True)
        envelope = envelope_vs_oracle(cfg, params_cpu, x_cpu, m_cpu, out)
        cpu = cpu_baseline_for(case.name, cfg, params_cpu, x_cpu, m_cpu)
        cpu["gpu_speedup"] = round(cpu["value"] / median_ms, 1)

    tokens = cfg.batch_size * cfg.seq_len
    line = {
        "metric": METRIC, "value": round(median_ms, 4), "unit": "ms", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,1) inputs, Xavier-uniform weights, causal + key padding)",
        "config": {"workload": f"{case.name}: {case.label()}", "plan": plan.name,
                   "precision": precision, "stage_precision": stage_precision},
        "control_f16x3_ms": round(control_ms, 4),
        "tokens_per_s": round(tokens * 1000.0 / median_ms, 1),
        "attn": attn,
        "layernorm": lnd,
        "envelope_vs_oracle": None if envelope is None else round(envelope, 5),
        "roofline": roof,
        "cpu_baseline": cpu,
        "kernels": kernels_out,
    }

    # ---- the metric's other shapes (median forward of every BASELINE config, with their
    # attention and LayerNorm rates) and the attention target check at hd 128
    if not args.no_per_config:
        del model, x, m, out
        torch.cuda.empty_cache()
        per = {case.name: {"workload": case.label(), "median_ms": round(median_ms, 4),
                           "steps": args.steps, "warmup": args.warmup,
                           "tokens_per_s": line["tokens_per_s"],
                           "plan": plan.name, "attn": attn, "layernorm": lnd,
                           "roofline_floor": floor_of(cfg, lengths, plan, median_ms),
                           "cpu_baseline": cpu}}
        for name in ("C1", "C2", "C3", "C4", "C5"):
            if name == case.name:
                continue
            # the long config's forward is ~60 ms: fewer steps keep the run within minutes
            steps, warm = ((args.per_config_steps, args.per_config_warmup) if name != "C5"
                           else (max(10, args.per_config_steps // 5), 3))
            print(f"[bench] per-config {name}", file=sys.stderr, flush=True)
            per[name] = per_config_line(name, steps, warm, cpu=not args.no_cpu_baseline)
        line["per_config"] = {k: per[k] for k in sorted(per)}
        print("[bench] attention hd128 check", file=sys.stderr, flush=True)
        line["attn_hd128"] = attention_microbench()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
