"""Roofline placement on MI355X (`kernelforge/roofline.py:96-164`).

Peaks are AMD's published dense figures for MI355X: fp16/bf16 MFMA 2.5 PFLOP/s,
fp32 MFMA 157.3 TFLOP/s, HBM3E 8 TB/s. The split modes (f16x3 / bf16x3) issue three
16-bit MFMAs per useful product, so their ceiling for *useful* flops is a third of the
16-bit peak; `useful_peak_tflops` states it.

Work formulas (reference conventions):
* GEMM FLOPs per layer = 2M*d*3d + 2M*d*d + 2M*d*F + 2M*F*d  (M = B*S).
* attention FLOPs = 4*B*H*S*S*Dh, halved when causal (the reference's mask-agnostic
  count, `roofline.py:112-114`); `attention_flops_padded` counts only the (query, key)
  pairs a padding-aware kernel must visit: 4*H*Dh*sum_b L_b(L_b+1)/2 (causal).
* LayerNorm bytes per call = M*d*(e_x + e_y + e_s + e_h) + M*e_keep + 2*d*e_w.
"""
from __future__ import annotations

import dataclasses
import json
import os
from typing import Iterable, Optional

PEAK_TFLOPS = {"float16": 2500.0, "bfloat16": 2500.0, "float32": 157.3,
               "fp8": 5000.0, "int8": 5000.0, "float64": 78.6}
HBM_GBS = 8000.0
# MFMA passes per product: f16x3p runs q.k in 3 passes and P.V in 2; f16x2 runs 2
SPLIT_FACTOR = {"f16x3": 3, "bf16x3": 3, "f16x3p": 2.5, "f16x2": 2}


def kernel_precision(stage_precision: str, attention: bool) -> str:
    """The precision one kernel of a stage runs: an attention stage's precision names its
    QKV GEMM and its attention kernel ("f16x2p" is an f16x2 GEMM and f16x3p attention,
    "f16x3p" an f16x3 GEMM, "f16x3s" an f16x3 GEMM and single-pass fp16 attention)."""
    if attention:
        return {"f16x2": "f16x3", "f16x2p": "f16x3p", "f16x3s": "float16"}.get(
            stage_precision, stage_precision)
    return {"f16x3p": "f16x3", "f16x2p": "f16x2", "f16x3s": "f16x3"}.get(
        stage_precision, stage_precision)


def useful_peak_tflops(precision: str) -> float:
    if precision in SPLIT_FACTOR:
        return PEAK_TFLOPS["float16"] / SPLIT_FACTOR[precision]
    return PEAK_TFLOPS[precision]


def mfma_peak_tflops(precision: str) -> float:
    """Dense peak of the MFMA pipe the precision runs on (fp16/bf16 for split modes)."""
    if precision in ("f16x3", "f16x3p", "f16x2", "float16"):
        return PEAK_TFLOPS["float16"]
    if precision in ("bf16x3", "bfloat16"):
        return PEAK_TFLOPS["bfloat16"]
    return PEAK_TFLOPS[precision]


@dataclasses.dataclass
class Roofline:
    flops: int
    bytes_moved: int
    seconds: float
    peak_tflops: float
    peak_bandwidth_gbs: float = HBM_GBS

    @property
    def achieved_tflops(self) -> float:
        return self.flops / self.seconds / 1e12

    @property
    def achieved_bandwidth_gbs(self) -> float:
        return self.bytes_moved / self.seconds / 1e9

    @property
    def arithmetic_intensity(self) -> float:
        return self.flops / max(self.bytes_moved, 1)

    @property
    def ridge_point(self) -> float:
        return self.peak_tflops * 1e12 / (self.peak_bandwidth_gbs * 1e9)

    @property
    def compute_bound(self) -> bool:
        return self.arithmetic_intensity > self.ridge_point

    @property
    def floor_seconds(self) -> float:
        return max(self.flops / (self.peak_tflops * 1e12),
                   self.bytes_moved / (self.peak_bandwidth_gbs * 1e9))

    @property
    def utilization(self) -> float:
        """Fraction of the binding ceiling reached (floor time / measured time)."""
        return self.floor_seconds / self.seconds


def gemm_flops(batch: int, seq: int, d: int, ffn: int, layers: int) -> int:
    M = batch * seq
    return layers * (2 * M * d * 3 * d + 2 * M * d * d + 2 * M * d * ffn + 2 * M * ffn * d)


def attention_flops(batch: int, seq: int, d: int, heads: int, layers: int,
                    causal: bool) -> int:
    f = 4 * batch * heads * seq * seq * (d // heads)
    return layers * (f // 2 if causal else f)


def attention_flops_padded(lengths: Iterable[int], seq: int, d: int, heads: int,
                           layers: int, causal: bool) -> int:
    """Useful attention FLOPs given per-sequence valid lengths (prefix masks)."""
    dh = d // heads
    pairs = 0
    for n in lengths:
        n = int(n)
        pairs += n * (n + 1) // 2 if causal else n * n
    return layers * 4 * heads * dh * pairs


def stack_flops(batch, seq, d_model, heads, ffn, layers, causal=False) -> int:
    return gemm_flops(batch, seq, d_model, ffn, layers) + attention_flops(
        batch, seq, d_model, heads, layers, causal)


def ln_bytes(M: int, d: int, has_y: bool = True, write_s: bool = True,
             e_x: int = 4, e_h: int = 4, e_keep: int = 1) -> int:
    return M * d * (e_x + (e_x if has_y else 0) + (4 if write_s else 0) + e_h) + M * e_keep + 2 * d * 4


def stack_floor_ms(cfg, lengths, stage_precision=None) -> dict:
    """Roofline floor of one forward: sum over kernels of max(flops / peak, bytes / HBM)
    with GEMM and (padding-aware) attention FLOPs on the MFMA and the LayerNorms' bytes
    (fp32 residual, all flags: 16 B per element) at 8 TB/s.

    `fp16_peak`: every product at the dense fp16 peak (2.5 PF/s, the convention of the
    per-config floor table). `plan`: each stage at the useful peak of the precision it runs
    (f16x3 2.5/3, f16x3p attention 2.5/2.5, f16x2 2.5/2, fp16 2.5 PF/s) -- the floor
    of this plan's arithmetic. GEMMs are MFMA-bound at these sizes, so their bytes do not
    enter."""
    B, S, d, H, F, L = (cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads,
                        cfg.ffn_dim, cfg.num_layers)
    M = B * S
    stages = {"attn": 2 * M * d * 3 * d, "out_proj": 2 * M * d * d, "ffn1": 2 * M * d * F,
              "ffn2": 2 * M * F * d}
    attn = attention_flops_padded(lengths, S, d, H, 1, cfg.causal)
    ln_s = (2 * L + 1) * (16 * M * d + 4 * M + 8 * d) / (HBM_GBS * 1e9)
    peak16 = PEAK_TFLOPS["float16"] * 1e12
    fp16 = L * (sum(stages.values()) + attn) / peak16 + ln_s
    out = {"floor_ms_fp16_peak": round(fp16 * 1e3, 4)}
    if stage_precision:
        t = 0.0
        for st, fl in stages.items():
            prec = kernel_precision(stage_precision[st], False)
            t += fl / (useful_peak_tflops(prec) * 1e12)
        prec = kernel_precision(stage_precision["attn"], True)
        t += attn / (useful_peak_tflops(prec) * 1e12)
        out["floor_ms_plan"] = round((L * t + ln_s) * 1e3, 4)
    return out


def stack_bytes(batch, seq, d_model, heads, ffn, layers, elem_size=4) -> int:
    """Lower bound on HBM traffic of a fused forward (`roofline.py:119-134`)."""
    weights = layers * (4 * d_model * d_model + 2 * d_model * ffn) * elem_size
    acts = layers * batch * seq * (4 * d_model + 2 * ffn) * elem_size
    return weights + acts


def analyse(case, millis: float, precision: str = "f16x3",
            bandwidth_gbs: float = HBM_GBS) -> Optional[Roofline]:
    """Stack roofline for one measured case (`millis` in milliseconds)."""
    return Roofline(
        flops=stack_flops(case.batch_size, case.seq_len, case.d_model, case.num_heads,
                          case.ffn_dim, case.num_layers, case.causal),
        bytes_moved=stack_bytes(case.batch_size, case.seq_len, case.d_model,
                                case.num_heads, case.ffn_dim, case.num_layers, 4),
        seconds=millis / 1000.0, peak_tflops=useful_peak_tflops(precision),
        peak_bandwidth_gbs=bandwidth_gbs)


def copy_calibration(mbytes: int = 1024, repeats: int = 5) -> None:
    """A plain device copy of `mbytes` MiB (read + write), repeated: the reference kernel
    whose rocprofv3 FETCH_SIZE / WRITE_SIZE readings calibrate the counters (the known
    answer is mbytes MiB fetched and mbytes MiB written per launch)."""
    import torch
    n = mbytes * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(repeats):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[roofline] copied {mbytes} MiB x {repeats}", flush=True)


# kernel-name fragment each wrapper label's dispatches must carry
_LABEL_KERNEL = {"gemm": "gemm", "gemm_qkv": "gemm", "flash": "kf::flash_", "add_mask_ln": "ln_rows",
                 "mask_prep": "mask_prep", "split": "split"}


def _counter_rows(directory: str, counter: str):
    """(kernel name, value) per dispatch of `counter`, in dispatch order, from a rocprofv3
    `--pmc <counter> --output-format csv` run."""
    import csv
    import glob
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {directory}")
    acc = {}
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] != counter:
                    continue
                did = int(r["Dispatch_Id"])
                name, v = r["Kernel_Name"], float(r["Counter_Value"])
                acc[did] = (name, acc.get(did, (name, 0.0))[1] + v)
    return [acc[k] for k in sorted(acc)]


def traffic_table(bench_fetch: str, bench_write: str, copy_fetch: str, copy_write: str,
                  labels_json: str, copy_mib: int = 1024) -> dict:
    """HBM bytes per launch per kernel label: FETCH_SIZE and WRITE_SIZE (KiB per dispatch)
    of the instrumented bench pass, each scaled by what the counter reads for the
    `copy_calibration` kernel (known answer: `copy_mib` MiB read and written).

    The kf dispatches of the instrumented pass are the last ones of the bench run; they are
    matched, in order, to the pass's [label, dispatches] log (bench.py --label-log), and
    each label's kernel name is checked against the dispatch it is matched to.
    """
    with open(labels_json, encoding="utf-8") as f:
        log = json.load(f)["labels"]
    expanded = [(lab, nbytes / n) for lab, n, nbytes in log for _ in range(n)]

    def scale_of(directory, counter):
        return copy_mib * 1024.0 / max(v for _, v in _counter_rows(directory, counter))

    out = {"calibration": {"copy_mib": copy_mib}, "kernels": {}}
    for counter, key, cdir, bdir in (("FETCH_SIZE", "fetch", copy_fetch, bench_fetch),
                                     ("WRITE_SIZE", "write", copy_write, bench_write)):
        sc = scale_of(cdir, counter)
        out["calibration"][f"{key}_scale"] = round(sc, 4)
        rows = [r for r in _counter_rows(bdir, counter) if "kf::" in r[0] or "_ZN2kf" in r[0]]
        if len(rows) < len(expanded):
            raise ValueError(f"{counter}: {len(rows)} kf dispatches, {len(expanded)} labelled")
        rows = rows[len(rows) - len(expanded):]
        for (label, nbytes), (kname, kib) in zip(expanded, rows):
            frag = _LABEL_KERNEL[label.split("[")[0]]
            if frag not in kname:
                raise ValueError(f"dispatch {kname!r} does not belong to label {label!r}")
            k = out["kernels"].setdefault(label, {"alg": []})
            k.setdefault(f"{key}_kib", []).append(kib)
            if key == "fetch":
                k["alg"].append(nbytes)
    for label, k in out["kernels"].items():
        alg = k.pop("alg")     # mean over calls (e.g. the first LayerNorm has no residual input)
        k["algorithmic_bytes_per_launch"] = (
            int(round(sum(alg) / len(alg) * next(n for lab, n, _ in log if lab == label)))
            if any(alg) else None)
        for key in ("fetch", "write"):
            v = k.pop(f"{key}_kib")
            k[f"{key}_kib_per_dispatch"] = round(sum(v) / len(v), 1)
            k["dispatches"] = len(v)
        k["hbm_fetch_bytes"] = int(k["fetch_kib_per_dispatch"] * 1024 * out["calibration"]["fetch_scale"])
        k["hbm_write_bytes"] = int(k["write_kib_per_dispatch"] * 1024 * out["calibration"]["write_scale"])
        # a label covering two dispatches (flash: prefix + general launch) counts both
        per_call = next(n for lab, n, _ in log if lab == label)
        k["hbm_bytes_per_launch"] = per_call * (k["hbm_fetch_bytes"] + k["hbm_write_bytes"])
    return out


def counter_table(pmc_dir: str, labels_json: str, counters) -> dict:
    """Per label, each counter's value per launch (a launch's dispatches summed), averaged
    over the labelled calls, from a rocprofv3 `--pmc <counters>` run of bench.py; the last
    kf dispatches are matched to the instrumented pass's launch log as in `traffic_table`."""
    with open(labels_json, encoding="utf-8") as f:
        log = json.load(f)["labels"]
    expanded = [(lab, i) for i, (lab, n, _b) in enumerate(log) for _ in range(n)]
    out: dict = {}
    for counter in counters:
        rows = [r for r in _counter_rows(pmc_dir, counter) if "kf::" in r[0] or "_ZN2kf" in r[0]]
        if len(rows) < len(expanded):
            raise ValueError(f"{counter}: {len(rows)} kf dispatches, {len(expanded)} labelled")
        rows = rows[len(rows) - len(expanded):]
        calls: dict = {}
        for (label, call), (kname, v) in zip(expanded, rows):
            if _LABEL_KERNEL[label.split("[")[0]] not in kname:
                raise ValueError(f"dispatch {kname!r} does not belong to label {label!r}")
            calls[(label, call)] = calls.get((label, call), 0.0) + v
        per: dict = {}
        for (label, _c), v in calls.items():
            per.setdefault(label, []).append(v)
        for label, vs in per.items():
            out.setdefault(label, {"calls": len(vs)})[counter] = sum(vs) / len(vs)
    return out


MFMA_COUNTERS = ("SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES",
                 "GRBM_GUI_ACTIVE")


def mfma_summary(table: dict, durations: dict, labels_json: str, commands,
                 workload: str) -> str:
    """Counter-measured MFMA work per kernel label: issued fp16-MFMA FLOPs (512 per
    SQ_INSTS_VALU_MFMA_MOPS_F16), their rate over the kernel-trace duration against the
    2.5 PF/s dense peak, the ratio of issued to algorithmic FLOPs (3 for an f16x3 GEMM,
    the known answer that pins the counter's unit), and MFMA-busy cycles per SIMD-cycle
    of the kernel: SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x 1024 SIMDs), the
    expression rocprofv3 lists for its MFMA-busy metric; the per-dispatch values here are
    summed over the eight XCDs, so GRBM_GUI_ACTIVE is divided by 8."""
    with open(labels_json, encoding="utf-8") as f:
        log = json.load(f)["labels"]
    lines = [f"# rocprofv3 MFMA counters per kernel: {workload}", "# commands:"]
    lines += [f"#   {c}" for c in commands]
    lines += ["# label | issued MFMA GFLOP/launch | algorithmic GFLOP | issued/alg | "
              "mean us (kernel trace) | issued TF/s | of 2.5 PF/s | MFMA-busy / SIMD-cycles"]
    alg = {}
    for lab, n, _b in log:
        alg.setdefault(lab, None)
    flops_of = _label_flops(log)
    for label in sorted(table, key=lambda k: -durations.get(k, {}).get("mean_us", 0.0)):
        r = table[label]
        mops = r.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0)
        issued = 512.0 * mops
        us = durations.get(label, {}).get("mean_us")
        busy, gui = r.get("SQ_VALU_MFMA_BUSY_CYCLES"), r.get("GRBM_GUI_ACTIVE")
        frac_busy = (busy / (gui * 256 * 4 / 8)) if busy and gui else None
        a = flops_of.get(label)
        lines.append(
            f"{label:28s} | {issued / 1e9:10.2f} | {a / 1e9 if a else float('nan'):10.2f} | "
            f"{issued / a if a else float('nan'):5.2f} | {us if us else float('nan'):10.2f} | "
            f"{issued / (us * 1e-6) / 1e12 if us else float('nan'):8.1f} | "
            f"{issued / (us * 1e-6) / 2.5e15 if us else float('nan'):6.3f} | "
            f"{frac_busy if frac_busy is not None else float('nan'):6.3f}")
    return "\n".join(lines) + "\n"


def counters_summary(table: dict, counters, commands, workload: str) -> str:
    """Per-label values per launch of SQ counters (summed over the launch's dispatches and
    the eight XCDs), with the ratios that read directly: instructions per MFMA
    instruction, and shares of wavefront cycles (SQ_WAVE_CYCLES) spent issuing VALU or
    waiting on an instruction dependency."""
    lines = [f"# rocprofv3 SQ counters per kernel launch: {workload}", "# commands:"]
    lines += [f"#   {c}" for c in commands]
    short = [c.replace("SQ_", "").lower() for c in counters]
    ratios = []
    if "SQ_INSTS_MFMA" in counters:
        ratios += [(f"{c.replace('SQ_INSTS_', '').lower()}/mfma", c, "SQ_INSTS_MFMA")
                   for c in counters if c.startswith("SQ_INSTS_") and c != "SQ_INSTS_MFMA"]
    if "SQ_WAVE_CYCLES" in counters:
        ratios += [(f"{c.replace('SQ_', '').lower()}/wave_cycles", c, "SQ_WAVE_CYCLES")
                   for c in ("SQ_ACTIVE_INST_VALU", "SQ_WAIT_INST_ANY", "SQ_WAIT_ANY")
                   if c in counters]
    lines.append("# label | " + " | ".join(short) + " | " + " | ".join(r[0] for r in ratios))
    for label in sorted(table):
        r = table[label]
        vals = " | ".join(f"{r.get(c, float('nan')):.4g}" for c in counters)
        rs = " | ".join(f"{r[n] / r[d]:.3f}" if r.get(d) else "nan" for _t, n, d in ratios)
        lines.append(f"{label:28s} | {vals} | {rs}")
    return "\n".join(lines) + "\n"


def _label_flops(log) -> dict:
    """Algorithmic FLOPs per launch of the GEMM labels, from their shape (2 M N K)."""
    import re as _re
    out = {}
    for lab, _n, _b in log:
        m = _re.match(r"gemm(?:_qkv)?\[(\d+)x(\d+)x(\d+)\]", lab)
        if m:
            M, N, K = (int(g) for g in m.groups())
            out[lab] = 2.0 * M * N * K
    return out


def trace_durations(trace_dir: str, labels_json: str) -> dict:
    """Mean kernel duration (us) per label from a rocprofv3 `--kernel-trace` run of bench.py:
    the run's last kf dispatches are its instrumented passes, attributed to labels in
    order as in `traffic_table` (a label's dispatches summed per call)."""
    import csv
    import glob
    files = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no kernel_trace.csv under {trace_dir}")
    with open(files[0], newline="") as fh:
        rows = sorted(((int(r["Dispatch_Id"]), r["Kernel_Name"],
                        (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
                       for r in csv.DictReader(fh)
                       if "kf::" in r["Kernel_Name"] or "_ZN2kf" in r["Kernel_Name"]))
    with open(labels_json, encoding="utf-8") as f:
        log = json.load(f)["labels"]
    expanded = [(lab, i) for i, (lab, n, _b) in enumerate(log) for _ in range(n)]
    per_pass = len(expanded)
    # whole passes from the end of the run (the trace may hold more passes than the log)
    n_pass = len(rows) // per_pass
    out: dict = {}
    names = None
    for p in range(1, n_pass + 1):
        tail = rows[len(rows) - p * per_pass:len(rows) - (p - 1) * per_pass]
        # every earlier pass must run exactly the last pass's kernels (a pass of another
        # plan, e.g. the control model, ends the walk)
        if names is None:
            names = [r[1] for r in tail]
        elif [r[1] for r in tail] != names:
            break
        calls: dict = {}
        for (label, call), (_, kname, us) in zip(expanded, tail):
            if _LABEL_KERNEL[label.split("[")[0]] not in kname:
                break
            calls[(label, call)] = calls.get((label, call), 0.0) + us
        else:
            for (label, _c), us in calls.items():
                out.setdefault(label, []).append(us)
            continue
        break
    return {k: {"mean_us": sum(v) / len(v), "calls": len(v)} for k, v in out.items()}


def traffic_summary(table: dict, commands) -> str:
    cal = table["calibration"]
    lines = ["# HBM traffic per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE), scaled by a "
             f"{cal['copy_mib']} MiB copy: FETCH_SIZE x{cal['fetch_scale']}, "
             f"WRITE_SIZE x{cal['write_scale']}", "# commands:"]
    lines += [f"#   {c}" for c in commands]
    lines.append("# kernel label | fetch KiB/dispatch | write KiB/dispatch | HBM bytes/launch "
                 "| algorithmic bytes/launch | ratio")
    for label, k in sorted(table["kernels"].items()):
        alg = k.get("algorithmic_bytes_per_launch")
        ratio = f"{k['hbm_bytes_per_launch'] / alg:5.2f}" if alg else "  n/a"
        lines.append(f"{label:28s} | {k['fetch_kib_per_dispatch']:10.1f} | "
                     f"{k['write_kib_per_dispatch']:10.1f} | {k['hbm_bytes_per_launch']:12d} | "
                     f"{int(alg) if alg else 'n/a':>12} | {ratio}")
    return "\n".join(lines) + "\n"


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser(description="roofline helpers")
    ap.add_argument("--copy-mib", type=int, default=1024,
                    help="run the counter-calibration copy of this many MiB")
    ap.add_argument("--repeats", type=int, default=5)
    ap.add_argument("--traffic", nargs=4, metavar=("BENCH_FETCH", "BENCH_WRITE", "COPY_FETCH",
                                                  "COPY_WRITE"), default=None,
                    help="build the traffic table from four rocprofv3 --pmc output folders")
    ap.add_argument("--labels", default=None, help="bench.py --label-log output")
    ap.add_argument("--out", default=None, help="traffic table JSON")
    ap.add_argument("--summary", default=None, help="text summary for profiles/")
    ap.add_argument("--workload", default="bench.py C2 forward")
    ap.add_argument("--bench-args", default="--no-per-config --no-cpu-baseline --steps 5 --warmup 2",
                    help="the bench.py flags of the profiled run (quoted in the summary's command)")
    ap.add_argument("--trace", default=None, help="rocprofv3 --kernel-trace output folder of "
                    "bench.py: per-label mean durations of its instrumented passes (needs --labels)")
    ap.add_argument("--counters", nargs="+", default=None, metavar="NAME",
                    help="with --pmc-dir: per-label values per launch of these SQ counters")
    ap.add_argument("--pmc-dir", default=None, help="rocprofv3 --pmc output folder of bench.py")
    ap.add_argument("--mfma", default=None, help="rocprofv3 --pmc output folder of bench.py "
                    "with the MFMA counters (needs --labels and --trace of a kernel-trace run)")
    a = ap.parse_args()
    if a.counters:
        tbl = counter_table(a.pmc_dir, a.labels, a.counters)
        cmds = ["cd /tmp && rocprofv3 --pmc " + " ".join(a.counters) + " --kernel-trace -d "
                "<out>/pmc -o run --output-format csv -- python3 <repo>/bench.py "
                f"{a.bench_args} --label-log <out>/labels_pmc.json",
                "python -m techjam2026_amd.roofline --counters " + " ".join(a.counters) +
                " --pmc-dir <out>/pmc --labels <out>/labels_pmc.json --summary <summary>"]
        text = counters_summary(tbl, a.counters, cmds, a.workload)
        if a.summary:
            with open(a.summary, "w", encoding="utf-8") as f:
                f.write(text)
        print(text)
    elif a.mfma:
        tbl = counter_table(a.mfma, a.labels, MFMA_COUNTERS)
        cmds = ["cd /tmp && rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) + " --kernel-trace -d "
                "<out>/mfma -o run --output-format csv -- python3 <repo>/bench.py "
                f"{a.bench_args} --label-log <out>/labels_mfma.json",
                "python -m techjam2026_amd.roofline --mfma <out>/mfma --labels "
                "<out>/labels_mfma.json --trace <kernel-trace folder of the same workload> "
                "--summary <summary>"]
        text = mfma_summary(tbl, trace_durations(a.trace, a.labels) if a.trace else {},
                            a.labels, cmds, a.workload)
        if a.summary:
            with open(a.summary, "w", encoding="utf-8") as f:
                f.write(text)
        print(text)
    elif a.trace:
        for label, r in sorted(trace_durations(a.trace, a.labels).items(),
                               key=lambda kv: -kv[1]["mean_us"]):
            print(f"{label:28s} {r['mean_us']:10.2f} us  ({r['calls']} calls)")
    elif a.traffic:
        t = traffic_table(*a.traffic, a.labels, a.copy_mib)
        cmds = ["cd /tmp && rocprofv3 --pmc FETCH_SIZE --kernel-trace -d <out>/tr_bench_FETCH_SIZE "
                "-o run --output-format csv -- python3 <repo>/bench.py "
                f"{a.bench_args} --label-log <out>/labels.json",
                "(the same with --pmc WRITE_SIZE)",
                "cd /tmp && rocprofv3 --pmc FETCH_SIZE --kernel-trace -d <out>/tr_copy_FETCH_SIZE "
                f"-o run --output-format csv -- python3 <repo>/techjam2026_amd/roofline.py "
                f"--copy-mib {a.copy_mib} --repeats 5", "(the same with --pmc WRITE_SIZE)",
                "python -m techjam2026_amd.roofline --traffic <out>/tr_bench_FETCH_SIZE "
                "<out>/tr_bench_WRITE_SIZE <out>/tr_copy_FETCH_SIZE <out>/tr_copy_WRITE_SIZE "
                "--labels <out>/labels.json --out <table> --summary <summary>"]
        t.update({"device": "MI355X (gfx950)", "workload": a.workload, "commands": cmds})
        text = traffic_summary(t, cmds)          # this run's kernels only
        if a.out:
            # labels name their shapes, so the tables of several workloads merge: each
            # kernel record keeps the workload and calibration it was measured with
            for k in t["kernels"].values():
                k["workload"] = a.workload
                k["calibration"] = dict(t["calibration"])
            if os.path.exists(a.out):
                with open(a.out, encoding="utf-8") as f:
                    old = json.load(f)
                merged = dict(old.get("kernels", {}))
                merged.update(t["kernels"])
                t = {**t, "kernels": merged}
            with open(a.out, "w", encoding="utf-8") as f:
                json.dump(t, f, indent=1)
        if a.summary:
            with open(a.summary, "w", encoding="utf-8") as f:
                f.write(text)
        print(text)
    else:
        copy_calibration(a.copy_mib, a.repeats)
