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
from typing import Iterable, Optional

PEAK_TFLOPS = {"float16": 2500.0, "bfloat16": 2500.0, "float32": 157.3,
               "fp8": 5000.0, "int8": 5000.0, "float64": 78.6}
HBM_GBS = 8000.0
SPLIT_FACTOR = {"f16x3": 3, "bf16x3": 3}


def useful_peak_tflops(precision: str) -> float:
    if precision in SPLIT_FACTOR:
        return PEAK_TFLOPS["float16"] / SPLIT_FACTOR[precision]
    return PEAK_TFLOPS[precision]


def mfma_peak_tflops(precision: str) -> float:
    """Dense peak of the MFMA pipe the precision runs on (fp16/bf16 for split modes)."""
    if precision in ("f16x3", "float16"):
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


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser(description="roofline helpers")
    ap.add_argument("--copy-mib", type=int, default=1024,
                    help="run the counter-calibration copy of this many MiB")
    ap.add_argument("--repeats", type=int, default=5)
    a = ap.parse_args()
    copy_calibration(a.copy_mib, a.repeats)
