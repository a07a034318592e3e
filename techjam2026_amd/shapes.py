"""Shape cases and the spec grammar (`kernelforge/shapes.py:27-100, 195-260`).

    B8-S128-d512-H8-F2048-L6[-causal][-pad0.4][-scale64][-float16]   (or 'x' separators)

`L` defaults to 6. `CONFIGS` holds BASELINE.json's five configurations (C1..C5) with
the padding ratios their valid-length ranges imply.
"""
from __future__ import annotations

import dataclasses
import re
from typing import List

import torch

from .model import TransformerConfig


@dataclasses.dataclass(frozen=True)
class Case:
    name: str
    regime: str
    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int = 6
    causal: bool = False
    padding_ratio: float = 0.0
    input_scale: float = 1.0
    dtype: str = "float32"

    def to_config(self) -> TransformerConfig:
        return TransformerConfig(self.batch_size, self.seq_len, self.d_model, self.num_heads,
                                 self.ffn_dim, self.num_layers, self.causal)

    @property
    def torch_dtype(self) -> torch.dtype:
        return {"float32": torch.float32, "float16": torch.float16,
                "bfloat16": torch.bfloat16}[self.dtype]

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    @property
    def tokens(self) -> int:
        return self.batch_size * self.seq_len

    def label(self) -> str:
        bits = [f"B{self.batch_size}", f"S{self.seq_len}", f"d{self.d_model}",
                f"H{self.num_heads}", f"F{self.ffn_dim}", f"L{self.num_layers}"]
        if self.causal:
            bits.append("causal")
        if self.padding_ratio:
            bits.append(f"pad{self.padding_ratio:g}")
        if self.input_scale != 1.0:
            bits.append(f"scale{self.input_scale:g}")
        bits.append(self.dtype)
        return "-".join(bits)


_SPEC_RE = re.compile(
    r"^B(?P<batch>\d+)[-x]S(?P<seq>\d+)[-x]d(?P<d>\d+)[-x]H(?P<h>\d+)"
    r"[-x]F(?P<ffn>\d+)(?:[-x]L(?P<layers>\d+))?(?P<rest>.*)$", re.I)


def _regime(batch: int, seq: int, d: int, ffn: int) -> str:
    tokens = batch * seq
    if tokens <= 512:
        return "latency"
    if seq >= 1024:
        return "attention"
    if ffn >= 4 * d and tokens * ffn >= 8_000_000:
        return "bandwidth"
    return "gemm"


def parse_spec(spec: str) -> Case:
    text = spec.strip()
    m = _SPEC_RE.match(text)
    if not m:
        raise ValueError(f"cannot parse shape {spec!r}. Expected e.g. "
                         f"B8-S128-d512-H8-F2048-L6[-causal][-pad0.4][-scale64][-float16]")
    g = m.groupdict()
    rest = (g.get("rest") or "").lower()
    dtype = next((c for c in ("bfloat16", "float16", "float32") if c in rest), "float32")
    pm = re.search(r"pad([0-9.]+)", rest)
    sm = re.search(r"scale([0-9.]+)", rest)
    batch, seq = int(g["batch"]), int(g["seq"])
    d, heads, ffn = int(g["d"]), int(g["h"]), int(g["ffn"])
    layers = int(g["layers"] or 6)
    if d % heads:
        raise ValueError(f"{spec}: d_model {d} is not divisible by {heads} heads")
    return Case(name=text, regime=_regime(batch, seq, d, ffn), batch_size=batch, seq_len=seq,
                d_model=d, num_heads=heads, ffn_dim=ffn, num_layers=layers,
                causal="causal" in rest, padding_ratio=float(pm.group(1)) if pm else 0.0,
                input_scale=float(sm.group(1)) if sm else 1.0, dtype=dtype)


# BASELINE.json configs; padding ratio p gives min valid length round(S * (1 - p)).
CONFIGS: List[Case] = [
    Case("C1", "latency", 2, 128, 256, 4, 1024, 2, True, 0.5),
    Case("C2", "gemm", 16, 512, 512, 8, 2048, 6, True, 0.875),
    Case("C3", "attention", 64, 1024, 64, 8, 256, 6, True, 0.875),
    Case("C4", "attention", 8, 4096, 1024, 4, 4096, 2, True, 0.75),
    Case("C5", "attention", 4, 65536, 1024, 16, 1024, 2, True, 0.5),
]


def config(name: str) -> Case:
    for c in CONFIGS:
        if c.name == name.upper():
            return c
    return parse_spec(name)


def resolve(names: List[str]) -> List[Case]:
    return [config(n) for n in names if n.strip()]
