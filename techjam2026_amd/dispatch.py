"""The frozen dispatch table (`kernelforge/dispatch.py`), with a gfx950 table.

Key: (arch, I/O dtype, shape signature "B{b}-S{s}-d{d}-H{h}-F{f}-L{l}[-causal]"),
identical to the reference's (`dispatch.py:40-44`). Tables live in
`techjam2026_amd/results/dispatch_<arch>[__<device-slug>].json` with the reference's
entry schema (`Entry.to_json`, `dispatch.py:92-109`); a device table overlays the
architecture table (`:209-244`). Lookup order: exact -> nearest (same arch and dtype:
conservative default) -> default (`:254-288`).

gfx950 default rules (`default_plan`):
* float32 I/O: every stage "f16x3" (split fp32 on the fp16 MFMA) with hipGraph capture,
  attention as "f16x3p" (probabilities enter P.V as one fp16 plane). gfx950 has no
  TF32-like MFMA, so the reference's argument for single-pass fp16 (the reference itself
  computing at 10 mantissa bits) does not hold: against a true-fp32 reference, single-pass
  fp16 used 0.56-1.41 of the tolerance on C1-C4 while f16x3 used 0.001-0.004 and f16x3p
  added at most 0.003 to it (the measured per-stage budget and sweep). Nothing else is
  narrowed, so the conservative (nearest) plan is the same plan.
* float16 / bfloat16 I/O: the reference forward replayed from a hipGraph
  ("safe(exact)+graph", `dispatch.py:300-364`): at those dtypes the gate compares against
  the reference's own narrow arithmetic, so only a bit-exact plan is admissible, and
  graph capture removes the per-op launches without touching arithmetic. Where the
  reference's score tensor cannot be formed (> 8 GiB), the native stack runs with fp32
  internals on the widened input ("stream(flash)+f16x3", `dispatch.py:325-353`).
"""
from __future__ import annotations

import dataclasses
import json
import os
from typing import Dict, List, Optional, Tuple

import torch

from .optimized import Plan

TABLE_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "results")

SAFE = Plan(name="safe", compute_dtype="f16x3", residual_dtype="float32")
BASELINE = Plan(name="baseline", compute_dtype="auto", residual_dtype="auto",
                fuse_qkv=False, attention="baseline", fused_norm=False)


def shape_signature(case_or_cfg, dtype: Optional[torch.dtype] = None) -> str:
    c = case_or_cfg
    causal = getattr(c, "causal", False)
    return (f"B{c.batch_size}-S{c.seq_len}-d{c.d_model}-H{c.num_heads}"
            f"-F{c.ffn_dim}-L{c.num_layers}{'-causal' if causal else ''}")


_NARROW_RISK = {"float16": 8, "bfloat16": 12, "bf16x3": 1, "f16x3": 0, "f16x3p": 1, "f16x2": 3,
                "f16x2p": 4, "float32": 0, "auto": 0}


def _aggressiveness(plan: Plan) -> int:
    """Numerical risk of a plan, lower is safer (`dispatch.py:55-77`).

    Single-pass 16-bit stages carry the risk (bf16 more than fp16); the split modes are
    fp32-level. Graph capture changes no arithmetic and carries none.
    """
    score = _NARROW_RISK.get(plan.compute_dtype, 8)
    score += sum(_NARROW_RISK.get(p, 8) + 2 for _, p in plan.overrides)
    if plan.residual_dtype in ("float16", "bfloat16"):
        score += 6
    if plan.attention != "baseline":
        score += 1
    return score


@dataclasses.dataclass
class Entry:
    signature: str
    dtype: str
    arch: str
    regime: str
    plan: Plan
    utilization: float
    speedup: float
    speedup_vs_compile: float
    case: str = ""

    def to_json(self) -> dict:
        d = dataclasses.asdict(self)
        d["plan"] = dataclasses.asdict(self.plan)
        d["plan"]["overrides"] = [list(o) for o in self.plan.overrides]
        if self.plan.flash_block:
            d["plan"]["flash_block"] = list(self.plan.flash_block)
        return d

    @staticmethod
    def from_json(d: dict) -> "Entry":
        p = dict(d["plan"])
        p["overrides"] = tuple(tuple(o) for o in p.get("overrides", []))
        fb = p.get("flash_block")
        p["flash_block"] = tuple(fb) if fb else None
        known = {f.name for f in dataclasses.fields(Plan)}
        p = {k: v for k, v in p.items() if k in known}   # older/newer schemas load
        return Entry(d["signature"], d["dtype"], d["arch"], d["regime"], Plan(**p),
                     d["utilization"], d["speedup"], d.get("speedup_vs_compile", float("nan")),
                     d.get("case", ""))


class DispatchTable:
    def __init__(self, entries: Optional[List[Entry]] = None, owned: Optional[set] = None):
        self.entries: List[Entry] = entries or []
        self._owned: set = (set(owned) if owned is not None else
                            {(e.arch, e.dtype, e.signature) for e in self.entries})
        self._index: Dict[Tuple[str, str, str], Entry] = {}
        self._reindex()

    def _reindex(self) -> None:
        self._index = {(e.arch, e.dtype, e.signature): e for e in self.entries}

    def add(self, entry: Entry) -> None:
        """Insert, resolving collisions conservatively (`dispatch.py:133-182`): a
        re-measurement of the same case supersedes; across data variants the less
        aggressive plan wins, ties go to the faster one, and the tighter (larger)
        envelope is remembered."""
        key = (entry.arch, entry.dtype, entry.signature)
        self._owned.add(key)
        existing = self._index.get(key)
        if existing is not None and existing.case == entry.case:
            self.entries = [e for e in self.entries if (e.arch, e.dtype, e.signature) != key]
            self.entries.append(entry)
            self._reindex()
            return
        old_risk = _aggressiveness(existing.plan) if existing else 0
        new_risk = _aggressiveness(entry.plan)
        if existing is not None and (old_risk < new_risk or (
                old_risk == new_risk and existing.speedup >= entry.speedup)):
            existing.utilization = max(existing.utilization, entry.utilization)
            return
        self.entries = [e for e in self.entries if (e.arch, e.dtype, e.signature) != key]
        if existing is not None:
            entry.utilization = max(existing.utilization, entry.utilization)
        self.entries.append(entry)
        self._reindex()

    @staticmethod
    def path_for(arch: str, device: Optional[str] = None) -> str:
        if device:
            return os.path.join(TABLE_DIR, f"dispatch_{arch}__{device}.json")
        return os.path.join(TABLE_DIR, f"dispatch_{arch}.json")

    def save(self, arch: str, device: Optional[str] = None) -> str:
        os.makedirs(TABLE_DIR, exist_ok=True)
        path = self.path_for(arch, device)
        entries = self.entries
        if device:
            entries = [e for e in entries if (e.arch, e.dtype, e.signature) in self._owned]
        blob = {"arch": arch, "entries": [e.to_json() for e in entries]}
        if device:
            blob["device"] = device
        with open(path, "w", encoding="utf-8") as f:
            json.dump(blob, f, indent=2)
        return path

    @staticmethod
    def load(arch: str, device: Optional[str] = None) -> "DispatchTable":
        """Architecture table with this card's entries laid over it."""
        merged, owned = {}, set()
        for tier in (None, device):
            path = DispatchTable.path_for(arch, tier)
            if not os.path.exists(path):
                continue
            with open(path, encoding="utf-8") as f:
                blob = json.load(f)
            for e in (Entry.from_json(x) for x in blob.get("entries", [])):
                k = (e.arch, e.dtype, e.signature)
                merged[k] = e
                if tier is not None:
                    owned.add(k)
        return DispatchTable(list(merged.values()), owned=owned)

    @staticmethod
    def load_for(spec) -> "DispatchTable":
        """The card's table by its name slug, else by its hardware slug (a host that can
        name the card and one that cannot then read the same measured table)."""
        from .hw import device_slug, hardware_slug
        for slug in (device_slug(spec), hardware_slug(spec)):
            if os.path.exists(DispatchTable.path_for(spec.arch, slug)):
                return DispatchTable.load(spec.arch, slug)
        return DispatchTable.load(spec.arch, device_slug(spec))

    def lookup(self, arch: str, dtype: torch.dtype, cfg, smem_kb: float = 160.0,
               ) -> Tuple[Plan, str]:
        dt = str(dtype).replace("torch.", "")
        sig = shape_signature(cfg)
        must_stream = score_matrix_bytes(cfg) > 8 * 2**30
        hit = self._index.get((arch, dt, sig))
        if hit is not None:
            plan = dataclasses.replace(hit.plan, smem_kb=smem_kb)
            if must_stream and plan.attention == "baseline":
                return default_plan(dtype, smem_kb, conservative=True, arch=arch,
                                    must_stream=True), "exact"
            return plan, "exact"
        if any(e.arch == arch and e.dtype == dt for e in self.entries):
            return default_plan(dtype, smem_kb, conservative=True, arch=arch,
                                must_stream=must_stream), "nearest"
        return default_plan(dtype, smem_kb, arch=arch, must_stream=must_stream), "default"


def score_matrix_bytes(cfg) -> int:
    """Bytes of the reference's fp32 [B, H, S, S] score tensor (`dispatch.py:291-298`)."""
    return cfg.batch_size * cfg.num_heads * cfg.seq_len * cfg.seq_len * 4


def default_plan(dtype: torch.dtype, smem_kb: float = 160.0, conservative: bool = False,
                 arch: Optional[str] = None, must_stream: bool = False) -> Plan:
    """The rule when the table has nothing to say (see the module docstring)."""
    if dtype in (torch.float16, torch.bfloat16):
        if must_stream:
            # the exact plan would form the [B, H, S, S] score tensor: run the native
            # stack with fp32 internals instead (input widened, output rounded once)
            return Plan(name="stream(flash)+f16x3", compute_dtype="f16x3",
                        residual_dtype="float32", attention="flash", smem_kb=smem_kb)
        return dataclasses.replace(BASELINE, smem_kb=smem_kb, cuda_graph=True,
                                   name="safe(exact)+graph")
    return Plan(name="f16x3p+graph", compute_dtype="f16x3", residual_dtype="float32",
                attention="flash", cuda_graph=True, smem_kb=smem_kb,
                overrides=(("attn", "f16x3p"),))


def summarize(table: DispatchTable) -> str:
    if not table.entries:
        return "(empty dispatch table)"
    lines = [f"{'signature':<40} {'dtype':<9} {'plan':<22} {'env':>6} {'vs base':>8}", "-" * 90]
    for e in sorted(table.entries, key=lambda e: (e.dtype, e.signature)):
        lines.append(f"{e.signature:<40} {e.dtype:<9} {e.plan.name:<22} "
                     f"{e.utilization:6.3f} {e.speedup:7.3f}x")
    return "\n".join(lines)
