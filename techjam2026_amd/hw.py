"""Hardware probe for the dispatch table (`kernelforge/hw.py:21-219`).

The dispatch key needs an architecture string and the LDS budget. On ROCm the
architecture is `gcnArchName` ("gfx950:sramecc+:xnack-" -> "gfx950"), not a CUDA-style
`sm_NM` built from major/minor (which would misparse gfx950 as major 95). The LDS
budget is 160 KB per CU on gfx950; torch reports the per-block shared-memory limit,
which is used when present. The nvidia-smi helpers of the reference have no place here.
"""
from __future__ import annotations

import dataclasses
import re

import torch

GFX950_LDS_KB = 160.0


@dataclasses.dataclass(frozen=True)
class GPUSpec:
    name: str
    arch: str                      # "gfx950"
    cu_count: int
    total_mem_gb: float
    shared_mem_per_block_kb: float
    warp_size: int
    l2_cache_mb: float
    measured_bw_gbs: float = 0.0

    @property
    def sm_count(self) -> int:     # the reference's field name
        return self.cu_count

    def summary(self) -> str:
        return (f"{self.name} [{self.arch}] {self.cu_count} CUs | {self.total_mem_gb:.1f} GB | "
                f"LDS/block {self.shared_mem_per_block_kb:.0f} KB | wave{self.warp_size}")


def arch_of(gcn_arch_name: str) -> str:
    """'gfx950:sramecc+:xnack-' -> 'gfx950'."""
    return (gcn_arch_name or "").split(":")[0].strip()


def measure_bandwidth(device: int = 0, mb: int = 1024, iters: int = 20) -> float:
    """Achieved device-to-device copy bandwidth in GB/s (read + write counted)."""
    n = mb * 2**20 // 4
    src = torch.empty(n, dtype=torch.float32, device=f"cuda:{device}")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize(device)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize(device)
    sec = a.elapsed_time(b) / 1e3
    out = 2 * src.numel() * 4 * iters / sec / 1e9
    del src, dst
    return out


def probe(device: int = 0, measure: bool = False) -> GPUSpec:
    if not torch.cuda.is_available():
        raise RuntimeError("no GPU available")
    p = torch.cuda.get_device_properties(device)
    arch = arch_of(getattr(p, "gcnArchName", "")) or f"sm_{p.major}{p.minor}"
    smem = getattr(p, "shared_memory_per_block_optin", 0) or getattr(p, "shared_memory_per_block", 0)
    smem_kb = smem / 1024 if smem else (GFX950_LDS_KB if arch == "gfx950" else 64.0)
    if arch == "gfx950":
        smem_kb = max(smem_kb, GFX950_LDS_KB)
    return GPUSpec(
        name=p.name, arch=arch, cu_count=p.multi_processor_count,
        total_mem_gb=p.total_memory / 2**30, shared_mem_per_block_kb=smem_kb,
        warp_size=getattr(p, "warp_size", 64), l2_cache_mb=getattr(p, "L2_cache_size", 0) / 2**20,
        measured_bw_gbs=measure_bandwidth(device) if measure else 0.0)


# what the marketing name reads as when the driver's name table is missing on a host
# (torch then reports "AMD Radeon Graphics" for every card)
_GENERIC_NAMES = ("", "graphics")


def hardware_slug(spec) -> str:
    """Identifier from what every host reports the same way: CUs, memory, arch."""
    return f"{getattr(spec, 'cu_count', 0)}cu-{spec.total_mem_gb:.0f}gb_{spec.arch}"


def device_slug(spec) -> str:
    """Filename-safe identifier of one card (`kernelforge/hw.py:194-219`): vendor and
    marketing junk removed, separators collapsed, memory size and arch appended. Where
    the host reports only a generic name, the hardware slug (CUs, memory, arch) is used,
    so one card's table is found whether or not that host can name it."""
    name = spec.name.lower()
    for junk in ("amd", "instinct", "radeon", "nvidia", "geforce", "rtx", "gpu", "pcie",
                 "sxm", "oam", "(r)", "(tm)"):
        name = name.replace(junk, " ")
    slug = "-".join(part for part in re.split(r"[\s/]+", name) if part)
    slug = re.sub(r"-{2,}", "-", slug).strip("-")
    if slug in _GENERIC_NAMES:
        return hardware_slug(spec)
    mem = f"{spec.total_mem_gb:.0f}gb"
    if mem not in slug:
        slug = f"{slug}-{mem}" if slug else mem
    return f"{slug}_{spec.arch}".strip("-")
