"""Build libkf950.so (the gfx950 kernels and their C ABI) in-tree with hipcc.

    python -m techjam2026_amd.build            # compile every source, link the library

Each `csrc/*.hip` file is compiled to an object in `csrc/_build/` in parallel, then linked
into `techjam2026_amd/libkf950.so`, which the ctypes loader (`_lib.py`) opens. Packed
fp32 instructions are disabled for every device compile (their results have been
unreliable on these machines); hipcc's host pass warns that it does not know the
feature, which is harmless.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time
from typing import List

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(CSRC, "_build")
LIB = os.path.join(HERE, "libkf950.so")
ROOT = os.path.dirname(HERE)

ARCH = os.environ.get("KF950_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wno-unused-command-line-argument",
    f"-I{os.path.join(ROOT, 'include')}",
]


# Per-source additions, by file-name prefix. The attention kernels (flash*.hip) rescale
# their output accumulators with VALU, so those are kept in VGPRs (MFMA C/D operands in
# the arch register file) rather than AGPRs, which would cost an accvgpr read and write
# per element per rescale.
SOURCE_FLAGS = {
    "flash": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _source_flags(name: str) -> List[str]:
    return [f for prefix, flags in SOURCE_FLAGS.items() if name.startswith(prefix) for f in flags]


def sources() -> List[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, extra: List[str]) -> str:
    obj = os.path.join(OUT_DIR, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *DEVICE_FLAGS, *_source_flags(os.path.basename(src)), *extra,
           "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{res.stderr[-6000:]}")
    return obj


def build(verbose: bool = False, extra: List[str] = ()) -> str:
    """Compile every kernel source and link libkf950.so; returns the library path."""
    os.makedirs(OUT_DIR, exist_ok=True)
    t0 = time.time()
    srcs = sources()
    workers = min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, list(extra)), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[kf950] built {LIB} from {len(srcs)} sources in {time.time() - t0:.1f}s")
    return LIB


if __name__ == "__main__":
    build(verbose=True, extra=sys.argv[1:])
