"""The C ABI: libkf950.so loads and exports exactly what include/kf950.h declares.

CPU only: no entry point that launches a kernel is called. `kf_abi_version` and
`kf_last_error` touch no device.
"""
from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess

import pytest

from techjam2026_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kf950.h")


def declared_functions():
    text = open(HEADER, encoding="utf-8").read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kf_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_python_export_list():
    assert declared_functions() == sorted(L.EXPORTS)


@pytest.mark.skipif(not L.available(), reason="libkf950.so not built")
def test_library_loads_and_exports_every_declared_symbol():
    h = L.lib()
    for name in declared_functions():
        assert hasattr(h, name), f"{name} missing from libkf950.so"
    assert h.kf_abi_version() == L.ABI_VERSION


def exported_kf_symbols():
    """The library's dynamic `kf_*` function symbols (GNU nm, defined text symbols)."""
    out = subprocess.run([shutil.which("nm") or "nm", "-D", "--defined-only", L.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    return sorted({ln.split()[-1] for ln in out.splitlines()
                   if len(ln.split()) == 3 and ln.split()[1] in "Tt"
                   and ln.split()[-1].startswith("kf_")})


@pytest.mark.skipif(not L.available() or shutil.which("nm") is None,
                    reason="libkf950.so not built, or no nm")
def test_library_exports_nothing_the_header_does_not_declare():
    """The exported kf_* set equals the header's: no internal helper leaks into the ABI."""
    assert exported_kf_symbols() == declared_functions()


@pytest.mark.skipif(not L.available(), reason="libkf950.so not built")
def test_header_constants_match_python_constants():
    text = open(HEADER, encoding="utf-8").read()
    consts = dict((k, int(v)) for k, v in re.findall(r"\b(KF_[A-Z0-9_]+)\s*=\s*(\d+)", text))
    assert consts["KF_F32"] == L.F32 and consts["KF_U8"] == L.U8
    assert consts["KF_MMA_F16X3"] == L.MMA_F16X3 and consts["KF_MMA_BF16X3"] == L.MMA_BF16X3
    assert consts["KF_LN_WRITE_S"] == L.LN_WRITE_S and consts["KF_LN_MASK_OUT"] == L.LN_MASK_OUT
    assert consts["KF_FLASH_SKIP_PAD_ROWS"] == L.FLASH_SKIP_PAD_ROWS
    assert consts["KF_EUNSUPPORTED"] == L.EUNSUPPORTED
    assert int(re.search(r"#define KF_ABI_VERSION (\d+)", text).group(1)) == L.ABI_VERSION


@pytest.mark.skipif(not L.available(), reason="libkf950.so not built")
def test_argument_errors_are_reported_without_a_device():
    """Validation happens before any launch: a NULL input is EINVAL with a message."""
    h = L.lib()
    st = h.kf_gemm(None, None, L.F32, 8, None, None, 8, None, None, None, L.F32, 8, 8, 8, 8,
                   L.MMA_F16X3, L.ACT_NONE, None)
    assert st == L.EINVAL
    assert b"kf_gemm" in h.kf_last_error()
    with pytest.raises(L.KernelError):
        L.check("kf_gemm", st)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(L, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(L, "_handle", None)
    with pytest.raises(RuntimeError, match="not found"):
        L.lib()


@pytest.mark.skipif(not L.available(), reason="libkf950.so not built")
@pytest.mark.parametrize("B,H,S,hd", [
    (1 << 20, 1 << 16, 1 << 26, 256),   # B*H*S*hd*2 = 2^71: wraps to 0 in 64 bits
    (1 << 20, 1 << 16, (1 << 26) - 8, 128),
    (1 << 19, 1 << 15, 1 << 20, 64),
    (64, 16, 65536, 64),                # no wrap, simply more than the 64 MiB scratch
])
def test_static_attention_rejects_oversized_staging_before_touching_a_device(B, H, S, hd):
    """The allocation-free attention sizes its staging by division, so extents whose
    byte product would wrap in 64 bits are refused (EINVAL) like any other oversized
    problem -- before any device call (the pointers here are never dereferenced)."""
    h = L.lib()
    fake = ctypes.c_void_p(4096)
    st4 = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    for mode in (L.MMA_F16, L.MMA_F16X3):
        st = h.kf_flash_attention_static(fake, st4, fake, st4, fake, st4, L.F32, fake, None, st4,
                                         L.F32, None, L.U8, S, B, H, S, hd, 0.125, mode, 0, None)
        assert st == L.EINVAL, (B, H, S, hd, mode)
        assert b"static scratch" in h.kf_last_error()


@pytest.mark.skipif(not L.available(), reason="libkf950.so not built")
def test_qkv_projection_takes_both_lo_planes_or_neither():
    """A split-mode kf_gemm_qkv with only one of the k / v^T lo planes is refused before any
    launch (EINVAL); f16x2 with none is refused too (it writes split planes). The pointers
    are never dereferenced."""
    h = L.lib()
    p = ctypes.c_void_p(4096)
    B, S, H, hd = 2, 64, 4, 64
    d = H * hd
    for k_lo, vt_lo, mode, a_dtype, want in ((p, None, L.MMA_F16X3, L.F16X2, L.EINVAL),
                                            (None, p, L.MMA_F16X3, L.F16X2, L.EINVAL),
                                            (None, None, L.MMA_F16X2, L.F16, L.EUNSUPPORTED)):
        st = h.kf_gemm_qkv(p, p, a_dtype, d, p, p, d, p, p, p, k_lo, p, vt_lo, S, B, S, H, hd,
                           mode, None)
        assert st == want, (mode, k_lo, vt_lo)
        assert b"kf_gemm_qkv" in h.kf_last_error()
