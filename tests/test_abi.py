"""The C ABI: libkf950.so loads and exports exactly what include/kf950.h declares.

CPU only: no entry point that launches a kernel is called. `kf_abi_version` and
`kf_last_error` touch no device.
"""
from __future__ import annotations

import os
import re

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
