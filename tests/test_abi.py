"""The C ABI library loads without a GPU and exports exactly what include/h3fp8.h declares (no compute calls)."""
import ctypes
import os
import re

from conftest import ROOT


def _declared():
    src = open(os.path.join(ROOT, "include", "h3fp8.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(h3fp8_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    names = _declared()
    assert "h3fp8_gemm" in names and "h3fp8_quant_rows" in names and "h3fp8_gemm_swiglu_quant" in names
    assert len(names) >= 15


def test_library_exports_every_declared_symbol():
    from h3_tp2_amd import _lib
    L = _lib.load()
    missing = [n for n in _declared() if not hasattr(L, n)]
    assert not missing, missing
    assert sorted(_lib.EXPORTS) == _declared(), "the ctypes signature table must cover the header exactly"


def test_abi_version_and_error_string_without_gpu():
    from h3_tp2_amd import _lib
    L = _lib.load()
    assert L.h3fp8_abi_version() == _lib.ABI_VERSION == 1
    assert isinstance(L.h3fp8_last_error(), bytes)


def test_argument_errors_are_reported_without_touching_the_gpu():
    """Shape checks run before any HIP call: a bad K returns EINVAL and sets the thread's error string."""
    from h3_tp2_amd import _lib
    L = _lib.load()
    rc = L.h3fp8_quant_rows(ctypes.c_void_p(16), 16, 4, 12, ctypes.c_void_p(16), 16, ctypes.c_void_p(16), None)
    assert rc == -22 and b"multiple of 8" in L.h3fp8_last_error()
    rc = L.h3fp8_gemm(None, 32, None, 32, None, 1, None, 1, None, None, 32, 0, 4, 24, 24, None, None)
    assert rc == -22 and b"multiples of 16" in L.h3fp8_last_error()
    rc = L.h3fp8_gemm(None, 32, None, 32, None, 1, None, 1, None, None, 32, 0, 4, 32, 0, None, None)
    assert rc == -22 and b"K must be positive" in L.h3fp8_last_error()


def test_missing_library_fails_loudly(tmp_path):
    import pytest

    from h3_tp2_amd import _lib
    with pytest.raises(FileNotFoundError):
        _lib.load(str(tmp_path / "libh3fp8.so"))
