"""The C-ABI library loads on a machine without a GPU and exports every symbol include/ingot_hip.h declares."""
import ctypes

from ingot_amd import _lib


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = _lib.declared_symbols()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_no_device_reports_an_error_not_a_crash():
    L = _lib.lib()
    h = ctypes.c_void_p()
    code = L.ih_init(999, ctypes.byref(h))
    assert code != 0 and h.value is None
    assert L.ih_last_error()
