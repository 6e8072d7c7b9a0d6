"""The device library loads without a GPU and exports every entry point its
header declares (no compute calls here)."""
import ctypes

from cpde_amd import hip


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(hip.LIB_PATH))
    declared = hip.header_symbols()
    assert len(declared) >= 40
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, missing


def test_binding_covers_header():
    assert sorted(hip.SIGNATURES) == hip.header_symbols()


def test_error_convention_without_device():
    lib = hip.load()
    # invalid trace kind is rejected as an argument error before any device work
    assert lib.cpde_trace_name(-1) == b''
    assert lib.cpde_trace_kinds() > 0
