"""The C-ABI library loads on the CPU and exports every symbol include/snnk.h declares."""
import ctypes
import pathlib
import re

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "snnk.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(snnk_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "snnk_lif_forward" in syms and "snnk_version" in syms


def test_library_exports_all_declared_symbols():
    from snnk import _abi
    lib = _abi.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), f"libsnnk.so does not export {name}"
    for name in _abi.PROTOTYPES:
        assert name in declared_symbols(), f"{name} bound in _abi but not declared in snnk.h"
    assert lib.snnk_version() >= 100
    assert lib.snnk_status_string(-1) == b"invalid argument"


def test_invalid_arguments_rejected_without_gpu():
    """Argument validation happens before any HIP call."""
    from snnk import _abi
    lib = _abi.lib()
    # negative T
    st = lib.snnk_lif_forward(None, 0, None, None, None, 0, 1.0, None, None, None, 0,
                              None, -1, 10, 1, 1, 0, 0.5, 0.5, 0.0, 0, None)
    assert st == _abi.EINVAL
    # empty problem is a no-op success
    st = lib.snnk_lif_forward(None, 0, None, None, None, 0, 1.0, None, None, None, 0,
                              None, 0, 10, 1, 1, 0, 0.5, 0.5, 0.0, 0, None)
    assert st == _abi.OK
    # bad threshold mode
    st = lib.snnk_lif_forward(ctypes.c_void_p(16), 0, None, None, None, 7, 1.0, None, None,
                              ctypes.c_void_p(16), 0, None, 4, 10, 1, 1, 0, 0.5, 0.5, 0.0,
                              0, None)
    assert st == _abi.EINVAL
