"""CPU tier: the C-ABI library loads and exports every symbol the header declares."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "latticequant_amd.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(lq_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_header_symbols():
    import torch  # noqa: F401  (binds the HIP runtime first, as the package does)
    from latticequant_amd import _lib
    lib = _lib.load()
    declared = _declared()
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert sorted(_lib.exported_symbols()) == declared
    assert lib.lq_version() >= 10000
    assert lib.lq_status_string(-3).decode().startswith("rANS alphabet")


def test_library_is_gfx950():
    path = os.path.join(ROOT, "latticequant_amd", "liblatticequant_amd.so")
    data = open(path, "rb").read()
    assert b"gfx950" in data
