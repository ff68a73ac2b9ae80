"""The C-ABI library loads without a GPU and exports every entry point the
header declares; the Python binding table matches the header."""
import ctypes as C
import re
from pathlib import Path

from qw3_amd import _native

ROOT = Path(__file__).resolve().parent.parent


def test_header_symbols_exported():
    lib = C.CDLL(str(_native.LIB_DIR / "libds3_hip.so"))
    names = _native.header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_table_covers_header():
    assert sorted(_native.SIGNATURES) == _native.header_functions()


def test_every_declaration_cites_the_reference():
    """Each ds3_metal.h replacement sits under a comment citing the reference
    declaration it replaces; the extensions section says it has none."""
    text = (ROOT / "include" / "ds3_hip.h").read_text()
    head, ext = text.split("Device-routed extensions")
    lines = head.splitlines()
    last_cite = -100
    for i, line in enumerate(lines):
        if "reference src/ds3_metal.h" in line:
            last_cite = i
        for name in re.findall(r"\b(ds3_hip_\w+)\s*\(", line):
            assert i - last_cite <= 14, f"{name} has no nearby reference citation"
    assert "no ds3_metal.h counterpart" in ext.splitlines()[0]


def test_generator_exports():
    lib = C.CDLL(str(_native.LIB_DIR / "libds3gen.so"))
    for n in _native.GEN_SIGNATURES:
        assert hasattr(lib, n)


def test_compat_header_maps_every_metal_name():
    """Every replacement of a ds3_metal.h entry point (the header part before
    the extensions section) has its ds3_metal_* alias."""
    compat = (ROOT / "include" / "ds3_metal_compat.h").read_text()
    head = (ROOT / "include" / "ds3_hip.h").read_text().split("Device-routed extensions")[0]
    names = sorted(set(re.findall(r"\b(ds3_hip_\w+)\s*\(", head)))
    assert len(names) >= 30
    for name in names:
        metal = name.replace("ds3_hip_", "ds3_metal_")
        assert f"#define {metal} {name}" in compat, metal
