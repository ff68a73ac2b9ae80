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


def test_capture_refusals(capfd):
    """While a graph capture is open, every entry point that would allocate,
    copy from or to the host or wait refuses with a diagnostic instead of
    breaking the capture.  The capture is simulated (no device here); the
    refusals come before any device or buffer access, so zeroed stand-in
    handles are enough."""
    lib = C.CDLL(str(_native.LIB_DIR / "libds3_hip.so"))
    _native._bind(lib, _native.SIGNATURES)
    if lib.ds3_hip_debug_simulate_capture(1) != 0:
        import pytest
        pytest.skip("a device context is open in this process")
    fake = C.create_string_buffer(64)            # a zeroed ds3_hip_buffer_t stand-in
    fp = C.cast(fake, C.c_void_p)
    data = C.create_string_buffer(4096)
    idx = (C.c_int32 * 8)(*range(8))
    sc = (C.c_float * 8)(*([0.125] * 8))
    try:
        assert lib.ds3_hip_buffer_alloc(4096) is None
        assert lib.ds3_hip_buffer_from_mmap(C.cast(data, C.c_void_p), 4096) is None
        assert lib.ds3_hip_buffer_write(fp, 0, C.cast(data, C.c_void_p), 0) == -1
        assert lib.ds3_hip_buffer_read(fp, 0, C.cast(data, C.c_void_p), 0) == -1
        assert lib.ds3_hip_moe_ffn_experts(fp, fp, fp, fp, 12, 12, 14, 1152, 1152, 630, None, None, None, 0, 0, 0,
                                           0, 0, 0, fp, None, fp, fp, 2048, 8, 768, 0,
                                           idx, sc) == -1
        assert lib.ds3_hip_router_stats(None, None, 0) == -1
        assert lib.ds3_hip_timer_start() == -1
        assert lib.ds3_hip_graph_launch(fp) == -1
        lib.ds3_hip_synchronize()
        lib.ds3_hip_end_batch()
    finally:
        assert lib.ds3_hip_debug_simulate_capture(0) == 0
    err = capfd.readouterr().err
    for what in ("buffer_alloc", "buffer_from_mmap", "buffer_write", "buffer_read", "moe_ffn_experts",
                 "router_stats", "timer_start", "graph_launch"):
        assert f"{what}" in err and "not allowed during graph capture" in err, what
    assert err.count("not allowed during graph capture") >= 8
