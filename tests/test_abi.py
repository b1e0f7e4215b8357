"""The C-ABI library loads and exports every symbol `include/omnia_hip.h` declares.

No compute entry point is called here (no GPU); `omnia_abi_version` is pure.
"""

import ctypes
import re
from pathlib import Path

import pytest

from mlx_omnia_amd.runtime import loader as lib_module

HEADER = Path(__file__).resolve().parent.parent / "include" / "omnia_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(omnia_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not lib_module.LIBRARY_PATH.exists():
        pytest.fail("libomnia_hip.so is not built; run __graft_entry__.build()")
    return lib_module.library()


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "omnia_abi_version" in names and "omnia_last_error" in names
    assert len(names) >= 3


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(str(lib_module.LIBRARY_PATH))
    missing = [name for name in declared_symbols() if not hasattr(raw, name)]
    assert not missing, missing


def test_bindings_cover_the_header(lib):
    assert set(declared_symbols()) == set(lib_module.SIGNATURES)


def test_abi_version(lib):
    assert lib.omnia_abi_version() == lib_module.ABI_VERSION
    match = re.search(r"#define OMNIA_ABI_VERSION (\d+)", HEADER.read_text())
    assert match and int(match.group(1)) == lib_module.ABI_VERSION


def test_argument_errors_come_back_as_codes(lib):
    """A rejected shape returns -EINVAL before any device call (no GPU needed)."""
    rc = lib.omnia_add_rms_norm(None, None, None, None, None, 4, 7, 1e-6, None)
    assert rc == -22
    assert "hidden" in lib_module.last_error()
    assert lib.omnia_add_rms_norm(None, None, None, None, None, 0, 2560, 1e-6, None) == 0
    assert lib.omnia_dense_gate_up_swiglu(None, None, 12, 8, None, None) == -22
    assert "hidden" in lib_module.last_error()
    assert lib.omnia_dense_gate_up_swiglu(None, None, 8200, 8, None, None) == -22
    assert lib.omnia_dense_down_residual(None, None, None, 8, 12, None, None) == -22
    assert "inner" in lib_module.last_error()
    assert lib.omnia_moe_down_combine(None, None, 4, 8, 2056, None, None, 1, None, None, None) == -22


def test_router_pack_size_is_pure(lib):
    assert lib.omnia_router_pack_bytes(128, 2048) == 2 * 128 * 2048 * 2 + 128 * 4
    assert lib.omnia_router_pack_bytes(100, 2048) == -22
    assert lib.omnia_router_pack_bytes(128, 2000) == -22
