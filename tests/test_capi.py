"""The C ABI library loads and exports what include/bsamd.h declares (CPU).

No compute is launched here: argument validation returns before any HIP
call, so the error paths are exercised without a GPU.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from blockstreamer_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "bsamd.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(bsa_\w+)\s*\(", text))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = declared_symbols()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in bsamd.h but not exported"


def test_binding_matches_header():
    assert declared_symbols() == set(_lib.symbols())


def test_version():
    """Library, header and binding agree on the ABI major number."""
    major = int(re.search(r"#define BSA_VERSION_MAJOR (\d+)", HEADER.read_text()).group(1))
    assert _lib.lib().bsa_version() // 100 == _lib.ABI_MAJOR == major


def test_dequant_rejects_bad_arguments_without_gpu():
    lib = _lib.lib()
    null = ctypes.c_void_p(0)
    rc = lib.bsa_dequant_mxfp4(null, null, null, 0, -1, 4, 4, null)
    assert rc == _lib.BSA_EINVAL
    assert b"negative shape" in lib.bsa_last_error()
    rc = lib.bsa_dequant_mxfp4(null, null, null, 7, 1, 4, 4, null)
    assert rc == _lib.BSA_EINVAL and b"dtype" in lib.bsa_last_error()
    rc = lib.bsa_dequant_mxfp4_mode(null, null, null, 0, 1, 4, 4, 9, null)
    assert rc == _lib.BSA_EINVAL and b"mode" in lib.bsa_last_error()
    rc = lib.bsa_dequant_mxfp4(null, null, null, 0, 1, 8, 4, null)
    assert rc == _lib.BSA_EINVAL and b"null" in lib.bsa_last_error()
    # empty problems are a no-op that succeeds
    assert lib.bsa_dequant_mxfp4(null, null, null, 0, 0, 8, 4, null) == _lib.BSA_OK
    with pytest.raises(ValueError, match="mode"):
        _lib.call("bsa_dequant_mxfp4_mode", None, None, None, 0, 1, 4, 4, 9, None)
