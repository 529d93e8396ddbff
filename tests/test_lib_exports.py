"""The C-ABI library loads and exports every symbol include/acorn_hip.h
declares (CPU: no compute calls)."""
import ctypes
import re
from pathlib import Path

import pytest

from acorninfer_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "acorn_hip.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\bint\s+(acorn_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "acorn_paged_attention" in names and "acorn_quant_gemm" in names
    assert len(names) >= 10


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"missing exports: {missing}"


def test_binding_table_matches_header():
    assert sorted(_lib.exported_symbols()) == _declared()


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_version_and_plan_need_no_gpu():
    lib = _lib.lib()
    assert lib.acorn_version() >= 1
    cfg = (ctypes.c_int * 6)()
    rc = lib.acorn_gemm_plan(8, 4096, 12288, _lib.WFMT_W4, cfg)
    assert rc == 0 and all(v >= 1 for v in cfg[:5]) and cfg[5] >= 1
    # an invalid shape maps to the reference's AssertionError
    rc = lib.acorn_gemm_plan(8, 4095, 4096, _lib.WFMT_W4, (ctypes.c_int * 6)())
    with pytest.raises(AssertionError):
        _lib.check(rc, "plan")
