"""CPU checks of the C ABI library: it loads without a GPU and exports every
symbol include/hearth_hip.h declares; the product path has no CPU fallback."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "hearth_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(hh_[a-z0-9_]+)\s*\(", txt)))


def test_header_declares_the_binding_surface():
    from hearth_amd.lib import exported_symbols
    assert sorted(exported_symbols()) == declared_symbols()


def test_library_exports_every_declared_symbol():
    from hearth_amd.lib import lib_path
    if not os.path.exists(lib_path()):
        pytest.fail("libhearth_hip.so not built (run __graft_entry__.build())")
    lib = C.CDLL(lib_path())
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_version_and_error_channel_without_gpu():
    from hearth_amd.lib import load_library
    lib = load_library()
    assert b"gfx950" in lib.hh_version()
    # a null output pointer is rejected before any device call
    rc = lib.hh_ctx_create(0, None)
    assert rc == 1 and b"null" in lib.hh_last_error()
    cfg_rc = lib.hh_model_create(None, None, None)
    assert cfg_rc == 1


def test_no_oracle_in_product():
    """The product package never imports or loads the oracle."""
    pkg = os.path.join(ROOT, "hearth_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                txt = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in txt.lower(), f
