"""The C-ABI library loads and exports every symbol include/vafa.h declares."""
import ctypes
import os
import re

from conftest import ROOT
from varlenabsorbflashattn_amd import _lib

HEADER = os.path.join(ROOT, "include", "vafa.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"VAFA_API\s+[\w\s\*]+?\b(vafa_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for name in ("vafa_varlen_fwd", "vafa_varlen_bwd", "vafa_absorb_fwd", "vafa_absorb_bwd",
                 "vafa_plan_varlen", "vafa_plan_absorb", "vafa_version", "vafa_last_error"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    h = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(h, s)]
    assert not missing, missing


def test_binding_covers_header():
    assert sorted(_lib.EXPORTED) == declared_symbols()


def test_version_string():
    assert _lib.lib().vafa_version().startswith(b"vafa")
