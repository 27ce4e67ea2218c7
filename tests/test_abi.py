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


def test_compiler_code_never_uses_m0():
    """The LDS-DMA helpers (csrc/common.h lds_dma16 / lds_dma4) write M0 from
    inline asm, and clang cannot honour M0 in a clobber list: the gfx950
    assembly of every source that uses them must show M0 only inside those asm
    blocks (no compiler-generated instruction that reads or writes it)."""
    import concurrent.futures as cf
    import shutil
    import subprocess
    import tempfile
    import pytest
    from varlenabsorbflashattn_amd import build as B
    try:
        hipcc = B._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    csrc = os.path.join(ROOT, "varlenabsorbflashattn_amd", "csrc")
    users = [f for f in B.SOURCES if f.endswith(".hip")
             and re.search(r"\blds_dma(16|4)\b|\bdma_block\b|\bdma_rows_f32\b",
                           open(os.path.join(csrc, f)).read())]
    assert users
    tmp = tempfile.mkdtemp()

    def asm_of(src):
        out = os.path.join(tmp, src + ".s")
        cmd = [hipcc, *B._flags(), "--cuda-device-only", "-S", "-o", out, os.path.join(csrc, src)]
        subprocess.run(cmd, check=True, capture_output=True)
        inside, bad = False, []
        for line in open(out):
            if "ASMSTART" in line:
                inside = True
            elif "ASMEND" in line:
                inside = False
            elif not inside and re.search(r"\bm0\b", line.split(";")[0]):
                bad.append(line.strip())
        return src, bad

    try:
        with cf.ThreadPoolExecutor(max_workers=min(4, len(users))) as ex:
            for src, bad in ex.map(asm_of, users):
                assert not bad, (src, bad[:5])
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
