"""The planner (csrc/plan.cpp, the host half of the C ABI) under
AddressSanitizer and UndefinedBehaviorSanitizer: tests/host_fuzz/plan_fuzz.cpp
drives every metadata and plan entry point of include/vafa.h with random
segment layouts and corrupted cu_seqlens (see its header for the checks).
Host code only: built with g++, no GPU involved."""
import os
import shutil
import subprocess
import tempfile

import pytest

from conftest import ROOT


def test_planner_under_host_sanitizers():
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    tmp = tempfile.mkdtemp()
    try:
        exe = os.path.join(tmp, "plan_fuzz")
        cmd = [gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
               "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
               "-I", os.path.join(ROOT, "include"),
               os.path.join(ROOT, "tests", "host_fuzz", "plan_fuzz.cpp"),
               os.path.join(ROOT, "varlenabsorbflashattn_amd", "csrc", "plan.cpp"), "-o", exe]
        subprocess.run(cmd, check=True, capture_output=True, text=True)
        for seed in (12345, 7):
            r = subprocess.run([exe, "300", str(seed)], capture_output=True, text=True,
                               timeout=300)
            assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
            assert "0 failed checks" in r.stdout
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
