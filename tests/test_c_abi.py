"""The C ABI from plain C: tests/c_abi/abi_check.c compiled with gcc -std=c99
-Wall -Werror against include/ullm_hip.h alone, linked to libullm_hip.so and
run (CPU only: every call it makes returns before any device work)."""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "ullm_amd")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no gcc")
def test_plain_c_client_builds_and_passes():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "abi_check")
        cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic",
               "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "c_abi", "abi_check.c"),
               "-L", LIBDIR, "-lullm_hip", f"-Wl,-rpath,{LIBDIR}", "-lm", "-o", exe]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stdout + r.stderr
        assert "all checks passed" in r.stdout
