"""The host-side request packing (ft_runtime.cpp: SSE2 row scan, token
sorting, length-norm table, key bounds) against a plain scalar restatement
of the staging format, on thousands of random requests -- compiled with g++
from the runtime's own source, no GPU."""

import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_packing_matches_scalar_restatement(tmp_path):
    exe = tmp_path / "staging_check"
    subprocess.check_call(
        ["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-D__HIP_PLATFORM_AMD__",
         "-I/opt/rocm/include", "-I" + os.path.join(ROOT, "include"),
         "-I" + os.path.join(ROOT, "flash-trie_amd", "csrc"),
         os.path.join(ROOT, "tests", "native", "staging_check.cpp"), "-o", str(exe),
         "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-lpthread"],
        stderr=subprocess.DEVNULL)
    p = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stdout
    assert "0 failures" in p.stdout and "0 streamed" not in p.stdout, p.stdout
    assert " 0 rows scanned" not in p.stdout, p.stdout
