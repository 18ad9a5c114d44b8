"""The output ring's slot and lease policy (gsplat_tt_amd/csrc/out_ring.h) on
the CPU: tests/out_ring_check.cpp is built with g++ against the header (malloc
and free as the allocator) and run, once plain and once under AddressSanitizer
(host code only) so that a buffer freed twice, used after free or leaked fails."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "out_ring_check.cpp")
INC = os.path.join(ROOT, "gsplat_tt_amd", "csrc")


def _build_and_run(tmp_path, extra):
    exe = str(tmp_path / "out_ring_check")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-Wall", "-Wextra", "-Werror", "-I", INC, SRC,
           "-o", exe, "-pthread"] + extra
    subprocess.run(cmd, check=True, timeout=120)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert r.stdout.startswith("ok"), r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_out_ring_policy(tmp_path):
    _build_and_run(tmp_path, [])


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_out_ring_policy_asan(tmp_path):
    probe = subprocess.run(["g++", "-fsanitize=address", "-x", "c++", "-", "-o",
                            str(tmp_path / "probe")], input="int main(){return 0;}",
                           text=True, capture_output=True)
    if probe.returncode != 0:
        pytest.skip("g++ has no AddressSanitizer runtime here")
    _build_and_run(tmp_path, ["-fsanitize=address,undefined", "-fno-omit-frame-pointer"])
