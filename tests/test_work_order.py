"""CPU test of the prefill kernel's work order inside one XCD's share and of the
balanced decode schedule's 32-bit tile gate (no GPU).

Builds tests/work_order_test.cpp against gaudirt_amd/csrc/work_order.hpp (the
code the kernel runs) with g++ and runs it: every share of many launch shapes
must be visited as a permutation, row tiles highest first, items ascending
within a row tile.
"""

import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parent.parent
CSRC = ROOT / "gaudirt_amd" / "csrc"


def test_heavy_first_order(tmp_path):
    exe = tmp_path / "work_order_test"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-fsanitize=address,undefined", "-I", str(CSRC),
                    str(ROOT / "tests" / "work_order_test.cpp"), "-o", str(exe)], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip() == "OK"
