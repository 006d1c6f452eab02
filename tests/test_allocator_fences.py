"""CPU test of the block allocator's stream-ordering contract (no GPU).

Builds tests/allocator_fence_test.cpp with the allocator's bookkeeping
(gaudirt_amd/csrc/block_allocator_core.cpp, the code the library runs) and a
recording mock of the device runtime, with g++, and runs it. The cases follow
the reference's tests/block_allocator_fences_unit_test.cpp:25-71: cross-stream
reuse fences every other producer with a record followed by a wait,
same-stream reuse needs none, producers survive splits and merges, an event is
never recorded again before its wait, and steady state creates no events.
"""

import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parent.parent
CSRC = ROOT / "gaudirt_amd" / "csrc"


def test_allocator_fence_contract(tmp_path):
    exe = tmp_path / "allocator_fence_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-fsanitize=address,undefined", "-I", str(CSRC),
                    str(ROOT / "tests" / "allocator_fence_test.cpp"), str(CSRC / "block_allocator_core.cpp"),
                    "-o", str(exe)], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    assert run.stdout.strip() == "OK"
