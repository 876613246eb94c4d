"""The arena's reuse rules across streams (vearo_amd/csrc/arena.h), on the CPU:
tests/cpp/test_arena.cpp drives the free-list core with a fake device that logs
allocations, event records and stream waits."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_arena_free_list_rules(tmp_path):
    exe = tmp_path / "test_arena"
    src = os.path.join(ROOT, "tests", "cpp", "test_arena.cpp")
    inc = os.path.join(ROOT, "vearo_amd", "csrc")
    subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fsanitize=address,undefined",
                    "-I", inc, "-o", str(exe), src], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "arena tests ok" in r.stdout
