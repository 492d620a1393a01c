"""The workspace growth rule, on the CPU: compiles tests/cpp/test_workspace_pool.cpp
against mlx-serve_amd/csrc/workspace_pool.h with g++ and runs it."""
import os
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_workspace_generations_survive_growth():
    src = os.path.join(ROOT, "tests", "cpp", "test_workspace_pool.cpp")
    inc = os.path.join(ROOT, "mlx-serve_amd", "csrc")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "t")
        subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", inc, src, "-o", exe],
                       check=True)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
        assert r.returncode == 0, r.stdout + r.stderr
