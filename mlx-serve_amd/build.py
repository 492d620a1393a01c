"""Builds libmi_qmm.so for gfx950 in-tree (mlx-serve_amd/mi_qmm/libmi_qmm.so).

Every HIP source is compiled by hipcc for --offload-arch=gfx950 with packed-fp32
instructions disabled, in parallel, then linked into one shared library.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "mi_qmm")
LIB = os.path.join(OUT_DIR, "libmi_qmm.so")
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HOST = os.path.join(HERE, "host")
ROOT = os.path.dirname(HERE)
SOURCES = ["csrc/qmv1_g64.hip", "csrc/qmv1_g32.hip", "csrc/qmv1_g128.hip", "csrc/qmv1.hip", "csrc/qmv1_fp.hip", "csrc/qmv1_odd.hip", "csrc/qmvm.hip", "csrc/qmvm_gather.hip", "csrc/qmvm_b8.hip", "csrc/qmvm_m64.hip", "csrc/qmvm_fp.hip", "csrc/qmvm_w2.hip", "csrc/qmvm_w3.hip", "csrc/qmvm_w5.hip", "csrc/qmvm_w6.hip", "csrc/qmvm_fp_gather.hip", "csrc/qmv.hip", "csrc/qmv16.hip", "csrc/qmm.hip", "csrc/prefill.hip", "csrc/gmm.hip", "csrc/quant.hip", "csrc/moe.hip", "csrc/moe_down.hip", "csrc/qmv_any.hip",
           "csrc/blas.cpp", "csrc/api.cpp", "host/mi_host.cpp", "host/mi_ckpt.cpp"]
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", os.path.join(ROOT, "include"), "-I", HOST]
TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_host.cpp")
TEST_BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_host")


def _stale(src, obj):
    """True when obj is older than src or than any header under csrc/, host/, include/."""
    if not os.path.exists(obj):
        return True
    newest = os.path.getmtime(os.path.join(HERE, src))
    for d in (os.path.join(HERE, "csrc"), HOST, os.path.join(ROOT, "include")):
        for f in os.listdir(d):
            if f.endswith((".h", ".hpp")):
                newest = max(newest, os.path.getmtime(os.path.join(d, f)))
    return newest > os.path.getmtime(obj)


def _compile(src, incremental=False):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if incremental and not _stale(src, obj):
        return obj
    cmd = [HIPCC] + FLAGS + ["-c", os.path.join(HERE, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stderr or "").splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{errs}")
    return obj


def build(verbose=True, incremental=False):
    """Compile every source (incremental=True skips objects newer than their inputs)."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(HERE, s))]
    with cf.ThreadPoolExecutor(max_workers=min(os.cpu_count() or 8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, incremental), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs + [
        "-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


def build_host_tests(verbose=True):
    """The C++ host-mirror test binary (tests/cpp/test_host.cpp), linked against
    libmi_qmm.so and the oracle (oracle/liboracle.so, its checker)."""
    os.makedirs(os.path.dirname(TEST_BIN), exist_ok=True)
    cmd = [HIPCC, "-O2", "-std=c++17", "-x", "hip", "--offload-arch=gfx950", TEST_SRC,
           "-I", HOST, "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "oracle"),
           "-L", OUT_DIR, "-lmi_qmm", "-L", os.path.join(ROOT, "oracle"), "-loracle",
           "-Wl,-rpath,$ORIGIN/../../../mlx-serve_amd/mi_qmm",
           "-Wl,-rpath,$ORIGIN/../../../oracle", "-o", TEST_BIN]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("test_host build failed:\n" + r.stderr)
    if verbose:
        print("built", TEST_BIN)
    return TEST_BIN


if __name__ == "__main__":
    build(incremental="-i" in sys.argv[1:])
    sys.exit(0)
