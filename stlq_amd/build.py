"""Builds libstlq_mi355.so (gfx950) in-tree: stlq_amd/lib/libstlq_mi355.so.

Every HIP translation unit is compiled with
  -ffp-contract=off   one IEEE-rounded operation per source operation (the candidate-cost,
                      LS and cost arithmetic must match the reference's non-FMA build)
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed fp32 VALU instructions
and the default correctly-rounded fp32 division and square root.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libstlq_mi355.so")
# test driver of the C++ host mirror (stlq_amd/host/stlq_mi355.hpp), linked against LIB
HOSTCHECK_SRC = os.path.join(ROOT, "tests", "host_mirror_check.cpp")
HOSTCHECK = os.path.join(LIBDIR, "libstlq_mi355_hostcheck.so")
SOURCES = ["k_precomp.hip", "k_gemm.hip", "k_beam.hip", "k_beam_queue.hip", "k_beam_staged_a.hip",
           "k_beam_staged_b.hip", "k_ls.hip", "capi.hip"]
HOST_SOURCES = ["base_store.cpp"]  # plain host C++ (the on-disk store), built by the host compiler
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-command-line-argument",
        f"-I{os.path.join(ROOT, 'include')}",
        f"-I{CSRC}",
    ]


def _compile(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc()] + common_flags() + ["-c", os.path.join(CSRC, src), "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return out


def host_flags() -> list[str]:
    return ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra",
            f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}"]


def _compile_host(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".host.o")
    cmd = [os.environ.get("CXX", "g++")] + host_flags() + ["-c", os.path.join(CSRC, src), "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return out


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    jobs = min(len(SOURCES) + len(HOST_SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        hip_objs = ex.map(_compile, SOURCES)
        host_objs = ex.map(_compile_host, HOST_SOURCES)
        objs = list(hip_objs) + list(host_objs)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    build_hostcheck()
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_hostcheck() -> str:
    """g++ build of the host-mirror test driver; only the C ABI header is needed."""
    tmp = HOSTCHECK + ".tmp"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
           f"-I{os.path.join(ROOT, 'include')}", HOSTCHECK_SRC, "-o", tmp,
           f"-L{LIBDIR}", "-lstlq_mi355", "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"host mirror build failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, HOSTCHECK)
    return HOSTCHECK


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
