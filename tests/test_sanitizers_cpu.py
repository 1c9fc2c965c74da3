"""Host AddressSanitizer + UndefinedBehaviorSanitizer builds of the CPU-side code (no GPU):

- the BaseBasicStore writer (stlq_amd/csrc/base_store.cpp) under tests/store_sanitize_main.cpp,
  which opens, appends every raw kind, flushes, checkpoints, truncates, resumes and walks the
  error paths;
- the oracle (oracle/stlq_oracle.cpp), loaded into a child Python that runs the oracle's own
  tests (tests/test_oracle_cpu.py: every oracle function, the large root included) through
  STLQ_ORACLE_LIB, with the sanitizer runtimes preloaded.

Any sanitizer report aborts the child (-fno-sanitize-recover=all), so these tests fail on an
out-of-bounds access, use after free or undefined arithmetic in that code."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")


def _runtime(name):
    p = subprocess.run(["g++", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


def _env(preload=False):
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    if preload:
        libs = [_runtime("libasan.so"), _runtime("libubsan.so")]
        if not all(libs):
            pytest.skip("sanitizer runtimes not found")
        env["LD_PRELOAD"] = ":".join(libs)
    return env


def test_store_writer_under_asan_ubsan(tmp_path):
    exe = str(tmp_path / "store_san")
    subprocess.run(["g++", "-std=c++17", *SAN, f"-I{ROOT}/include", f"-I{ROOT}/stlq_amd/csrc",
                    f"{ROOT}/tests/store_sanitize_main.cpp", f"{ROOT}/stlq_amd/csrc/base_store.cpp", "-o", exe],
                   check=True)
    r = subprocess.run([exe, str(tmp_path / "data")], capture_output=True, text=True, env=_env(), timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "store sanitizer run ok" in r.stdout


def test_oracle_under_asan_ubsan(tmp_path):
    so = str(tmp_path / "libstlq_oracle_san.so")
    subprocess.run(["g++", "-std=c++17", "-fPIC", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", *SAN,
                    "-shared", f"{ROOT}/oracle/stlq_oracle.cpp", "-o", so], check=True)
    env = _env(preload=True)
    env["STLQ_ORACLE_LIB"] = so
    env["OMP_NUM_THREADS"] = "4"
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        f"{ROOT}/tests/test_oracle_cpu.py"], capture_output=True, text=True, env=env, cwd=ROOT,
                       timeout=900)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert " passed" in r.stdout
