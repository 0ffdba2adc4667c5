"""The host C library (the .sp-model loader, bridge, session verbs, hashes and
OK_Q4B producer) and the oracle under AddressSanitizer and
UndefinedBehaviorSanitizer, on the CPU: `make asan` builds instrumented copies
into lib-asan/, and the format, boundary and session-routing tests -- the
malformed-file cases included -- run against them in a child process with the
ASan runtime preloaded.  Any report aborts the child (-fno-sanitize-recover,
halt_on_error), so the test fails on the first finding.  Leak checking is off:
the interpreter itself does not free everything at exit."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "shannon-prime-system_amd")
ORACLE = os.path.join(ROOT, "oracle")


def _runtime():
    try:
        p = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True, check=True)
    except (OSError, subprocess.CalledProcessError):
        return None
    path = os.path.realpath(p.stdout.strip())
    return path if os.path.isfile(path) else None


def test_host_c_under_asan_and_ubsan(tmp_path):
    asan = _runtime()
    if not asan:
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    if not os.path.exists(os.path.join(PKG, "build", "hip", "kvd_table.o")):
        pytest.skip("the HIP objects are not built (the sanitizer build relinks them)")
    for d in (PKG, ORACLE):
        r = subprocess.run(["make", "-s", "-j8", "-C", d, "asan"], capture_output=True, text=True)
        assert r.returncode == 0, r.stdout + r.stderr
    env = dict(os.environ,
               LD_PRELOAD=asan,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               SPKV_LIB_DIR=os.path.join(PKG, "lib-asan"),
               ORC_LIB_DIR=os.path.join(ORACLE, "lib-asan"),
               OMP_NUM_THREADS="2")
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
           "--basetemp", str(tmp_path / "t"),
           os.path.join(ROOT, "tests", "test_format.py"),
           os.path.join(ROOT, "tests", "test_boundary_abi.py"),
           os.path.join(ROOT, "tests", "test_session_routing.py"),
           os.path.join(ROOT, "tests", "test_oracle_exact.py"),
           # the oracle's larger sweeps run in the plain build only (minutes under the sanitizers)
           "-k", "not threads_do_not_change and not tracks_float_mode"]
    r = subprocess.run(cmd, env=env, capture_output=True, text=True, cwd=ROOT, timeout=900)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert " passed" in r.stdout and "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, tail
