"""The host side and the oracle under AddressSanitizer + UndefinedBehaviorSanitizer.

The C++ host module (host/*.cpp: argument checks, pinned staging pool, copy
threads, checkpoint reader and writer) and the C oracle are rebuilt with
`-fsanitize=address,undefined` by g++ (host code only: no GPU code is built
with a sanitizer) into _build/asan/ and oracle/_build/asan/, and the CPU
suites that drive them run again in a child interpreter with libasan and
libubsan preloaded.  Any sanitizer report fails the run (UBSan halts on the
first error; ASan aborts on its first).  Leak detection is off: the Python
interpreter itself does not free everything at exit.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "callaghandev.ml_amd")
SUITES = ["tests/test_host_cpu.py", "tests/test_checkpoint.py", "tests/test_oracle.py",
          "tests/test_oracle_train.py"]


def _runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


def _stale(target, sources):
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(s) > t for s in sources)


@pytest.fixture(scope="module")
def sanitized_builds():
    sys.path[:0] = [p for p in (ROOT, PKG) if p not in sys.path]
    import sysconfig

    from cdml import build as B

    ext = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    host_so = os.path.join(B.SANITIZE_OUT, "_cdml_host" + ext)
    srcs = (glob.glob(os.path.join(B.HOST, "*.cpp")) + glob.glob(os.path.join(B.HOST, "*.h")) +
            [os.path.join(B.INCLUDE, "cdml.h")])
    if _stale(host_so, srcs):
        B.build_host(sanitize=True)
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    return B.SANITIZE_OUT, os.path.join(ROOT, "oracle", "_build", "asan", "librefcpu.so")


def test_host_and_oracle_suites_under_asan_ubsan(sanitized_builds):
    asan, ubsan = _runtime("libasan.so"), _runtime("libubsan.so")
    if not asan or not ubsan:
        pytest.skip("gcc's libasan / libubsan runtime is not installed")
    host_dir, oracle_lib = sanitized_builds
    env = dict(os.environ)
    env["LD_PRELOAD"] = ":".join([asan, ubsan] + ([env["LD_PRELOAD"]] if env.get("LD_PRELOAD") else []))
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["CDML_HOST_BUILD"] = host_dir
    env["CDML_ORACLE_LIB"] = oracle_lib
    # the child must load the sanitized builds, not the plain ones
    probe = ("import sys; sys.path[:0] = ['.', 'callaghandev.ml_amd']\n"
             "from cdml import host; from oracle import oracle as O; O.lib()\n"
             "print(host.module().__file__); print(O._LIB_PATH)")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    loaded = r.stdout.split()
    assert loaded[0].startswith(host_dir) and loaded[1] == oracle_lib, loaded
    r = subprocess.run([sys.executable, "-m", "pytest", *SUITES, "-x", "-q", "-m", "not gpu",
                        "-p", "no:cacheprovider"], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-5000:]
    for marker in ("runtime error:", "AddressSanitizer", "LeakSanitizer"):
        assert marker not in out, out[-5000:]
