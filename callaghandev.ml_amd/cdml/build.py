"""Builds the native libraries in-tree (no JIT cache, no site-packages).

* ``_build/libcdml_hip.so``: the gfx950 kernels and the C ABI of
  ``include/cdml.h`` (hipcc, one object per ``csrc/*.hip``, compiled in
  parallel, then linked).
* ``_build/_cdml_host*.so``: the C++ host-side manager
  (``host/*.cpp``) with its pybind11 module, linked against the C ABI only.

Every HIP object is compiled for gfx950 with packed-fp32 instruction
selection disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
OUT = os.path.join(PKG, "_build")
LIB = os.path.join(OUT, "libcdml_hip.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("CDML_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-I" + INCLUDE,
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + r.stdout + r.stderr)
    return r


def build_hip(verbose: bool = False) -> str:
    os.makedirs(os.path.join(OUT, "obj"), exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = [os.path.join(OUT, "obj", os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = min(len(srcs), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", s, "-o", o]) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


# Host-code-only sanitizer build (g++; no GPU code is built with it): the
# checked variant of the host module that tests load from _build/asan/.
SANITIZE_FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                  "-fno-sanitize-recover=undefined"]
SANITIZE_OUT = os.path.join(OUT, "asan")


def build_host(verbose: bool = False, sanitize: bool = False) -> str:
    """The pybind11 host module; with sanitize, an ASan + UBSan build of the
    same sources into _build/asan/ (it needs libasan preloaded to import)."""
    import pybind11

    srcs = sorted(glob.glob(os.path.join(HOST, "*.cpp")))
    if not srcs:
        return ""
    ext = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out_dir = SANITIZE_OUT if sanitize else OUT
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "_cdml_host" + ext)
    tmp = out + ".tmp"
    opt = SANITIZE_FLAGS if sanitize else ["-O2"]
    rpath = "-Wl,-rpath,$ORIGIN/.." if sanitize else "-Wl,-rpath,$ORIGIN"
    if sanitize:
        # one object per source in parallel: the sanitized compile is slow
        objs = [os.path.join(out_dir, os.path.basename(s)[:-4] + ".o") for s in srcs]
        base = ["g++", *opt, "-std=c++17", "-fPIC", "-fvisibility=hidden", "-I" + INCLUDE, "-I" + HOST,
                "-I" + pybind11.get_include(), "-I" + sysconfig.get_paths()["include"]]
        with cf.ThreadPoolExecutor(min(len(srcs), os.cpu_count() or 4)) as ex:
            for f in [ex.submit(_run, base + ["-c", s, "-o", o]) for s, o in zip(srcs, objs)]:
                f.result()
        _run(["g++", *opt, "-shared", *objs, "-o", tmp, "-L" + OUT, "-lcdml_hip", rpath])
    else:
        _run(["g++", *opt, "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
              "-I" + INCLUDE, "-I" + HOST, "-I" + pybind11.get_include(),
              "-I" + sysconfig.get_paths()["include"], *srcs, "-o", tmp,
              "-L" + OUT, "-lcdml_hip", rpath])
    os.replace(tmp, out)
    if verbose:
        print("built", out)
    return out


def build(verbose: bool = False):
    build_hip(verbose)
    build_host(verbose)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
