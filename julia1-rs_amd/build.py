"""Build the gfx950 HIP library in-tree, as a shared object and as a static
archive, and a plain-C caller linked against the archive:

    julia1-rs_amd/lib/libjulia1_hip.so   (ctypes: the Python package and tests)
    julia1-rs_amd/lib/libjulia1_hip.a    (what a Rust build.rs links)
    julia1-rs_amd/lib/jh_caller          (tests/c_abi/jh_caller.c, C99, against the .a)

    python julia1-rs_amd/build.py [--jobs N]

Every source is compiled with hipcc for gfx950 only (non-relocatable device
code: each object carries its own code object and registers it at load, so
the archive links like any C++ library); packed-FP32 instructions are disabled
on the device (the host pass warns that it does not know the feature, which
is harmless).  Objects go to julia1-rs_amd/_build/.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib", "libjulia1_hip.so")
ARCHIVE = os.path.join(HERE, "lib", "libjulia1_hip.a")
CALLER_SRC = os.path.join(ROOT, "tests", "c_abi", "jh_caller.c")
CALLER = os.path.join(HERE, "lib", "jh_caller")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++20", "-fPIC", "-Wall", "-Wno-unused-function", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{os.path.join(ROOT, 'include')}"]


def sources():
    out = []
    for d in (CSRC, HOST):
        if not os.path.isdir(d):
            continue
        for f in sorted(os.listdir(d)):
            if f.endswith((".hip", ".cpp")):
                out.append(os.path.join(d, f))
    return out


def compile_one(src: str) -> str:
    obj = os.path.join(BUILD, os.path.relpath(src, HERE).replace(os.sep, "_") + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *FLAGS, *lang, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    build_static(objs)
    return LIB


def _run(cmd, what):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed: {' '.join(cmd)}\n{r.stdout}{r.stderr}")


def build_static(objs):
    """libjulia1_hip.a from the same objects, and the C99 caller linked against it with the system
    C/C++ toolchain plus the HIP runtime (the link a Rust build.rs performs)."""
    tmp = ARCHIVE + ".tmp"
    if os.path.exists(tmp):
        os.remove(tmp)
    _run(["ar", "rcs", tmp, *objs], "ar")
    os.replace(tmp, ARCHIVE)
    obj = os.path.join(BUILD, "jh_caller.o")
    _run(["gcc", "-std=c99", "-O2", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{os.path.join(ROOT, 'include')}",
          "-c", CALLER_SRC, "-o", obj], "compiling the C caller")
    _run(["g++", "-o", CALLER + ".tmp", obj, ARCHIVE, f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"],
         "linking the C caller against the static library")
    os.replace(CALLER + ".tmp", CALLER)


def clean():
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--clean", action="store_true")
    args = ap.parse_args()
    if args.clean:
        clean()
    print(build(args.jobs))
