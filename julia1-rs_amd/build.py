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
import json
import re
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


RESOURCE_REMARK = "kernel-resource-usage"
RESOURCES = os.path.join(BUILD, "kernel_resources.json")


def kernel_resources(text: str) -> dict:
    """{kernel: {"vgprs", "agprs", "sgprs", "scratch", "lds"}} from the compiler's
    -Rpass-analysis=kernel-resource-usage remarks (one "Function Name:" line per
    kernel followed by its figures)."""
    keys = {"VGPRs": "vgprs", "AGPRs": "agprs", "SGPRs": "sgprs", "ScratchSize [bytes/lane]": "scratch",
            "LDS Size [bytes/block]": "lds"}
    out, cur = {}, None
    for line in text.splitlines():
        if RESOURCE_REMARK not in line or "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].rsplit("[-Rpass-analysis", 1)[0].strip()
        if body.startswith("Function Name:"):
            cur = body.split(":", 1)[1].strip()
            out[cur] = {}
        elif cur is not None and ":" in body:
            k, v = body.rsplit(":", 1)
            if k.strip() in keys:
                out[cur][keys[k.strip()]] = int(v.strip())
    return out


def compile_one(src: str) -> tuple[str, dict]:
    obj = os.path.join(BUILD, os.path.relpath(src, HERE).replace(os.sep, "_") + ".o")
    hip = src.endswith(".hip")
    lang = ["-x", "hip", f"-Rpass-analysis={RESOURCE_REMARK}"] if hip else []
    cmd = [HIPCC, *FLAGS, *lang, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    text = r.stdout + r.stderr
    keep, in_remark = [], False
    for l in text.splitlines():
        if RESOURCE_REMARK in l:
            in_remark = True  # the remark and the source excerpt under it
        elif not (in_remark and re.match(r"^\s*\d*\s*\|", l)):
            in_remark = False
            if "packed-fp32-ops" not in l:
                keep.append(l)
    msgs = "\n".join(keep)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj, kernel_resources(text) if hip else {}


def check_no_scratch(resources: dict) -> None:
    """Every kernel keeps its state in registers and LDS: a kernel with per-lane
    scratch (a private array the compiler could not keep in registers, or
    spills) fails the build."""
    bad = {k: v.get("scratch") for k, v in resources.items() if v.get("scratch", 0) != 0}
    if bad:
        raise RuntimeError("kernels with per-lane scratch memory: " +
                           ", ".join(f"{k} ({n} B/lane)" for k, n in sorted(bad.items())))


def build(jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        built = list(ex.map(compile_one, srcs))
    objs = [o for o, _ in built]
    resources = {}
    for _, r in built:
        resources.update(r)
    with open(RESOURCES, "w") as f:
        json.dump(resources, f, indent=1, sort_keys=True)
    check_no_scratch(resources)
    write_build_info()
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    build_static(objs)
    return LIB


BUILD_INFO = os.path.join(HERE, "lib", "build_info.json")


def write_build_info():
    """lib/build_info.json: the git commit of the last change under csrc/ and whether csrc/ differs from it, so
    a run on another machine (which gets the built library without the history) can name what it measured."""
    info = {"csrc_commit": None, "csrc_dirty": None}
    try:
        r = subprocess.run(["git", "-C", ROOT, "log", "-1", "--format=%h", "--", "julia1-rs_amd/csrc"],
                           capture_output=True, text=True, timeout=20)
        if r.returncode == 0 and r.stdout.strip():
            info["csrc_commit"] = r.stdout.strip()
            d = subprocess.run(["git", "-C", ROOT, "status", "--porcelain", "--", "julia1-rs_amd/csrc"],
                               capture_output=True, text=True, timeout=20)
            info["csrc_dirty"] = bool(d.stdout.strip()) if d.returncode == 0 else None
    except (OSError, subprocess.SubprocessError):
        pass
    with open(BUILD_INFO, "w") as f:
        json.dump(info, f)


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
