"""Build libaoakv.so (HIP, gfx950) in-tree with hipcc.

    python aoa-kv_amd/aoakv/_build.py     (a plain script: importing the
                                          package would load the old library)
    python aoa-kv_amd/aoakv/_build.py --timeline
                                          also the profiling build
                                          libaoakv_timeline.so (phase
                                          timestamps, AOAKV_TIMELINE); load it
                                          with AOAKV_LIB for bench.py
                                          --timeline-pass
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import json
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
SRC_DIR = os.path.join(os.path.dirname(PKG_DIR), "csrc")
OBJ_DIR = os.path.join(os.path.dirname(PKG_DIR), "_build")
LIB = os.path.join(PKG_DIR, "libaoakv.so")
TIMELINE_LIB = os.path.join(PKG_DIR, "libaoakv_timeline.so")
# build record beside the library (travels with it; the GPU box has no .git)
BUILDINFO = os.path.join(PKG_DIR, "libaoakv.buildinfo.json")
SOURCES = ["append.hip", "decode.hip", "prefill.hip", "generic.hip", "norm.hip", "capi.cpp"]
REPO_DIR = os.path.dirname(os.path.dirname(PKG_DIR))

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # exact fp16 rounding chains: no multiply-add fusion across rounding points
    "-ffp-contract=off",
    # packed fp32 VALU ops have given wrong results on these boxes
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def _compile(src: str, obj_dir: str = OBJ_DIR, defines=()) -> str:
    obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *[f"-D{d}" for d in defines], "-x", "hip", "-c",
           os.path.join(SRC_DIR, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def source_files() -> list:
    """Every file the library is compiled from (kernels, headers, the C ABI)."""
    out = [os.path.join(SRC_DIR, f) for f in sorted(os.listdir(SRC_DIR))
           if f.endswith((".hip", ".hpp", ".cpp", ".h"))]
    return out + [os.path.join(REPO_DIR, "include", "aoakv.h")]


def source_md5() -> str:
    """md5 over the library's source files (names and contents, in order)."""
    h = hashlib.md5()
    for p in source_files():
        h.update(os.path.basename(p).encode())
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def file_md5(path: str) -> str:
    with open(path, "rb") as f:
        return hashlib.md5(f.read()).hexdigest()


def _git(*args) -> str:
    try:
        r = subprocess.run(["git", "-C", REPO_DIR, *args], capture_output=True, text=True,
                           timeout=10)
        return r.stdout.strip() if r.returncode == 0 else ""
    except (OSError, subprocess.SubprocessError):
        return ""


def write_buildinfo() -> dict:
    """Record what the library was built from: the git HEAD of the tree, whether
    its sources differed from HEAD, the source and library md5s."""
    head = _git("rev-parse", "HEAD") or None
    dirty = bool(_git("status", "--porcelain", "--", "aoa-kv_amd/csrc", "include")) \
        if head else None
    info = {"git_head": head, "sources_differ_from_head": dirty, "src_md5": source_md5(),
            "so_md5": file_md5(LIB), "arch": ARCH}
    with open(BUILDINFO, "w") as f:
        json.dump(info, f, indent=1)
    return info


def _link(lib: str, obj_dir: str, defines=()) -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(obj_dir, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(SRC_DIR, s))]
    with cf.ThreadPoolExecutor(max_workers=min(4, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir, defines), srcs))
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)
    shutil.rmtree(obj_dir, ignore_errors=True)
    return lib


def build(verbose: bool = True, timeline: bool = False) -> str:
    """Compile every source for gfx950 and link libaoakv.so.  Always rebuilds.
    With timeline, also the profiling build libaoakv_timeline.so."""
    _link(LIB, OBJ_DIR)
    write_buildinfo()
    if verbose:
        print(f"built {LIB} ({os.path.getsize(LIB)} bytes)")
    if timeline:
        _link(TIMELINE_LIB, OBJ_DIR + "_timeline", ("AOAKV_TIMELINE",))
        if verbose:
            print(f"built {TIMELINE_LIB} ({os.path.getsize(TIMELINE_LIB)} bytes)")
    return LIB


if __name__ == "__main__":
    build(timeline="--timeline" in sys.argv[1:])
    sys.exit(0)
