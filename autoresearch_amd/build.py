"""Build libautoresearch_amd.so (gfx950) and the ar_train driver in-tree.

Usage: python -m autoresearch_amd.build [--jobs N] [--force]

Each csrc/*.hip is compiled with hipcc and each csrc/*.cpp (host-only code)
with g++ to an object under autoresearch_amd/_build/; all are linked into
autoresearch_amd/libautoresearch_amd.so.  host/ar_train.cpp is linked against
it into autoresearch_amd/ar_train (rpath $ORIGIN).  Objects are rebuilt only
when their source or a header is newer.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libautoresearch_amd.so")
HOST = os.path.join(HERE, "host")
TRAIN = os.path.join(HERE, "ar_train")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-result",
    "-munsafe-fp-atomics",
    # Packed-fp32 VALU ops (v_pk_*_f32) are kept out of every kernel: some of
    # their forms have given silently wrong results on this hardware pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _headers():
    return glob.glob(os.path.join(CSRC, "*.hpp")) + glob.glob(os.path.join(ROOT, "include", "*.h"))


def _needs(obj: str, src: str, deps) -> bool:
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return os.path.getmtime(src) > t or any(os.path.getmtime(h) > t for h in deps)


HOST_CFLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{os.path.join(ROOT, 'include')}"]


def _compile(src: str, obj: str) -> str:
    if src.endswith(".cpp"):
        cmd = [CXX, *HOST_CFLAGS, "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {os.path.basename(src)}\n{r.stderr[-6000:]}")
    # The host pass warns that it does not know the packed-fp32 feature: harmless.
    return src


def build(jobs: int = 8, force: bool = False, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    deps = _headers()
    todo = []

    def objname(src):
        return os.path.join(BUILD, os.path.splitext(os.path.basename(src))[0] + ".o")

    for s in srcs:
        obj = objname(s)
        if force or _needs(obj, s, deps):
            todo.append((s, obj))
    if todo:
        with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
            futs = [ex.submit(_compile, s, o) for s, o in todo]
            for f in cf.as_completed(futs):
                src = f.result()
                if verbose:
                    print(f"[build] compiled {os.path.basename(src)}", flush=True)
    objs = [objname(s) for s in srcs]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[build] linked {LIB}", flush=True)
    # the training driver (host code over the C ABI)
    drv = os.path.join(HOST, "ar_train.cpp")
    tmp = TRAIN + ".tmp"
    cmd = [HIPCC, "-O2", "-std=c++17", "-Wall", f"-I{os.path.join(ROOT, 'include')}", drv, "-o", tmp,
           f"-L{HERE}", "-lautoresearch_amd", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"ar_train link failed\n{r.stderr[-4000:]}")
    os.replace(tmp, TRAIN)
    if verbose:
        print(f"[build] linked {TRAIN}", flush=True)
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--force", action="store_true")
    a = ap.parse_args(argv)
    build(a.jobs, a.force)
    return 0


if __name__ == "__main__":
    sys.exit(main())
