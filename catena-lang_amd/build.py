"""Build libcatena_mi355x: gfx950 code objects + the host C-ABI library.

Kernels (csrc/kernels/*.hip) are compiled for gfx950 only into raw code
objects (lib/<name>.co) that the host library loads with hipModuleLoad.
Flags keep the reference's arithmetic contract (no FMA contraction, no
fast-math: catena-lang/src/runtime/artifact.rs:59-71) and disable packed
fp32 instruction selection.  The host side (csrc/host/*.cpp) is plain C++17
compiled with g++ against the HIP runtime.

Usage: python catena-lang_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
KDIR = os.path.join(HERE, "csrc", "kernels")
HDIR = os.path.join(HERE, "csrc", "host")
OUT = os.path.join(HERE, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

KERNEL_FLAGS = [
    "-x", "hip", "--offload-arch=gfx950", "--offload-device-only", "--no-gpu-bundle-output",
    "-O3", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]
HOST_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter",
    "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{os.path.join(ROOT, 'include')}",
]
HOST_LIBS = [f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-ldl", "-pthread"]

LIB_NAME = "libcatena_mi355x.so"


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "not a recognized feature" not in l
                    and "is not a recognized feature for this target" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build_kernel(src: str) -> str:
    name = os.path.splitext(os.path.basename(src))[0]
    out = os.path.join(OUT, name + ".co")
    tmp = out + ".tmp"
    _run([HIPCC, *KERNEL_FLAGS, "-c", src, "-o", tmp])
    os.replace(tmp, out)
    return out


# Host-side HIP sources (csrc/host/*.hip) hold device globals the library
# addresses from the host (hipGetSymbolAddress): compiled by hipcc for the
# host and gfx950 into one object each, then linked into the library.
HOST_HIP_FLAGS = [
    "-x", "hip", "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", f"-I{os.path.join(ROOT, 'include')}",
]


def build_host() -> str:
    srcs = sorted(glob.glob(os.path.join(HDIR, "*.cpp")))
    objs = []
    os.makedirs(os.path.join(OUT, "obj"), exist_ok=True)
    for hs in sorted(glob.glob(os.path.join(HDIR, "*.hip"))):
        obj = os.path.join(OUT, "obj", os.path.splitext(os.path.basename(hs))[0] + ".o")
        _run([HIPCC, *HOST_HIP_FLAGS, "-c", hs, "-o", obj])
        objs.append(obj)
    out = os.path.join(OUT, LIB_NAME)
    tmp = out + ".tmp"
    cxx = os.environ.get("CXX", "g++")
    _run([cxx, *HOST_FLAGS, *srcs, *objs, "-o", tmp, *HOST_LIBS])
    os.replace(tmp, out)
    return out


def build(jobs: int = 8) -> list[str]:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(OUT, exist_ok=True)
    # The library goes first and comes back only when everything built: the
    # host passes structs by value that the kernels read with their own
    # layout, so an old library beside new code objects (or the reverse)
    # must never be loadable.
    lib = os.path.join(OUT, LIB_NAME)
    if os.path.exists(lib):
        os.remove(lib)
    srcs = sorted(glob.glob(os.path.join(KDIR, "*.hip")))
    # code objects whose source is gone would otherwise linger in lib/
    live = {os.path.splitext(os.path.basename(s))[0] for s in srcs}
    for co in glob.glob(os.path.join(OUT, "*.co")):
        if os.path.splitext(os.path.basename(co))[0] not in live:
            os.remove(co)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(build_kernel, s) for s in srcs]
        futs.append(ex.submit(build_host))
        try:
            return [f.result() for f in futs]
        except Exception:
            for f in futs:
                f.exception()  # wait for the rest before removing anything
            if os.path.exists(lib):
                os.remove(lib)
            raise


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    args = ap.parse_args(argv)
    for p in build(args.jobs):
        print(os.path.relpath(p, ROOT))
    return 0


if __name__ == "__main__":
    sys.exit(main())
