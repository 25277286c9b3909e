"""Builds the gfx950 backend library in-tree: tensor-adapt_amd/libtadapt.so.

Every .hip under csrc/ is compiled with hipcc for gfx950 only (no other
targets, no CUDA path) and every .cpp (host-only C++: the C++ host API over
the C-ABI) with the host compiler, in parallel, then linked into one shared
library whose exported symbols are the C-ABI of include/ta_backend.h and
include/ta_engine.h plus the C++ API of include/tensor/.  Object files go to
csrc/_build/ (git-ignored).
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libtadapt.so")
BUILD = os.path.join(CSRC, "_build")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: packed F32 VALU forms are avoided on this pool.
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
         "-Wno-unused-function", "-Wno-unused-variable",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I" + CSRC, "-I" + INCLUDE]


CXX = os.environ.get("CXX", "g++")
CXXFLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__",
            "-I/opt/rocm/include", "-I" + CSRC, "-I" + INCLUDE]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith(".hip") or f.endswith(".cpp"))


def _compile(src):
    base, ext = os.path.splitext(os.path.basename(src))
    obj = os.path.join(BUILD, base + (".o" if ext == ".hip" else ".cpp.o"))
    if ext == ".hip":
        cmd = [HIPCC] + FLAGS + ["-c", src, "-o", obj]
    else:
        cmd = [CXX] + CXXFLAGS + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass warns that it does not know the packed-fp32 feature: harmless
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    return src, obj, r.returncode, err


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    objs = []
    failed = False
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for src, obj, rc, err in ex.map(_compile, srcs):
            if err.strip() and (verbose or rc):
                print(err, file=sys.stderr)
            if rc != 0:
                failed = True
                print("hipcc failed: " + src, file=sys.stderr)
            objs.append(obj)
    if failed:
        raise RuntimeError("HIP compilation failed")
    tmp = OUT + ".tmp"
    # -z defs: a symbol left undefined fails the link instead of the first load
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp] + objs
    subprocess.check_call(cmd)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
