"""Build libzkh.so (the C-ABI library) for gfx950 with hipcc, in-tree.

Compiles csrc/*.hip to objects in parallel and links one shared library next to this
file, then the zkob_*-compatible drivers `zkh_fc`, `zkh_rescale`, `zkh_glu` and `zkh_rope` (cli/*.cpp, host C++
against it).  Flags: -O3, C++17, gfx950 only, packed FP32 disabled (the field arithmetic is
integer-only; the flag keeps hipcc from forming packed fp32 ops anywhere).
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libzkh.so")
CLIS = ("zkh_fc", "zkh_rescale", "zkh_glu", "zkh_rope", "zkh_batchopen")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
SOURCES = ["kernels.hip", "g1.hip", "zkh.hip"]


def _compile(src):
    obj = os.path.join(OBJ, src.replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (src, msgs))
    return obj, msgs


def build(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        results = list(ex.map(_compile, SOURCES))
    for _, msgs in results:
        if msgs.strip() and verbose:
            print(msgs, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    # the zkob_*-compatible drivers (host C++ over the C ABI)
    for name in CLIS:
        out = os.path.join(HERE, name)
        cmd = ["g++", "-O2", "-std=c++17", "-Wall", os.path.join(HERE, "cli", name + ".cpp"), "-o", out + ".tmp",
               "-L" + HERE, "-lzkh", "-Wl,-rpath,$ORIGIN"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("%s build failed:\n%s%s" % (name, r.stdout, r.stderr))
        os.replace(out + ".tmp", out)
    return LIB


if __name__ == "__main__":
    print(build())
