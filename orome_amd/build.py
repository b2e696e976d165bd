"""Build recipe for liborome_moe.so (gfx950).

C sources are compiled with gcc, HIP sources with hipcc for gfx950 only, and
everything is linked by hipcc into orome_amd/liborome_moe.so (in-tree, so the
library travels with the source tree).  Run `python orome_amd/build.py` (a plain script: it must not import the
package, whose import loads the library it builds).
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liborome_moe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

C_SOURCES = ["gguf.c", "format.c", "synth.c"]
HIP_SOURCES = ["host.hip", "moe_route.hip", "moe_gemv.hip", "moe_gemm.hip", "moe_misc.hip"]
INCLUDES = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
# Packed FP32 instructions are disabled for all device code.
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall",
             "-Wno-unused-function", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-fvisibility=hidden"]
C_FLAGS = ["-O2", "-fPIC", "-std=c11", "-Wall", "-fopenmp", "-fvisibility=hidden",
           "-D_GNU_SOURCE"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    for s in C_SOURCES:
        o = os.path.join(BUILD, s + ".o")
        jobs.append(["gcc", *C_FLAGS, *INCLUDES, "-c", os.path.join(CSRC, s), "-o", o])
    for s in HIP_SOURCES:
        o = os.path.join(BUILD, s + ".o")
        jobs.append([HIPCC, *HIP_FLAGS, *INCLUDES, "-c", os.path.join(CSRC, s), "-o", o])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    objs = [os.path.join(BUILD, s + ".o") for s in C_SOURCES + HIP_SOURCES]
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs, "-fopenmp", "-lm"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
