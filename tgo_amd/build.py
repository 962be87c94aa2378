"""Builds libtgohip.so in-tree for gfx950 (hipcc for the HIP sources, g++ for
the host-only mirrors). `python -m tgo_amd.build` or tgo_amd.build.build()."""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libtgohip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_SOURCES = ["runtime.hip", "kernels/attention.hip", "kernels/gemm.hip",
               "kernels/elementwise.hip", "kernels/probe.hip"]
CXX_SOURCES = ["host/hostlogic.cpp", "host/checkpoint.cpp"]

HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall",
             "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-lambda-capture",
             # Packed FP32 VALU ops are kept out of every kernel.
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall"]


def _obj(src):
    return os.path.join(OBJ, src.replace("/", "_") + ".o")


def _compile(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("compile failed: %s\n%s%s" % (" ".join(cmd), r.stdout, r.stderr))
    return r.stderr


def build(verbose=False):
    """Compile every source (always; the driver's build check) and link."""
    os.makedirs(OBJ, exist_ok=True)
    jobs = []
    for s in HIP_SOURCES:
        jobs.append([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, s), "-o", _obj(s)])
    for s in CXX_SOURCES:
        jobs.append(["g++"] + CXX_FLAGS + ["-c", os.path.join(CSRC, s), "-o", _obj(s)])
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for err in ex.map(_compile, jobs):
            if verbose and err:
                sys.stderr.write(err)
    objs = [_obj(s) for s in HIP_SOURCES + CXX_SOURCES]
    tmp = LIB + ".tmp"
    _compile([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
