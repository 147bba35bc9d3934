"""Build recipe for the dsmoe library: the gfx950 code object (hipcc --genco)
and the host C-ABI library (g++ against the HIP runtime).  Outputs go to
deepseek-rs_amd/lib/.  Run as `python deepseek-rs_amd/build.py`."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
    # packed fp32 ops are kept out of every kernel (see README of the pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_code_object():
    outs = []
    for name in ("dsmoe_kernels", "dsmoe_gemm"):
        out = os.path.join(LIB, name + ".hsaco")
        run([os.path.join(ROCM, "bin", "hipcc"), "--genco", *HIP_FLAGS, "-I", CSRC,
             os.path.join(CSRC, name + ".hip"), "-o", out])
        outs.append(out)
    return outs


def build_host():
    out = os.path.join(LIB, "libdsmoe.so")
    # the static scratch of dsmoe_forward_noalloc: device code inside the library
    obj = os.path.join(LIB, "dsmoe_noalloc.o")
    run([os.path.join(ROCM, "bin", "hipcc"), "-c", "-fPIC", *HIP_FLAGS, os.path.join(CSRC, "dsmoe_noalloc.hip"),
         "-o", obj])
    run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-ffp-contract=off", "-Wall",
         "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"),
         "-I", CSRC, os.path.join(CSRC, "dsmoe_host.cpp"), os.path.join(CSRC, "dsmoe_gguf.cpp"), obj, "-o", out,
         "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib"),
         "-ldl", "-lpthread"])
    return out


def build():
    os.makedirs(LIB, exist_ok=True)
    build_code_object()
    build_host()


if __name__ == "__main__":
    build()
    sys.exit(0)
