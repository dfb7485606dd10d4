"""Build libsam3hip.so (gfx950 only) in this directory.

hipcc compiles each HIP kernel file for --offload-arch=gfx950; gcc
compiles the C host layer against the HIP runtime API; hipcc links the
shared library. Always rebuilds. Run as `python build.py` or call
build().
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJ = os.path.join(HERE, "_obj")
LIB = os.path.join(HERE, "libsam3hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
    # Packed fp32 VALU instructions are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
# MFMA accumulators in VGPRs: no AGPR <-> VGPR copies around the VALU work
# on scores and outputs. Not for the NT GEMM, whose 128 x 128 wave tiles
# keep 256 accumulators per lane in the AGPRs.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
AGPR_FILES = {"k_gemm_nt.hip"}
C_FLAGS = ["-O2", "-fPIC", "-std=gnu11", "-Wall", "-Wextra",
           "-Wno-unused-parameter", "-D__HIP_PLATFORM_AMD__"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    out = "\n".join(line for line in r.stdout.splitlines()
                    if "is not a recognized feature for this target" not in line)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    inc = ["-I" + INCLUDE, "-I" + CSRC, "-I" + os.path.join(ROCM, "include")]
    jobs = []
    objs = []
    for f in sorted(os.listdir(CSRC)):
        src = os.path.join(CSRC, f)
        obj = os.path.join(OBJ, os.path.splitext(f)[0] + ".o")
        if f.endswith(".hip"):
            flags = HIP_FLAGS + ([] if f in AGPR_FILES else VGPR_FORM)
            jobs.append([os.path.join(ROCM, "bin", "hipcc")] + flags + inc +
                        ["-c", src, "-o", obj])
        elif f.endswith(".c"):
            jobs.append(["gcc"] + C_FLAGS + inc + ["-c", src, "-o", obj])
        else:
            continue
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        outs = list(ex.map(_run, jobs))
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
    tmp = LIB + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), "--offload-arch=gfx950",
          "-shared", "-fPIC", "-o", tmp] + objs +
         ["-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-lpthread",
          "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
