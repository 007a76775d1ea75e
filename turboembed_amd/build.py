"""Builds libturbo_rocm.so in place: the gfx950 kernels and the host side.

hipcc cross-compiles for gfx950 without a GPU, so this runs anywhere the
ROCm toolchain is. Objects go to turboembed_amd/_build/, the library next to
this file.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libturbo_rocm.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["rowwise.hip", "gemm.hip", "attention.hip", "session.cpp", "backend.cpp", "checks.cpp", "rerank.cpp",
           "autotune.cpp", "allocs.cpp"]

# The backend's own heap allocations are counted (allocs.cpp): its objects'
# calls of these go to the __wrap_ functions there first.
WRAPPED = ["malloc", "calloc", "realloc", "aligned_alloc", "posix_memalign", "_Znwm", "_Znam",
           "_ZnwmRKSt9nothrow_t", "_ZnamRKSt9nothrow_t", "_ZnwmSt11align_val_t", "_ZnamSt11align_val_t"]

# Per-source device flags. Attention: matrix-core results in ordinary VGPRs,
# so the softmax's vector ops on its accumulators need no copies through the
# accumulation registers; and no NaN operands (its inputs are finite), so a
# max of scores is one v_max3_f32 without a quieting v_max_f32 per score.
EXTRA = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"]}

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    # No packed FP32 instructions in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


# Host-only sources: compiled by the host compiler against the HIP headers.
HOST_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__", "-Wall", "-Wno-unused-function",
    "-I", "/opt/rocm/include", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def _compile(src):
    obj = os.path.join(OUT, src + ".o")
    if src.endswith(".hip"):
        cmd = [HIPCC] + FLAGS + EXTRA.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj]
    else:
        cmd = [os.environ.get("CXX", "g++")] + HOST_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc {src} failed:\n{r.stdout}\n{r.stderr}")
    return obj, r.stderr


def build(verbose=False):
    os.makedirs(OUT, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        results = list(ex.map(_compile, SOURCES))
    if verbose:
        for _, err in results:
            if err.strip():
                print(err)
    objs = [o for o, _ in results]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp] + objs + [f"-Wl,--wrap={w}" for w in WRAPPED]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
