"""Build libubridge_hip.so for gfx950 in-tree (ubridge_amd/lib/).

Every HIP/C++ source under ubridge_amd/csrc is compiled with hipcc in
parallel and linked into one shared library whose exported symbols are the
extern "C" entry points declared in include/ubridge_hip.h; then the C++ host
driver (driver/ub_drive.cpp) is linked against it as lib/ub_drive.

    python ubridge_amd/build.py
"""
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libubridge_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting packed FP32 VALU ops
# (the host pass warns that it does not know the feature; harmless).
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def _compile(src):
    base = os.path.splitext(os.path.basename(src))[0]
    obj = os.path.join(OBJ, base + ".o")
    cmd = [HIPCC, *FLAGS, "-I", CSRC, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    return obj, err


def build(verbose=False, jobs=None):
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_compile, srcs))
    for _, err in results:
        if verbose and err.strip():
            print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lhipblaslt"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    _build_driver()
    return LIB


DRIVER_SRC = os.path.join(HERE, "driver", "ub_drive.cpp")
DRIVER = os.path.join(LIBDIR, "ub_drive")


def _build_driver():
    """The C++ host driver (driver/ub_drive.cpp): a program over the C ABI
    only, linked against the library next to it."""
    inc = os.path.join(os.path.dirname(HERE), "include")
    tmp = DRIVER + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-Wall",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", inc, DRIVER_SRC,
           "-o", tmp, "-L", LIBDIR, "-lubridge_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("driver build failed:\n" + r.stderr)
    os.replace(tmp, DRIVER)


if __name__ == "__main__":
    print(build(verbose=True))
