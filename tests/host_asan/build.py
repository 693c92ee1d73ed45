"""Build recipe of the host-sanitizer check of the C-ABI (test infrastructure).

Every ``csrc/*.hip`` is compiled with AddressSanitizer and UBSan on its host
code only (``-Xarch_host`` before each ``-fsanitize=``; the gfx950 device code
is built as in the product), the driver ``abi_host_check.cpp`` with g++ on a
line of its own, and all of it linked by g++ against the HIP runtime into
``tests/host_asan/_build/abi_host_check``.  The executable carries the
sanitizer runtimes itself, so it runs with no preloading.

Usage: ``python tests/host_asan/build.py`` or ``build()`` (called by
``__graft_entry__.build``).
"""
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "ojasx-vector-24x96_amd", "csrc")
OUT = os.path.join(HERE, "_build")
EXE = os.path.join(OUT, "abi_host_check")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", os.path.join(ROCM, "bin", "hipcc"))
ARCH = os.environ.get("OJASX_OFFLOAD_ARCH", "gfx950")

HOST_SAN = ["-Xarch_host", "-fsanitize=address,undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer"]
HIP_FLAGS = [f"--offload-arch={ARCH}", "-O1", "-g", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-command-line-argument",
             "-I", os.path.join(ROOT, "include"), "-I", CSRC, *HOST_SAN]
GXX_SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{' '.join(cmd[:3])} ... failed:\n{r.stderr[-6000:]}")


def _compile_hip(src):
    obj = os.path.join(OUT, os.path.basename(src) + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
    return obj


def build(verbose=True):
    os.makedirs(OUT, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile_hip, srcs))
    drv = os.path.join(OUT, "abi_host_check.o")
    _run(["g++", "-std=c++17", "-O1", "-g", *GXX_SAN, "-D__HIP_PLATFORM_AMD__",
          "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"),
          "-c", os.path.join(HERE, "abi_host_check.cpp"), "-o", drv])
    _run(["g++", *GXX_SAN, drv, *objs, "-o", EXE + ".tmp",
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib"),
          "-lpthread"])
    os.replace(EXE + ".tmp", EXE)
    if verbose:
        print(f"built {EXE}")
    return EXE


if __name__ == "__main__":
    build()
    sys.exit(0)
