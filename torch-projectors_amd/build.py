"""Build the MI355X projector library in-tree.

Outputs (both inside torch_projectors/, so they travel with the tree):

  libtorch_projectors_hip.so  the HIP kernels + the C ABI of
                              include/torch_projectors_hip.h (hipcc, gfx950)
  _C.so                       the PyTorch dispatcher registration
                              (csrc/torch_projectors.cpp), linked against the
                              library above with an $ORIGIN rpath

Kernel flags: -O3, no fast-math, -ffp-contract=off (sample coordinates and
stencil weights must round exactly like the reference CPU code), and packed
FP32 instructions disabled.

Usage: python torch-projectors_amd/build.py [-j N] [--only-lib]
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(HERE, "torch_projectors")
BUILD = os.path.join(HERE, "_build")
HIP_SRC = os.path.join(HERE, "csrc", "hip")
LIB = os.path.join(PKG, "libtorch_projectors_hip.so")
EXT = os.path.join(PKG, "_C.so")

ARCH = os.environ.get("TP_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

KERNEL_FLAGS = [
    "-O3", f"--offload-arch={ARCH}", "-fPIC", "-std=c++17",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"),
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + r.stdout)
    return r.stdout


def hip_sources():
    return sorted(os.path.join(HIP_SRC, f) for f in os.listdir(HIP_SRC) if f.endswith(".hip"))


def build_lib(jobs=8):
    os.makedirs(BUILD, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        # the compiler's per-kernel register / scratch / LDS / occupancy report, kept beside the
        # object (tests/test_kernel_resources_cpu.py checks the budgets of the tiled kernels)
        out = _run([HIPCC, *KERNEL_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", obj])
        with open(os.path.join(BUILD, os.path.basename(src) + ".resources.txt"), "w") as f:
            f.write(out)
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, hip_sources()))
    tmp = LIB + ".tmp"
    rocm_lib = os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(HIPCC))), "lib")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
          f"-L{rocm_lib}", f"-Wl,-rpath,{rocm_lib}", "-lhipfft"])
    os.replace(tmp, LIB)
    return LIB


def _torch_flags():
    import torch
    from torch.utils import cpp_extension as ce
    inc = []
    for p in ce.include_paths():
        inc += ["-isystem", p]
    inc += ["-isystem", sysconfig.get_paths()["include"]]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    defs = [f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
            "-DTORCH_EXTENSION_NAME=_C"]
    libs = []
    for d in ce.library_paths():
        libs += [f"-L{d}", f"-Wl,-rpath,{d}"]
    libs += ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip"]
    return inc, defs, libs


def build_ext():
    inc, defs, libs = _torch_flags()
    src = os.path.join(HERE, "csrc", "torch_projectors.cpp")
    tmp = EXT + ".tmp"
    _run([HIPCC, "-O2", "-fPIC", "-std=c++17", "-shared", "-w", *defs, *inc, src, "-o", tmp,
          f"-L{PKG}", "-ltorch_projectors_hip", "-Wl,-rpath,$ORIGIN", *libs])
    os.replace(tmp, EXT)
    return EXT


def build(jobs=8, only_lib=False, quiet=False):
    out = [build_lib(jobs)]
    if not only_lib:
        out.append(build_ext())
    if not quiet:
        for p in out:
            print("built", os.path.relpath(p, ROOT))
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    ap.add_argument("--only-lib", action="store_true")
    a = ap.parse_args()
    try:
        build(a.j, a.only_lib)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
