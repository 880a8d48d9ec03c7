"""Test infrastructure: compile the reference's CPU kernels into oracle/_ref/.

The sources are compiled where they lie under the reference checkout (never
copied); outputs go only to oracle/_ref/ (git-ignored).  Flags follow the
reference's CPU build (setup.py:33,46: -O3 -std=c++20 -fopenmp, no -march).
The product never loads the result; see oracle/ref_shim.cpp.

Usage: python oracle/build_ref.py [--ref /root/reference] [-j 8]
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_ref")
LIB = os.path.join(OUT, "libtp_ref.so")
SOURCES = [
    "csrc/cpu/2d/projection_2d_kernels.cpp",
    "csrc/cpu/2d/backprojection_2d_kernels.cpp",
    "csrc/cpu/3d/projection_3d_to_2d_kernels.cpp",
    "csrc/cpu/3d/backprojection_2d_to_3d_kernels.cpp",
]


def flags():
    import torch
    from torch.utils import cpp_extension as ce
    import sysconfig
    inc = ["-isystem", sysconfig.get_paths()["include"]]
    for p in ce.include_paths():
        inc += ["-isystem", p]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return inc, ["-O3", "-std=c++20", "-fopenmp", "-fPIC", "-w",
                 f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_API_INCLUDE_EXTENSION_H",
                 "-DTORCH_EXTENSION_NAME=tp_ref"], ce.library_paths()


def build(ref, jobs=8, quiet=False):
    if not os.path.isdir(os.path.join(ref, "csrc", "cpu")):
        raise FileNotFoundError(f"reference sources not found under {ref}")
    os.makedirs(OUT, exist_ok=True)
    inc, cflags, libdirs = flags()
    jobs_list = [(os.path.join(ref, s), os.path.join(OUT, os.path.basename(s) + ".o"), []) for s in SOURCES]
    jobs_list.append((os.path.join(HERE, "ref_shim.cpp"), os.path.join(OUT, "ref_shim.o"),
                      ["-I", os.path.join(ref, "csrc")]))

    def compile_one(job):
        src, obj, extra = job
        if os.path.exists(obj) and os.path.getmtime(obj) > os.path.getmtime(src):
            return obj
        cmd = ["g++", *cflags, *inc, *extra, "-c", src, "-o", obj]
        subprocess.run(cmd, check=True)
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, jobs_list))
    link = ["g++", "-shared", "-fopenmp", *objs, "-o", LIB]
    for d in libdirs:
        link += [f"-L{d}", f"-Wl,-rpath,{d}"]
    link += ["-lc10", "-ltorch_cpu", "-ltorch"]
    subprocess.run(link, check=True)
    if not quiet:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args()
    build(a.ref, a.j)
