"""Register, scratch and LDS budgets of the tile-owner kernels (CPU: the compiler's report).

The build keeps hipcc's per-kernel resource report (`-Rpass-analysis=kernel-resource-usage`) beside
each object (torch-projectors_amd/build.py); when it is missing or older than the sources, the
tiled sources are compiled here for it. Three budgets are checked:

* LDS is allocated in 1280-byte granules on gfx950 (160 KB per CU = 128 granules): a 256-lane
  workgroup of at most 40960 bytes runs four per CU, of at most 53760 bytes three. The compiler's
  occupancy estimate does not round that way (it counts three workgroups for up to 54272 bytes),
  and a kernel between the two lines ran at two: every tiled kernel's granule-rounded LDS times the
  workgroups per CU the compiler assumes must fit in 160 KB.
* The kernels of the measured workloads keep their registers without spills (scratch 0).
* The headline forward and backprojection keep four workgroups (16 waves) per CU.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "torch-projectors_amd")
HIP = os.path.join(PKG, "csrc", "hip")
BUILD = os.path.join(PKG, "_build")
SOURCES = ("tp_tiled3d.hip", "tp_tiled2d.hip")
LDS_PER_CU, GRANULE = 163840, 1280

# (mangled-name fragment, what it runs)
SPILL_FREE = {
    "16k_scatter3_tiledILb0ELi0ELb1ELi6ELb1ELb0E": "headline backprojection",
    "13k_forw3_tiledILb0ELi5ELb1ELi0ELb1ELb0EfLb0E": "headline forward",
    "16k_scatter3_tiledILb1ELi1ELb0ELi4ELb1ELb0E": "c4 reconstruction gradient (cubic)",
    "16k_scatter3_tiledILb1ELi0ELb1ELi4ELb1ELb0E": "cubic backprojection",
    "13k_forw3_tiledILb1ELi5ELb1ELi0ELb1ELb0EfLb0E": "cubic forward",
    "13k_forw3_tiledILb1ELi2ELb1ELi1ELb1ELb0EfLb0E": "c4 rotation/shift gradients",
    "13k_forw3_tiledILb0ELi2ELb1ELi2ELb1ELb1EfLb0E": "linear backprojection backward",
}
FOUR_PER_CU = ("16k_scatter3_tiledILb0ELi0ELb1ELi6ELb1ELb0E", "13k_forw3_tiledILb0ELi5ELb1ELi0ELb1ELb0EfLb0E")


def _newest_source_mtime():
    return max(os.path.getmtime(os.path.join(HIP, f)) for f in os.listdir(HIP)
               if f.endswith((".hip", ".hh", ".h")))


def _report(src):
    """The resource report of `src`: the build's, or a fresh compile when it is stale."""
    path = os.path.join(BUILD, src + ".resources.txt")
    if os.path.exists(path) and os.path.getmtime(path) >= _newest_source_mtime():
        return open(path).read()
    hipcc = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available and no build report")
    import importlib.util
    spec = importlib.util.spec_from_file_location("tp_build", os.path.join(PKG, "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    r = subprocess.run([hipcc, *b.KERNEL_FLAGS, "--offload-device-only", "-Rpass-analysis=kernel-resource-usage",
                        "-c", os.path.join(HIP, src), "-o", os.devnull], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stderr


def _kernels(text):
    """{mangled name: {VGPRs, ScratchSize, Occupancy, LDS}} of the device functions in a report."""
    out, cur = {}, None
    for line in text.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        if cur is None:
            continue
        for key, pat in (("VGPRs", r"\bVGPRs: (\d+)"), ("ScratchSize", r"ScratchSize \[bytes/lane\]: (\d+)"),
                         ("Occupancy", r"Occupancy \[waves/SIMD\]: (\d+)"), ("LDS", r"LDS Size \[bytes/block\]: (\d+)")):
            m = re.search(pat, line)
            if m and key not in cur:
                cur[key] = int(m.group(1))
    return {k: v for k, v in out.items() if "_tiled" in k and "Occupancy" in v and "LDS" in v}


@pytest.fixture(scope="module")
def kernels():
    ks = {}
    for src in SOURCES:
        ks.update(_kernels(_report(src)))
    assert ks, "no tiled kernels in the resource reports"
    return ks


def test_lds_granules_allow_the_assumed_occupancy(kernels):
    bad = []
    for name, k in kernels.items():
        granular = -(-k["LDS"] // GRANULE) * GRANULE
        # 256-lane workgroups: one wave per SIMD each, so waves/SIMD = workgroups per CU
        if granular * k["Occupancy"] > LDS_PER_CU:
            bad.append(f"{name}: {k['LDS']} B of LDS ({granular} in granules) x {k['Occupancy']} per CU")
    assert not bad, "\n".join(bad)


@pytest.mark.parametrize("frag", sorted(SPILL_FREE), ids=lambda f: SPILL_FREE[f].replace(" ", "_"))
def test_measured_kernels_are_spill_free(kernels, frag):
    hits = [(n, k) for n, k in kernels.items() if frag in n]
    assert hits, f"kernel {SPILL_FREE[frag]} ({frag}) not in the report"
    for n, k in hits:
        assert k["ScratchSize"] == 0, f"{SPILL_FREE[frag]}: {k['ScratchSize']} bytes/lane of scratch ({n})"


@pytest.mark.parametrize("frag", FOUR_PER_CU, ids=("headline_backprojection", "headline_forward"))
def test_headline_kernels_keep_four_workgroups_per_cu(kernels, frag):
    (n, k), = [(n, k) for n, k in kernels.items() if frag in n]
    granular = -(-k["LDS"] // GRANULE) * GRANULE
    assert k["Occupancy"] >= 4 and 4 * granular <= LDS_PER_CU, (n, k)
