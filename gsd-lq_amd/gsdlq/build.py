"""Builds the native libraries in-tree (they travel with the source tree):

  libgsdhip.so  -- HIP kernels + C ABI for gfx950 (hipcc)
  libgsdpack.so -- host encoder / synthetic weights (g++, OpenMP)
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(PKG_DIR, "csrc")
HIP_LIB = os.path.join(PKG_DIR, "libgsdhip.so")
PACK_LIB = os.path.join(PKG_DIR, "libgsdpack.so")
ARCH = os.environ.get("GSD_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
               # packed fp32 VALU ops are disabled for all device code
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               # a single-lane device atomic keeps its own wait: the atomic
               # optimizer would turn it into a wave-wide form whose result
               # is needed (s_waitcnt vmcnt(0)) right after it, ahead of the
               # loads the attention kernels issue behind their arrival
               "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
               "-Wall", "-Wno-unused-function"]
GXX_FLAGS = ["-O2", "-fPIC", "-shared", "-std=c++17", "-fopenmp", "-ffp-contract=off", "-Wall"]


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")


def build_hip(out: str = HIP_LIB) -> str:
    """Each source compiled on its own (in parallel), then linked."""
    import concurrent.futures
    import tempfile
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    tmp = out + ".tmp"
    with tempfile.TemporaryDirectory(prefix="gsdhip_") as d:
        objs = [os.path.join(d, os.path.basename(s) + ".o") for s in srcs]
        with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            list(ex.map(lambda so: _run([_hipcc()] + HIPCC_FLAGS + ["-c", so[0], "-o", so[1]]), zip(srcs, objs)))
        _run([_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}"] + objs + ["-o", tmp])
    os.replace(tmp, out)
    return out


def build_pack(out: str = PACK_LIB) -> str:
    tmp = out + ".tmp"
    _run([shutil.which("g++") or "g++"] + GXX_FLAGS + [os.path.join(CSRC, "gsdpack.cpp"), "-o", tmp])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_pack()
    build_hip()


def hip_sources_newer_than(lib: str = HIP_LIB) -> bool:
    if not os.path.exists(lib):
        return True
    t = os.path.getmtime(lib)
    files = glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.h"))
    return any(os.path.getmtime(f) > t for f in files)
