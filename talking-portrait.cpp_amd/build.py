"""Build libtpmd.so (HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

    python talking-portrait.cpp_amd/build.py

Every translation unit is compiled to an object under _build/ in parallel,
then linked into talking-portrait.cpp_amd/libtpmd.so.  HIP code is compiled
with packed-FP32 instructions disabled (-packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOSTDIR = os.path.join(PKG, "host")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libtpmd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
          f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}", f"-I{HOSTDIR}"]
HIP_FLAGS = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-munsafe-fp-atomics"]

SOURCES = ["k_gather.hip", "k_conv.hip", "k_conv_async.hip", "k_conv_hfrag.hip", "k_conv_hfrag8.hip", "k_conv_hfrag16.hip", "k_conv_hfrag_tail.hip", "k_conv_fused.hip", "k_conv_up.hip", "k_conv_halo.hip", "k_tail.hip", "k_style.hip", "k_enc.hip", "k_fmt.hip", "k_probe.hip", "tpmd.cpp", "tpme.cpp", "tpfm.cpp"]
# plain C++ over the C ABI (no HIP): the tp::motion_dec shim, in the library
# hipBLASLt: the FMT's f16 linear products (tpfm.cpp)
LINK_LIBS = ["-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]
HOST_SOURCES = ["motion_dec.cpp", "motion_enc.cpp", "gguf.cpp", "gguf_abi.cpp"]
CXX = os.environ.get("CXX", "g++")
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{os.path.join(ROOT, 'include')}", f"-I{HOSTDIR}"]
SHIM_CHECK = os.path.join(PKG, "shim_check")


def _run(cmd):
    p = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (p.stdout + p.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + out)
    return out


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    for s in SOURCES:
        src = os.path.join(CSRC, s)
        obj = os.path.join(BUILD, s + ".o")
        # .cpp files hold host code only; hipcc compiles them as HIP so the
        # runtime headers resolve, and the device pass is empty
        jobs.append([HIPCC, *COMMON, *HIP_FLAGS, "-x", "hip", "-c", src, "-o", obj])
    for s in HOST_SOURCES:
        src = os.path.join(HOSTDIR, s)
        obj = os.path.join(BUILD, "host_" + s + ".o")
        jobs.append([CXX, *HOST_FLAGS, "-c", src, "-o", obj])
    objs = [j[-1] for j in jobs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, *LINK_LIBS])
    os.replace(tmp, LIB)
    # the shim's driver, linked against the library next to it
    tmp = SHIM_CHECK + ".tmp"
    _run([CXX, *HOST_FLAGS, os.path.join(HOSTDIR, "shim_check.cpp"), "-o", tmp, f"-L{PKG}", "-ltpmd",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, SHIM_CHECK)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
