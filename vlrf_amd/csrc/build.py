"""Builds vlrf_amd/libvlrf_hip.so for gfx950 with hipcc (cross-compiles on a
host without a GPU).  Objects go to vlrf_amd/_build/, the library next to the
package so that it travels with the source tree.

    python -m vlrf_amd.csrc.build [-j N]
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libvlrf_hip.so")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    # Correctly rounded f32 division and sqrt (bit-exact KV quantization).
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-fast-math",
    # No packed-FP32 instructions in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-pthread"]

HIP_SOURCES = ["api.hip", "model.hip", "kernels/qlinear.hip", "kernels/attention.hip",
               "kernels/elementwise.hip", "kernels/gemm.hip", "kernels/ops.hip", "kernels/qkv_attn.hip"]
CXX_SOURCES = ["host/format.cpp", "host/nfw.cpp"]


def _obj(src):
    return os.path.join(BUILD, src.replace("/", "_") + ".o")


def _compile(src):
    path = os.path.join(HERE, src)
    out = _obj(src)
    if src.endswith(".hip"):
        cmd = [HIPCC, *HIP_FLAGS, "-c", path, "-o", out]
    else:
        cmd = ["g++", *CXX_FLAGS, "-c", path, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    return src, r.returncode, err


def build(jobs=None, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = HIP_SOURCES + CXX_SOURCES
    jobs = jobs or min(len(srcs), os.cpu_count() or 4)
    failed = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        for src, rc, err in ex.map(_compile, srcs):
            if rc != 0:
                failed.append((src, err))
            elif verbose and err.strip():
                print(f"[{src}]\n{err}", file=sys.stderr)
    if failed:
        for src, err in failed:
            print(f"==== {src} failed ====\n{err}", file=sys.stderr)
        raise RuntimeError("vlrf_amd build failed: " + ", ".join(s for s, _ in failed))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", tmp] + [_obj(s) for s in srcs] + ["-pthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("vlrf_amd link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
