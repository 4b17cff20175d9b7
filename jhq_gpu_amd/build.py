"""Build recipes for the HIP engine (libjhq_amd.so) and the C oracle.

The engine is compiled for gfx950 only.  Every HIP translation unit gets
-ffp-contract=off (the kernels place each fused multiply-add explicitly) and
-Xclang -target-feature -Xclang -packed-fp32-ops (no packed FP32 VALU ops).
"""
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libjhq_amd.so")
ORACLE = os.path.join(ROOT, "oracle")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "-O3", "--offload-arch=gfx950", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-pthread"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError("build step failed: " + " ".join(cmd))
    return r.stdout


def build_engine(verbose=False):
    """Compile kernels.hip, jhq_capi.hip, kmeans.hip, noalloc.hip, assign_mfma.hip and
    host_train.cpp into libjhq_amd.so."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = [
        ([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, "kernels.hip"),
                                "-o", os.path.join(BUILD, "kernels.o")]),
        ([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, "jhq_capi.hip"),
                                "-o", os.path.join(BUILD, "jhq_capi.o")]),
        ([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, "kmeans.hip"),
                                "-o", os.path.join(BUILD, "kmeans.o")]),
        ([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, "noalloc.hip"),
                                "-o", os.path.join(BUILD, "noalloc.o")]),
        ([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, "assign_mfma.hip"),
                                "-o", os.path.join(BUILD, "assign_mfma.o")]),
        (["g++"] + CXX_FLAGS + ["-c", os.path.join(CSRC, "host_train.cpp"),
                                "-o", os.path.join(BUILD, "host_train.o")]),
    ]
    procs = [subprocess.Popen(j, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
             for j in jobs]
    failed = False
    for j, p in zip(jobs, procs):
        out, _ = p.communicate()
        if p.returncode != 0:
            sys.stderr.write(out)
            failed = True
        elif verbose and out.strip():
            sys.stderr.write(out)
    if failed:
        raise RuntimeError("HIP engine compilation failed")
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-pthread", "-o", tmp,
          os.path.join(BUILD, "kernels.o"), os.path.join(BUILD, "jhq_capi.o"),
          os.path.join(BUILD, "kmeans.o"), os.path.join(BUILD, "noalloc.o"),
          os.path.join(BUILD, "assign_mfma.o"), os.path.join(BUILD, "host_train.o")])
    os.replace(tmp, LIB)
    return LIB


def build_oracle(with_ref=None):
    """Compile the C oracle; also oracle/_ref when the reference checkout exists."""
    _run(["make", "-C", ORACLE, "-s", "all"])
    if with_ref is None:
        with_ref = os.path.isdir("/root/reference/cpu")
    if with_ref:
        _run(["make", "-C", ORACLE, "-s", "ref"])


if __name__ == "__main__":
    build_engine(verbose=True)
    build_oracle()
    print(LIB)
