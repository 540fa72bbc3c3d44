"""Build the gfx950 libraries in-tree with hipcc (no CMake, no JIT cache).

    python -m llmengine_amd.build          # or llmengine_amd.build.build_all()

Outputs (git-ignored, shipped to the GPU box with the tree):
  llmengine_amd/libmle_q8_0.so      C ABI + hand-written HIP kernels (include/mle_q8_0.h)
  llmengine_amd/libminillm_hip.so   C++ host runtime mirroring the reference's graph /
                                    registry / executor API, with HipBackend/HipExecutor
  tests/cpp/bin/*                   C++ test executables (reference-style asserts)

All HIP code is compiled for gfx950 only, with packed-fp32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
BUILD = os.path.join(PKG, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

KERNEL_LIB = os.path.join(PKG, "libmle_q8_0.so")
HOST_LIB = os.path.join(PKG, "libminillm_hip.so")


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _compile(src, obj, flags):
    os.makedirs(os.path.dirname(obj), exist_ok=True)
    _run([HIPCC, *flags, "-c", src, "-o", obj])
    return obj


def _link_atomic(objs, out, extra):
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp, *extra])
    os.replace(tmp, out)


def build_kernels(jobs: int = 8) -> str:
    srcs = sorted(glob.glob(os.path.join(PKG, "csrc", "kernels", "*.hip")))
    srcs.append(os.path.join(PKG, "csrc", "capi.hip"))
    objs = [os.path.join(BUILD, "kernels", os.path.basename(s) + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], HIP_FLAGS), zip(srcs, objs)))
    _link_atomic(objs, KERNEL_LIB, [])
    return KERNEL_LIB


def build_host(jobs: int = 8) -> str | None:
    srcs = sorted(glob.glob(os.path.join(PKG, "csrc", "host", "*.cpp")))
    if not srcs:
        return None
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG, "csrc", "host")]
    objs = [os.path.join(BUILD, "host", os.path.basename(s) + ".o") for s in srcs]
    flags = HIP_FLAGS + inc + ["-x", "hip"]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], flags), zip(srcs, objs)))
    _link_atomic(objs, HOST_LIB, ["-L", PKG, "-lmle_q8_0", "-Wl,-rpath,$ORIGIN"])
    return HOST_LIB


def build_cpp_tests(jobs: int = 8) -> list[str]:
    srcs = sorted(glob.glob(os.path.join(ROOT, "tests", "cpp", "*.cpp")))
    bindir = os.path.join(ROOT, "tests", "cpp", "bin")
    os.makedirs(bindir, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG, "csrc", "host")]

    def one(src):
        exe = os.path.join(bindir, os.path.splitext(os.path.basename(src))[0])
        tmp = exe + ".tmp"
        _run([HIPCC, *HIP_FLAGS, "-UNDEBUG", *inc, "-x", "hip", src, "-o", tmp,
              "-L", PKG, "-lminillm_hip", "-lmle_q8_0",
              "-Wl,-rpath,$ORIGIN/../../../llmengine_amd"])
        os.replace(tmp, exe)
        return exe

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        return list(ex.map(one, srcs))


def build_all(jobs: int = 8) -> None:
    build_kernels(jobs)
    if build_host(jobs):
        build_cpp_tests(jobs)


if __name__ == "__main__":
    build_all(int(sys.argv[1]) if len(sys.argv) > 1 else 8)
    print("built", KERNEL_LIB)
