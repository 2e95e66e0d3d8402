"""Builds libpadra_hip.so in-tree for gfx950 (python -m padra_amd.build).

One hipcc invocation over every source in padra_amd/csrc.  Flags:
  -ffp-contract=off  every float op rounds once, as the reference's __f*_rn intrinsics;
  -Xclang -target-feature -Xclang -packed-fp32-ops  no packed-FP32 instructions;
  -mllvm -amdgpu-mfma-vgpr-form  MFMA accumulators in VGPRs (the attention kernels rescale
      theirs with ordinary VALU multiplies, which AGPR accumulators would route through
      accvgpr moves; 2-4% faster there, no effect on kernels without MFMA).
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = ["csrc/kernels.hip", "csrc/kv_codec.hip", "csrc/swiglu_embed.hip", "csrc/combine.hip",
           "csrc/attention.hip", "csrc/rope_table.cpp"]
OUT = os.path.join(HERE, "libpadra_hip.so")


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


# The host-sanitizer build: the library's host code (argument checks, launch set-up, the
# RoPE table builder) under AddressSanitizer and UndefinedBehaviorSanitizer; device code
# is compiled as usual (no GPU sanitizer).  The CPU tests run against it with the clang
# ASan runtime preloaded (python is not instrumented):
#   python -m padra_amd.build --asan
#   PADRA_HIP_LIB=padra_amd/_asan/libpadra_hip.so ASAN_OPTIONS=detect_leaks=0 \
#     LD_PRELOAD=$(hipcc -print-file-name=libclang_rt.asan-x86_64.so) \
#     python -m pytest tests/test_abi.py -m "not gpu"
ASAN_OUT = os.path.join(HERE, "_asan", "libpadra_hip.so")
ASAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
              "-Xarch_host", "-fno-sanitize-recover=undefined", "-shared-libasan", "-g"]


def command(out: str = OUT, asan: bool = False) -> list[str]:
    return [hipcc(), "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-mllvm", "-amdgpu-mfma-vgpr-form"] + (ASAN_FLAGS if asan else []) + \
           ["-Wall", "-I", os.path.join(ROOT, "include"), "-o", out] + \
           [os.path.join(HERE, s) for s in SOURCES]


CALLER_SRC = os.path.join(ROOT, "tests", "cpp", "padra_caller.cpp")
CALLER_OUT = os.path.join(ROOT, "tests", "cpp", "padra_caller")


def build_caller(lib: str = OUT) -> str:
    """The C++20 test program that calls the library through include/padra_hip.h only
    (tests/test_gpu_cpp_caller.py runs it): host code, linked against libpadra_hip.so with
    an rpath to the package directory."""
    cmd = [hipcc(), "-std=c++20", "-O2", "-Wall", "-I", os.path.join(ROOT, "include"),
           CALLER_SRC, "-L", os.path.dirname(lib), "-lpadra_hip",
           "-Wl,-rpath," + os.path.dirname(lib), "-o", CALLER_OUT]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed (C++ caller):\n" + res.stdout + res.stderr)
    return CALLER_OUT


def build(out: str = OUT, verbose: bool = False, asan: bool = False) -> str:
    if asan:
        out = ASAN_OUT
        os.makedirs(os.path.dirname(out), exist_ok=True)
    cmd = command(out, asan)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "warning: argument unused")
    msgs = [l for l in (res.stdout + res.stderr).splitlines() if l and not any(n in l for n in noise)]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), file=sys.stderr)
    return out


if __name__ == "__main__":
    print(build(verbose=True, asan="--asan" in sys.argv[1:]))
    if "--asan" not in sys.argv[1:]:
        print(build_caller())
