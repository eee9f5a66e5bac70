"""Ahead-of-time build of the tiler-hip backend (the analogue of
tiler-metal-aot's offline driver, tiler-metal-aot/src/driver.rs:61-453).

1. The gfx950 kernels are compiled offline into one code object
   (clang -x hip --offload-arch=gfx950 --offload-device-only), with
   -ffp-contract=off (no implicit FMA) and packed-FP32 disabled.
2. The host runtime (C ABI of include/tiler_hip.h) is compiled with g++ and
   links that code object in as bytes, producing tiler_amd/_build/libtiler_hip.so.

Run `python -m tiler_amd.build` or call build().
"""
from __future__ import annotations

import os
import shlex
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
HSACO = os.path.join(BUILD, "tiler_kernels.hsaco")
LIB = os.path.join(BUILD, "libtiler_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
CLANG = os.path.join(ROCM, "llvm", "bin", "clang++")

DEVICE_FLAGS = [
    "-x", "hip", "--offload-arch=gfx950", "--offload-device-only", "--no-gpu-bundle-output",
    "-O3", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd, **kw):
    subprocess.run(cmd, check=True, **kw)


def _toolchain_identity() -> str:
    out = subprocess.run([CLANG, "--version"], check=True, capture_output=True, text=True).stdout
    return out.splitlines()[0].strip()


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    kernels = os.path.join(CSRC, "kernels", "tiler_kernels.hip")
    tmp = HSACO + ".tmp"
    _run([CLANG, *DEVICE_FLAGS, "-o", tmp, kernels])
    os.replace(tmp, HSACO)

    info = os.path.join(BUILD, "build_info.h")
    flags = " ".join(shlex.quote(f) for f in DEVICE_FLAGS)
    with open(info, "w") as fh:
        fh.write("#pragma once\n")
        fh.write(f"#define TILER_HIP_BUILD_TOOLCHAIN {_c_string(_toolchain_identity())}\n")
        fh.write(f"#define TILER_HIP_BUILD_FLAGS {_c_string(flags)}\n")
        fh.write("#define TILER_HIP_BUILD_FLAG_LIST " + ", ".join(_c_string(f) for f in DEVICE_FLAGS) + "\n")
        fh.write(f"#define TILER_HIP_BUILD_FLAG_COUNT {len(DEVICE_FLAGS)}\n")
    bundle = os.path.join(BUILD, "source_bundle.bin")
    with open(bundle + ".tmp", "wb") as fh:
        fh.write(source_bundle())
    os.replace(bundle + ".tmp", bundle)

    # The no-allocation entry point's static device array: one small HIP
    # translation unit compiled by hipcc for gfx950, so the runtime registers
    # the array and hipGetSymbolAddress can resolve it per device.
    noalloc_obj = os.path.join(BUILD, "noalloc.o")
    _run([os.path.join(ROCM, "bin", "hipcc"), "-x", "hip", "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC",
          "-c", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{ROOT}/include",
          "-o", noalloc_obj, os.path.join(CSRC, "runtime", "noalloc.hip")], stderr=subprocess.DEVNULL)
    payload_obj = os.path.join(BUILD, "payload.o")
    _run(["gcc", "-c", f'-DTILER_HSACO_PATH="{HSACO}"', f'-DTILER_SOURCE_BUNDLE_PATH="{bundle}"', "-o", payload_obj,
          os.path.join(CSRC, "runtime", "payload.S")])
    tmp_lib = LIB + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-result",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{ROOT}/include", f"-I{BUILD}",
          "-o", tmp_lib,
          os.path.join(CSRC, "runtime", "tiler_hip.cpp"),
          os.path.join(CSRC, "runtime", "program.cpp"),
          os.path.join(CSRC, "runtime", "digest.cpp"),
          os.path.join(CSRC, "runtime", "envelope.cpp"),
          os.path.join(CSRC, "runtime", "code_object.cpp"),
          payload_obj, noalloc_obj,
          f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp_lib, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def source_bundle() -> bytes:
    """The exact kernel sources the code object is compiled from, as one
    canonical byte run: the file count, then each file's path (relative to
    csrc/kernels, sorted) and contents, every run preceded by its length as a
    u64 big-endian (the identity framing of tiler-ir/src/identity.rs:84-111).
    The payload metadata carries it as the compiled source."""
    kdir = os.path.join(CSRC, "kernels")
    names = sorted(f for f in os.listdir(kdir) if f.endswith((".hip", ".h")))
    out = bytearray(len(names).to_bytes(8, "big"))
    for name in names:
        with open(os.path.join(kdir, name), "rb") as fh:
            body = fh.read()
        for run in (name.encode(), body):
            out += len(run).to_bytes(8, "big") + run
    return bytes(out)


def _c_string(s: str) -> str:
    return '"' + s.replace("\\", "\\\\").replace('"', '\\"') + '"'


if __name__ == "__main__":
    build(verbose=True)
