"""Build recipes for the native code of vvllm_amd.

* ``lib/libvvllm_hip.so``          -- HIP kernels + C ABI (hipcc, gfx950 only)
* ``lib/libvvllm_backend_hip.so``  -- BackendHIP, C++20 host code (g++) over the C ABI
* ``tests/cpp/bin/test_pool``      -- CPU test of the caching allocator logic
* ``tests/cpp/bin/test_backend_hip`` -- GPU test of BackendHIP
* ``tests/cpp/bin/test_forward_hip`` -- GPU test: whole forward passes through
  Backend/KVCache, checked against the CPU oracle (oracle/oracle.c, linked
  into the test binary only)

Everything is built in-tree so the artefacts travel with the source tree.
Run ``python -m vvllm_amd.build`` or call :func:`build_all`.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "lib")
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
INCLUDE = os.path.join(ROOT, "include")
TEST_BIN = os.path.join(ROOT, "tests", "cpp", "bin")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

HIP_SOURCES = ["runtime.hip", "linear_kernels.hip", "gemm_kernels.hip", "model_kernels.hip", "aux_kernels.hip"]
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-fvisibility=hidden",
    # no packed-fp32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE fp32 division for the quantizer's scale and reciprocal
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # the leading scalar kernel arguments (up to 16 dwords) arrive in SGPRs at
    # dispatch instead of through a load from the kernel-argument segment
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-I" + INCLUDE,
]

HIP_LIB = os.path.join(LIB, "libvvllm_hip.so")
BACKEND_LIB = os.path.join(LIB, "libvvllm_backend_hip.so")


def _run(cmd: list[str], out: str) -> None:
    tmp = out + ".tmp"
    p = subprocess.run(cmd + ["-o", tmp], capture_output=True, text=True)
    if p.returncode != 0:
        msg = "\n".join(l for l in p.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{msg}")
    os.replace(tmp, out)


OBJ = os.path.join(ROOT, "_build", "hip")


def build_hip_lib() -> str:
    """One hipcc per source, in parallel (no device code crosses a file), then
    one link."""
    os.makedirs(LIB, exist_ok=True)
    os.makedirs(OBJ, exist_ok=True)
    objs = [os.path.join(OBJ, os.path.splitext(s)[0] + ".o") for s in HIP_SOURCES]
    with ThreadPoolExecutor(max_workers=min(len(HIP_SOURCES), os.cpu_count() or 1)) as ex:
        for f in [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, s)], o)
                  for s, o in zip(HIP_SOURCES, objs)]:
            f.result()
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs], HIP_LIB)
    return HIP_LIB


def build_backend_lib() -> str:
    os.makedirs(LIB, exist_ok=True)
    _run([CXX, "-std=c++20", "-O2", "-fPIC", "-shared", "-Wall", "-I" + INCLUDE, "-I" + HOST,
          os.path.join(HOST, "backend_hip.cc"), "-L" + LIB, "-lvvllm_hip",
          "-Wl,-rpath,$ORIGIN"], BACKEND_LIB)
    return BACKEND_LIB


def build_test_pool() -> str:
    os.makedirs(TEST_BIN, exist_ok=True)
    out = os.path.join(TEST_BIN, "test_pool")
    _run([CXX, "-std=c++20", "-O1", "-g", "-Wall", "-fsanitize=address,undefined",
          "-I" + CSRC, "-I" + INCLUDE, os.path.join(ROOT, "tests", "cpp", "test_pool.cc")], out)
    return out


def build_test_backend() -> str:
    os.makedirs(TEST_BIN, exist_ok=True)
    out = os.path.join(TEST_BIN, "test_backend_hip")
    _run([CXX, "-std=c++20", "-O2", "-Wall", "-I" + INCLUDE, "-I" + HOST,
          os.path.join(ROOT, "tests", "cpp", "test_backend_hip.cc"), "-L" + LIB,
          "-lvvllm_backend_hip", "-lvvllm_hip", "-Wl,-rpath,$ORIGIN/../../../vvllm_amd/lib"], out)
    return out


def build_test_forward() -> str:
    os.makedirs(TEST_BIN, exist_ok=True)
    out = os.path.join(TEST_BIN, "test_forward_hip")
    obj = os.path.join(TEST_BIN, "oracle.o")
    # the oracle with the reference's CPU flags (-mavx2 -mfma, oracle/Makefile)
    _run(["gcc", "-std=gnu11", "-O2", "-DNDEBUG", "-mavx2", "-mfma", "-c",
          os.path.join(ROOT, "oracle", "oracle.c")], obj)
    _run([CXX, "-std=c++20", "-O2", "-Wall", "-I" + INCLUDE, "-I" + HOST, "-I" + os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests", "cpp", "test_forward_hip.cc"), obj, "-L" + LIB,
          "-lvvllm_backend_hip", "-lvvllm_hip", "-lm", "-Wl,-rpath,$ORIGIN/../../../vvllm_amd/lib"], out)
    return out


def build_all(verbose: bool = True) -> None:
    with ThreadPoolExecutor(max_workers=2) as ex:
        f_hip = ex.submit(build_hip_lib)
        f_pool = ex.submit(build_test_pool)
        f_hip.result()
        build_backend_lib()
        build_test_backend()
        build_test_forward()
        f_pool.result()
    if verbose:
        print(f"built {HIP_LIB}, {BACKEND_LIB}, tests in {TEST_BIN}")


if __name__ == "__main__":
    build_all()
    sys.exit(0)
