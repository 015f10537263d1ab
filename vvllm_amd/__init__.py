"""vvllm_amd -- MI355X (gfx950) INT8 per-channel linear path for vvllm.

Contents:
  csrc/     HIP kernels and the C ABI (built into lib/libvvllm_hip.so)
  host/     BackendHIP, the C++20 vvllm Backend over that ABI
            (built into lib/libvvllm_backend_hip.so)
  capi.py   ctypes binding of the same ABI (tests, bench.py)
  build.py  build recipes

Importing the package does not touch the GPU; :func:`capi.load` raises if the
native library has not been built.
"""
from . import capi  # noqa: F401

__all__ = ["capi"]
__version__ = "0.1.0"
