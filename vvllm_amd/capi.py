"""ctypes binding of the C ABI in include/vvllm_hip.h (libvvllm_hip.so).

The binding table below is the one a maintainer of the reference would add to
call the path from Python; the C++ host code (vvllm_amd/host/backend_hip.cc)
calls the same functions directly.  There is no fallback: if the library is
not built, :func:`load` raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_size_t, c_uint64, c_void_p

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libvvllm_hip.so")

F32, F16, BF16 = 0, 1, 2
OP_ADD, OP_MUL, OP_SILU, OP_SILU_MUL = 0, 1, 2, 3
IN_NONE, IN_RMS_NORM, IN_SILU_MUL = 0, 1, 2
KERNEL_AUTO, KERNEL_GENERIC, KERNEL_GEMV_F32, KERNEL_SKINNY, KERNEL_GEMM, KERNEL_STREAM, KERNEL_DOT = range(7)
KERNEL_NAMES = {0: "auto", 1: "generic", 2: "gemv_f32", 3: "skinny", 4: "gemm", 5: "stream", 6: "dot"}
STATUS = {0: "VVH_OK", 1: "VVH_ERR_INVALID_ARG", 2: "VVH_ERR_NO_DEVICE", 3: "VVH_ERR_OUT_OF_MEMORY",
          4: "VVH_ERR_HIP", 5: "VVH_ERR_NOT_INITIALIZED", 6: "VVH_ERR_UNKNOWN_HANDLE",
          7: "VVH_ERR_UNSUPPORTED"}


class PoolStats(ctypes.Structure):
    _fields_ = [(n, c_uint64) for n in ("bytes_in_use", "bytes_cached", "bytes_reserved", "peak_reserved",
                                        "alloc_calls", "cache_hits", "driver_allocs", "oom_releases")]


class Q8Problem(ctypes.Structure):
    _fields_ = [("out", c_void_p), ("inp", c_void_p), ("residual", c_void_p), ("weight", c_void_p),
                ("scales", c_void_p), ("bias", c_void_p), ("M", c_uint64), ("N", c_uint64), ("K", c_uint64)]


_PP = POINTER(c_void_p)
# name -> (restype, argtypes); every VVH_API function of include/vvllm_hip.h
SIGNATURES = {
    "vvh_status_string": (c_char_p, [c_int]),
    "vvh_last_error": (c_char_p, []),
    "vvh_version": (c_char_p, []),
    "vvh_init": (c_int, [c_int, c_char_p, c_size_t]),
    "vvh_sync": (c_int, []),
    "vvh_device_cu_count": (c_int, []),
    "vvh_malloc": (c_int, [_PP, c_size_t]),
    "vvh_free": (c_int, [c_void_p]),
    "vvh_malloc_host": (c_int, [_PP, c_size_t]),
    "vvh_free_host": (c_int, [c_void_p]),
    "vvh_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_size_t]),
    "vvh_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_size_t]),
    "vvh_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_size_t]),
    "vvh_workspace_release": (c_int, [c_void_p]),
    "vvh_pool_alloc": (c_int, [_PP, c_size_t]),
    "vvh_pool_free": (c_int, [c_void_p]),
    "vvh_pool_release_cached": (c_int, []),
    "vvh_pool_get_stats": (c_int, [POINTER(PoolStats)]),
    "vvh_weight_register": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, POINTER(c_uint64)]),
    "vvh_weight_ingest": (c_int, [c_void_p, c_int, c_void_p, c_size_t, c_size_t, c_void_p, POINTER(c_uint64)]),
    "vvh_weight_register_device": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, POINTER(c_uint64)]),
    "vvh_weight_find": (c_int, [c_void_p, POINTER(c_uint64)]),
    "vvh_weight_release": (c_int, [c_uint64]),
    "vvh_weight_device_ptrs": (c_int, [c_uint64, _PP, _PP, _PP, POINTER(c_size_t), POINTER(c_size_t)]),
    "vvh_weight_stats": (c_int, [POINTER(c_uint64), POINTER(c_uint64)]),
    "vvh_linear_q8": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p, c_size_t, c_size_t, c_size_t,
                              c_int, c_int, c_void_p]),
    "vvh_linear_q8_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                  c_size_t, c_size_t, c_int, c_int, c_void_p]),
    "vvh_linear_q8_dev_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                          c_size_t, c_size_t, c_int, c_int, c_void_p]),
    "vvh_plan_create": (c_int, [POINTER(Q8Problem), c_size_t, c_int, c_int, POINTER(c_uint64)]),
    "vvh_plan_run": (c_int, [c_uint64, c_void_p]),
    "vvh_plan_set_input_op": (c_int, [c_uint64, c_int, c_void_p, c_float]),
    "vvh_plan_set_rope": (c_int, [c_uint64, c_size_t, c_size_t, c_size_t, c_size_t, c_float, c_void_p, c_void_p]),
    "vvh_plan_set_rope_table": (c_int, [c_uint64, c_size_t]),
    "vvh_plan_run_pos": (c_int, [c_uint64, c_size_t, c_void_p]),
    "vvh_plan_set_glu": (c_int, [c_uint64, c_size_t]),
    "vvh_kv_append": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "vvh_linear_q8_dev_in": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                     c_size_t, c_size_t, c_int, c_int, c_int, c_void_p, c_float, c_void_p]),
    "vvh_rope_append": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t,
                                c_size_t, c_size_t, c_float, c_int, c_void_p]),
    "vvh_plan_destroy": (c_int, [c_uint64]),
    "vvh_plan_launches": (c_int, [c_uint64, POINTER(c_int)]),
    "vvh_plan_kernel": (c_int, [c_uint64, POINTER(c_int)]),
    "vvh_quantize_per_channel": (c_int, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, c_void_p]),
    "vvh_convert": (c_int, [c_void_p, c_int, c_void_p, c_int, c_size_t, c_void_p]),
    "vvh_fill_normal": (c_int, [c_void_p, c_int, c_size_t, c_uint64, c_float, c_float, c_void_p]),
    "vvh_linear_q8_choice": (c_int, [c_size_t, c_size_t, c_size_t, c_int, c_int]),
    "vvh_set_kernel_override": (c_int, [c_int]),
    "vvh_eltwise": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_size_t, c_int, c_void_p]),
    "vvh_rms_norm": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_float, c_int, c_void_p]),
    "vvh_softmax": (c_int, [c_void_p, c_void_p, c_size_t, c_size_t, c_int, c_void_p]),
    "vvh_rope": (c_int, [c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_size_t, c_size_t, c_float, c_int,
                         c_void_p]),
    "vvh_embedding": (c_int, [c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_int, c_void_p]),
    "vvh_attention": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_size_t,
                              c_size_t, c_float, c_int, c_void_p]),
    "vvh_attention_parts": (c_int, [c_void_p, c_size_t, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                    c_size_t, c_size_t, c_size_t, c_float, c_int, c_void_p]),
    "vvh_linear_q8_dev_attn": (c_int, [c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_size_t, c_size_t, c_int, c_void_p]),
    "vvh_dense": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t,
                          c_int, c_void_p]),
    "vvh_matmul": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_int, c_void_p]),
    "vvh_argmax": (c_int, [c_void_p, c_size_t, c_void_p, c_void_p]),
    "vvh_sample": (c_int, [c_void_p, c_int, c_size_t, ctypes.c_float, ctypes.c_float, ctypes.c_uint64, ctypes.c_int32,
                           c_void_p, c_void_p]),
    "vvh_mirror_f32": (c_int, [c_void_p, c_size_t, c_int, POINTER(c_void_p)]),
    "vvh_mirror_release": (c_int, [c_void_p]),
    "vvh_memcpy_d2d_async": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "vvh_gemm_variant": (c_int, [c_size_t, c_size_t, c_size_t, POINTER(c_int), POINTER(c_int)]),
}
# entries that return a value rather than a vvh_status
_NOT_STATUS = {"vvh_status_string", "vvh_last_error", "vvh_version", "vvh_device_cu_count",
               "vvh_linear_q8_choice", "vvh_gemm_variant"}


class VVHError(RuntimeError):
    def __init__(self, fn: str, status: int, message: str):
        self.fn, self.status, self.message = fn, status, message
        super().__init__(f"{fn}: {STATUS.get(status, status)}: {message}")


_lib: ctypes.CDLL | None = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libvvllm_hip.so and bind its signatures; raise if it is missing."""
    global _lib
    if _lib is not None and path == LIB_PATH:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built: run __graft_entry__.build() "
                          "(python -m vvllm_amd.build); there is no fallback path")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    if path == LIB_PATH:
        _lib = lib
    return lib


def call(name: str, *args) -> int:
    """Call a status-returning entry point; raise VVHError unless VVH_OK."""
    lib = load()
    st = getattr(lib, name)(*args)
    if name not in _NOT_STATUS and st != 0:
        raise VVHError(name, st, lib.vvh_last_error().decode(errors="replace"))
    return st


def status_of(name: str, *args) -> int:
    """Call an entry point and return its raw status (no raise)."""
    return getattr(load(), name)(*args)


# ---------------------------------------------------------------------------
# small host-side helpers used by tests and bench.py
# ---------------------------------------------------------------------------
_initialised = False


def init(device: int = 0) -> str:
    global _initialised
    buf = ctypes.create_string_buffer(256)
    call("vvh_init", device, buf, 256)
    _initialised = True
    return buf.value.decode()


class DevBuf:
    """Device allocation from vvh_malloc (freed with the object)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = c_void_p()
        call("vvh_malloc", ctypes.byref(p), self.nbytes)
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(a)
        b = cls(max(a.nbytes, 1))
        if a.nbytes:
            call("vvh_memcpy_h2d", b.ptr, a.ctypes.data, a.nbytes)
        return b

    def to_array(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            call("vvh_memcpy_d2h", out.ctypes.data, self.ptr, out.nbytes)
        return out

    def addr(self, byte_offset: int = 0) -> int:
        return self.ptr + byte_offset

    def free(self) -> None:
        if getattr(self, "ptr", None):
            load().vvh_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def np_dtype(d: int):
    return np.float32 if d == F32 else np.float16


def linear_q8_dev(out, inp, w, scales, bias, residual, M, N, K, act=F32, outd=F32, stream=None) -> None:
    """vvh_linear_q8_dev on raw device addresses (ints) or DevBufs."""
    a = lambda x: None if x is None else (x.ptr if isinstance(x, DevBuf) else x)
    call("vvh_linear_q8_dev", a(out), a(inp), a(w), a(scales), a(bias), a(residual), M, N, K, act, outd, stream)


def set_kernel(kernel: int) -> None:
    call("vvh_set_kernel_override", kernel)


def kernel_choice(M, N, K, act, outd) -> str:
    return KERNEL_NAMES.get(load().vvh_linear_q8_choice(M, N, K, act, outd), "?")


def gemm_variant(M, N, K) -> str:
    """Name of the GEMM kernel an fp16 call of this shape dispatches to."""
    tn, sp = c_int(), c_int()
    v = load().vvh_gemm_variant(M, N, K, ctypes.byref(tn), ctypes.byref(sp))
    if v in (3, 4):
        return f"k_gemm3 {128 if v == 3 else 64}x{tn.value}" + (f" split {sp.value}" if sp.value > 1 else "")
    return "k_gemm" if v == 1 else "?"


def sync() -> None:
    call("vvh_sync")


def plan_kernel(plan: int) -> str:
    k = c_int()
    call("vvh_plan_kernel", plan, ctypes.byref(k))
    return KERNEL_NAMES.get(k.value, "?")
