"""ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product (vvllm_amd).  Two libraries can sit behind it:

* ``liboracle.so``  -- this repository's C restatement (oracle.c) of
  quantize_per_channel (src/quantize/quantize.cc:9-48) and
  BackendCPU::linear_q8 / linear_q8_add (src/backend/backend_naive.cc:155-291,
  :322-335);
* ``_ref/libvvllm_ref.so`` -- the reference's own two source files compiled
  in place by ``make ref`` (present only where the reference tree was).

Both take numpy arrays; ``kind`` picks the library ("port" or "reference").
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_PORT = os.path.join(_HERE, "liboracle.so")
_REF = os.path.join(_HERE, "_ref", "libvvllm_ref.so")

_P = ctypes.c_void_p
_S = ctypes.c_size_t
_libs: dict[str, ctypes.CDLL] = {}


def build(ref: bool = False) -> None:
    """Compile liboracle.so (and _ref/ when ``ref`` and the reference exists)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    if ref and os.path.isdir("/root/reference"):
        subprocess.run(["make", "-s", "-C", _HERE, "ref"], check=True)


def available(kind: str = "port") -> bool:
    return os.path.exists(_PORT if kind == "port" else _REF)


def _lib(kind: str) -> ctypes.CDLL:
    if kind not in _libs:
        path = _PORT if kind == "port" else _REF
        if not os.path.exists(path):
            raise FileNotFoundError(f"oracle library {path} is not built")
        lib = ctypes.CDLL(path)
        pre = "orc_" if kind == "port" else "ref_"
        getattr(lib, pre + "quantize_per_channel").argtypes = [_P, _S, _S, _P, _P]
        getattr(lib, pre + "linear_q8").argtypes = [_P, _P, _P, _P, _P, _S, _S, _S]
        getattr(lib, pre + "linear_q8_add").argtypes = [_P, _P, _P, _P, _P, _P, _S, _S, _S]
        if kind == "port":
            lib.orc_linear_q8_f64.argtypes = [_P, _P, _P, _P, _P, _P, _S, _S, _S]
            lib.orc_bf16_to_f32.argtypes = [_P, _S, _P]
            lib.orc_ingest_bf16.argtypes = [_P, _S, _S, _P, _P]
        _libs[kind] = lib
    return _libs[kind]


def _ptr(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def quantize_per_channel(w: np.ndarray, kind: str = "port"):
    """w: [N, K] float32 -> (codes int8 [N, K], scales float32 [N])."""
    w = _f32(w)
    N, K = w.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((N,), np.float32)
    pre = "orc_" if kind == "port" else "ref_"
    getattr(_lib(kind), pre + "quantize_per_channel")(_ptr(w), N, K, _ptr(q), _ptr(s))
    return q, s


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 BF16 bit patterns -> float32 (safetensors.cc:135-141)."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    _lib("port").orc_bf16_to_f32(_ptr(bits), bits.size, _ptr(out))
    return out


def ingest_bf16(bits: np.ndarray):
    """[N, K] uint16 BF16 bit patterns -> (codes, scales) of the host path:
    widen to fp32, then quantize_per_channel."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    N, K = bits.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((N,), np.float32)
    _lib("port").orc_ingest_bf16(_ptr(bits), N, K, _ptr(q), _ptr(s))
    return q, s


def linear_q8(x, q, scales, bias=None, residual=None, kind: str = "port", inplace=False):
    """out[M,N] = (x @ q.T) * scales + bias (+ residual), reference semantics.

    ``inplace`` runs linear_q8_add with out aliasing residual, as the model
    does (include/vvllm/model/transformer.h:165-166)."""
    x = _f32(x)
    M, K = x.shape
    N = q.shape[0]
    q = np.ascontiguousarray(q, dtype=np.int8)
    scales = _f32(scales)
    bias = _f32(bias)
    lib = _lib(kind)
    pre = "orc_" if kind == "port" else "ref_"
    if residual is None:
        out = np.empty((M, N), np.float32)
        getattr(lib, pre + "linear_q8")(_ptr(out), _ptr(x), _ptr(q), _ptr(scales), _ptr(bias), M, N, K)
        return out
    residual = _f32(residual).copy()
    out = residual if inplace else np.empty((M, N), np.float32)
    getattr(lib, pre + "linear_q8_add")(_ptr(out), _ptr(x), _ptr(q), _ptr(scales), _ptr(bias),
                                        _ptr(residual), M, N, K)
    return out


def linear_q8_f64(x, q, scales, bias=None, residual=None):
    x = _f32(x)
    M, K = x.shape
    N = q.shape[0]
    q = np.ascontiguousarray(q, dtype=np.int8)
    out = np.empty((M, N), np.float64)
    _lib("port").orc_linear_q8_f64(_ptr(out), _ptr(x), _ptr(q), _ptr(_f32(scales)), _ptr(_f32(bias)),
                                   _ptr(_f32(residual)), M, N, K)
    return out
