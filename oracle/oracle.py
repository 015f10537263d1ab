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
        F = ctypes.c_float
        for nm, at in (("add", [_P, _P, _P, _S]), ("mul", [_P, _P, _P, _S]), ("silu", [_P, _P, _S]),
                       ("silu_mul", [_P, _P, _P, _S]), ("rms_norm", [_P, _P, _P, _S, F]), ("softmax", [_P, _P, _S]),
                       ("rope", [_P, _P, _S, _S, _S, _S, _S, F]), ("linear", [_P, _P, _P, _P, _S, _S, _S]),
                       ("linear_add", [_P, _P, _P, _P, _P, _S, _S, _S]), ("matmul", [_P, _P, _P, _S, _S, _S]),
                       ("causal_attention", [_P, _P, _S, _P, _P, _S, _S, _S, _S, F])):
            getattr(lib, pre + nm).argtypes = at
        if kind == "port":
            lib.orc_linear_q8_f64.argtypes = [_P, _P, _P, _P, _P, _P, _S, _S, _S]
            lib.orc_bf16_to_f32.argtypes = [_P, _S, _P]
            lib.orc_ingest_bf16.argtypes = [_P, _S, _S, _P, _P]
            lib.orc_sample_hash.argtypes = [ctypes.c_uint64, ctypes.c_int32, ctypes.c_int32]
            lib.orc_sample_hash.restype = ctypes.c_uint64
            lib.orc_sample_uniform.argtypes = [ctypes.c_uint64, ctypes.c_int32, ctypes.c_int32]
            lib.orc_sample_uniform.restype = ctypes.c_float
            lib.orc_sample.argtypes = [_P, _S, ctypes.c_float, ctypes.c_uint64, ctypes.c_int32, _P, _P]
            lib.orc_sample.restype = ctypes.c_int32
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


# ---- the other BackendCPU operators (src/backend/backend_naive.cc) ----
def _fn(kind, name):
    return getattr(_lib(kind), ("orc_" if kind == "port" else "ref_") + name)


def eltwise(op: str, x, y=None, kind: str = "port"):
    """op in add / mul / silu / silu_mul (y = up for silu_mul)."""
    x = _f32(x).ravel()
    out = np.empty_like(x)
    if op == "silu":
        _fn(kind, op)(_ptr(out), _ptr(x), x.size)
    else:
        y = _f32(y).ravel()
        _fn(kind, op)(_ptr(out), _ptr(x), _ptr(y), x.size)
    return out


def rms_norm(x, w, eps, kind: str = "port"):
    """Row by row over the last axis."""
    x = _f32(x)
    rows = x.reshape(-1, x.shape[-1])
    w = _f32(w)
    out = np.empty_like(rows)
    for r in range(rows.shape[0]):
        _fn(kind, "rms_norm")(_ptr(out[r]), _ptr(np.ascontiguousarray(rows[r])), _ptr(w), rows.shape[1], eps)
    return out.reshape(x.shape)


def softmax(x, kind: str = "port"):
    x = _f32(x)
    rows = x.reshape(-1, x.shape[-1])
    out = np.empty_like(rows)
    for r in range(rows.shape[0]):
        _fn(kind, "softmax")(_ptr(out[r]), _ptr(np.ascontiguousarray(rows[r])), rows.shape[1])
    return out.reshape(x.shape)


def rope(q, k, pos, theta, kind: str = "port"):
    """q [S, H, D], k [S, KVH, D] -> rotated copies."""
    q, k = _f32(q).copy(), _f32(k).copy()
    S, H, D = q.shape
    _fn(kind, "rope")(_ptr(q), _ptr(k), S, H, k.shape[1], D, pos, theta)
    return q, k


def linear(x, w, bias=None, residual=None, kind: str = "port"):
    """out = x @ w.T + bias (+ residual): Backend::linear / linear_add."""
    x, w = _f32(x), _f32(w)
    M, K = x.shape
    N = w.shape[0]
    out = np.empty((M, N), np.float32)
    if residual is None:
        _fn(kind, "linear")(_ptr(out), _ptr(x), _ptr(w), _ptr(_f32(bias)), M, N, K)
    else:
        _fn(kind, "linear_add")(_ptr(out), _ptr(x), _ptr(w), _ptr(_f32(bias)), _ptr(_f32(residual)), M, N, K)
    return out


def matmul(a, b, kind: str = "port"):
    a, b = _f32(a), _f32(b)
    M, K = a.shape
    N = b.shape[1]
    out = np.empty((M, N), np.float32)
    _fn(kind, "matmul")(_ptr(out), _ptr(a), _ptr(b), M, N, K)
    return out


def causal_attention(q, k, v, q_idx, attend_len, scale, kind: str = "port"):
    """q [S, H, D], k/v [T, KVH, D] -> out [H * D] for query q_idx over the
    first attend_len positions."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    S, H, D = q.shape
    out = np.empty(H * D, np.float32)
    _fn(kind, "causal_attention")(_ptr(out), _ptr(q), q_idx, _ptr(k), _ptr(v), attend_len, H, k.shape[1], D, scale)
    return out


def sample_hash(seed: int, step: int, idx: int) -> int:
    """gpu_rand's 64-bit hash (src/backend/cuda_kernels.cu:1230-1235)."""
    return int(_lib("port").orc_sample_hash(seed, step, idx))


def sample_uniform(seed: int, step: int, idx: int) -> float:
    """gpu_rand (src/backend/cuda_kernels.cu:1228-1237)."""
    return float(_lib("port").orc_sample_uniform(seed, step, idx))


def sample(logits, temperature: float, seed: int, step: int):
    """(index, best noisy value, second best) of the device sampler's
    Gumbel-max trick (temperature > 0) or the greedy argmax (temperature 0)."""
    x = _f32(np.ravel(logits))
    best, second = ctypes.c_float(), ctypes.c_float()
    i = _lib("port").orc_sample(x.ctypes.data, x.size, temperature, seed, step, ctypes.byref(best),
                               ctypes.byref(second))
    return int(i), best.value, second.value
