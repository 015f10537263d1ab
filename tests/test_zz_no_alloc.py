"""vvh_linear_q8_dev_noalloc: the allocation-free variant of vvh_linear_q8_dev.

Its split-K partial planes live in a fixed device array instead of the
stream's workspace.  Checked here, through the C ABI:
  * two calls in a row, the second with a smaller input, on shapes the
    dispatcher splits (so the fixed scratch is what carries the partial
    sums), give the same bits as vvh_linear_q8_dev and agree with the CPU
    oracle to the normalized-error bar of the linear path;
  * fp32 activations at the configs[3] shapes (M = 512), whose split fp16
    form also lives in the fixed scratch, give the same bits as well;
  * a call that needs more than VVH_NOALLOC_SCRATCH_BYTES is refused before
    any launch;
  * a call on a stream that has no workspace yet leaves the device's free
    memory unchanged, while vvh_linear_q8_dev on that stream allocates its
    workspace (so the check can see an allocation).
"""
import ctypes

import numpy as np
import pytest

from vvllm_amd import capi

pytestmark = pytest.mark.gpu

F16, F32 = capi.F16, capi.F32
TOL = {F16: 2e-3, F32: 2e-3}  # fp16 activations: the fp16-activation bar


def _inputs(oracle, M, N, K, act, outd, seed):
    rng = np.random.default_rng(seed)
    w = rng.normal(0.0, 0.02, (N, K)).astype(np.float32)
    q, s = oracle.quantize_per_channel(w)
    b = rng.normal(0.0, 0.01, N).astype(np.float32)
    x = rng.normal(0.0, 1.0, (M, K)).astype(np.float16 if act == F16 else np.float32)
    r = rng.normal(0.0, 1.0, (M, N)).astype(np.float16 if outd == F16 else np.float32)
    return q, s, b, x, r


def _run(entry, M, N, K, act, outd, bufs, stream=None):
    d_q, d_s, d_b, d_x, d_r, d_y = bufs
    capi.call(entry, d_y.ptr, d_x.ptr, d_q.ptr, d_s.ptr, d_b.ptr, d_r.ptr, M, N, K, act, outd, stream)
    capi.sync()
    return d_y.to_array(np.float16 if outd == F16 else np.float32, (M, N))


@pytest.mark.parametrize("outd", [F16, F32])
def test_noalloc_matches_linear_q8_dev_two_calls(gpu, oracle, outd):
    N, K = 896, 4864
    for i, M in enumerate((512, 128)):  # second call smaller than the first
        print(f"[case] noalloc M={M} N={N} K={K} out={outd} {capi.gemm_variant(M, N, K)}", flush=True)
        assert "split" in capi.gemm_variant(M, N, K), "shape must exercise the split-K scratch"
        q, s, b, x, r = _inputs(oracle, M, N, K, F16, outd, seed=71 + i)
        bufs = [capi.DevBuf.from_array(a) for a in (q, s, b, x, r)] + [capi.DevBuf(r.nbytes)]
        y_ref = _run("vvh_linear_q8_dev", M, N, K, F16, outd, bufs)
        y_na = _run("vvh_linear_q8_dev_noalloc", M, N, K, F16, outd, bufs)
        assert np.array_equal(y_na.view(np.uint8), y_ref.view(np.uint8)), "noalloc differs from vvh_linear_q8_dev"
        ref = oracle.linear_q8(x.astype(np.float32), q, s, b, r.astype(np.float32))
        err = float(np.abs(y_na.astype(np.float32) - ref).max() / np.abs(ref).max())
        assert err <= TOL[outd], f"normalized max error {err:.3e}"


@pytest.mark.parametrize("N,K", [(896, 4864), (4864, 896)], ids=["down", "gate_up"])
def test_noalloc_fp32_activations_prefill(gpu, oracle, N, K):
    """configs[3] shapes at M = 512 with fp32 activations (the reference's
    default mode): the split fp16 activations (and, for down, the split-K
    planes) in the fixed scratch; the same bits as vvh_linear_q8_dev and the
    fp32-activation bar against the oracle."""
    M = 512
    print(f"[case] noalloc fp32 M={M} N={N} K={K}", flush=True)
    q, s, b, x, r = _inputs(oracle, M, N, K, F32, F32, seed=13)
    bufs = [capi.DevBuf.from_array(a) for a in (q, s, b, x, r)] + [capi.DevBuf(r.nbytes)]
    y_ref = _run("vvh_linear_q8_dev", M, N, K, F32, F32, bufs)
    y_na = _run("vvh_linear_q8_dev_noalloc", M, N, K, F32, F32, bufs)
    assert np.array_equal(y_na.view(np.uint32), y_ref.view(np.uint32)), "noalloc differs from vvh_linear_q8_dev"
    ref = oracle.linear_q8(x, q, s, b, r)
    err = float(np.abs(y_na - ref).max() / np.abs(ref).max())
    assert err <= 1e-4, f"normalized max error {err:.3e}"


def test_noalloc_refuses_oversize_call(gpu, oracle):
    """An fp32-activation GEMM whose split activations alone (2048 x 4864 x 4
    bytes = 39.8 MB) exceed VVH_NOALLOC_SCRATCH_BYTES is refused before any
    launch: VVH_ERR_UNSUPPORTED, the output untouched; vvh_linear_q8_dev runs
    the same call."""
    M, N, K = 2048, 896, 4864
    assert M * K * 4 > 32 << 20
    rng = np.random.default_rng(3)
    q, s = oracle.quantize_per_channel(rng.normal(0.0, 0.02, (N, K)).astype(np.float32))
    x = rng.normal(0.0, 1.0, (M, K)).astype(np.float32)
    d_q, d_s, d_x = (capi.DevBuf.from_array(a) for a in (q, s, x))
    sentinel = np.full((M, N), 7.0, np.float32)
    d_y = capi.DevBuf.from_array(sentinel)
    st = capi.status_of("vvh_linear_q8_dev_noalloc", d_y.ptr, d_x.ptr, d_q.ptr, d_s.ptr, None, None, M, N, K, F32,
                        F32, None)
    capi.sync()
    assert st == 7, f"status {st}: expected VVH_ERR_UNSUPPORTED"
    assert "workspace" in capi.load().vvh_last_error().decode()
    assert np.array_equal(d_y.to_array(np.float32, (M, N)), sentinel), "a refused call wrote its output"
    capi.call("vvh_linear_q8_dev", d_y.ptr, d_x.ptr, d_q.ptr, d_s.ptr, None, None, M, N, K, F32, F32, None)
    capi.sync()
    rows = [0, 1, 1023, 2047]
    ref = oracle.linear_q8(x[rows], q, s, None, None)
    got = d_y.to_array(np.float32, (M, N))[rows]
    assert float(np.abs(got - ref).max() / np.abs(ref).max()) <= 1e-4


def test_noalloc_decode_shape(gpu, oracle):
    M, N, K = 1, 4864, 896
    q, s, b, x, r = _inputs(oracle, M, N, K, F16, F16, seed=5)
    bufs = [capi.DevBuf.from_array(a) for a in (q, s, b, x, r)] + [capi.DevBuf(r.nbytes)]
    y_ref = _run("vvh_linear_q8_dev", M, N, K, F16, F16, bufs)
    y_na = _run("vvh_linear_q8_dev_noalloc", M, N, K, F16, F16, bufs)
    assert np.array_equal(y_na.view(np.uint16), y_ref.view(np.uint16))


def test_noalloc_allocates_nothing(gpu, oracle):
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t)] * 2
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]

    def free_bytes():
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        assert hip.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
        return f.value

    M, N, K = 512, 896, 4864
    q, s, b, x, r = _inputs(oracle, M, N, K, F16, F16, seed=9)
    bufs = [capi.DevBuf.from_array(a) for a in (q, s, b, x, r)] + [capi.DevBuf(r.nbytes)]
    _run("vvh_linear_q8_dev", M, N, K, F16, F16, bufs)  # kernels loaded, null-stream workspace made
    stream = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        before = free_bytes()
        for _ in range(3):
            _run("vvh_linear_q8_dev_noalloc", M, N, K, F16, F16, bufs, stream.value)
        after_noalloc = free_bytes()
        _run("vvh_linear_q8_dev", M, N, K, F16, F16, bufs, stream.value)  # grows this stream's workspace
        after_dev = free_bytes()
        print(f"[free] before {before} after noalloc {after_noalloc} after dev {after_dev}", flush=True)
        assert after_noalloc == before, "vvh_linear_q8_dev_noalloc allocated device memory"
        assert after_dev < after_noalloc, "the check cannot see the workspace allocation"
    finally:
        capi.call("vvh_workspace_release", stream.value)
        hip.hipStreamDestroy(stream)
