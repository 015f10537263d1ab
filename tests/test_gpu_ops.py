"""GPU parity of the decode-step operators besides linear_q8 (vvh_eltwise,
vvh_rms_norm, vvh_softmax, vvh_rope, vvh_embedding, vvh_attention, vvh_dense,
vvh_matmul, vvh_argmax, vvh_mirror_f32) against the CPU oracle, which restates
BackendCPU (src/backend/backend_naive.cc) and is pinned bit-for-bit to the
reference's own build (tests/test_oracle.py).

Tolerances: normalized max error max|y - r| / max|r| <= 1e-4 with fp32
activations, <= 2e-3 with fp16 activations (inputs are rounded to fp16 first
and the oracle gets the rounded values).  Argmax and the mirrors are exact.
"""
import ctypes

import numpy as np
import pytest

from vvllm_amd import capi

pytestmark = pytest.mark.gpu

F16, F32 = capi.F16, capi.F32
TOL = {F32: 1e-4, F16: 2e-3}


def npd(d):
    return np.float16 if d == F16 else np.float32


def up(a, d):
    """Device copy of `a` in activation dtype d; returns (buffer, the values the device holds)."""
    a = np.ascontiguousarray(a, dtype=npd(d))
    return capi.DevBuf.from_array(a), a.astype(np.float32)


def down(buf, d, shape):
    return buf.to_array(npd(d), shape).astype(np.float32)


def nerr(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def mirror(a, as_dtype=F32):
    a = np.ascontiguousarray(a, dtype=np.float32)
    dev = ctypes.c_void_p()
    capi.call("vvh_mirror_f32", a.ctypes.data, a.size, as_dtype, ctypes.byref(dev))
    return a, dev.value


@pytest.mark.parametrize("d", [F32, F16])
@pytest.mark.parametrize("n", [1, 1000, (1 << 20) + 3])
@pytest.mark.parametrize("op", ["add", "mul", "silu", "silu_mul"])
def test_eltwise(gpu, oracle, op, n, d):
    print(f"[case] eltwise {op} n={n} dtype={d}", flush=True)
    rng = np.random.default_rng(n)
    dx, x = up(rng.normal(0, 2, n), d)
    dy, y = up(rng.normal(0, 2, n), d)
    do = capi.DevBuf(n * np.dtype(npd(d)).itemsize)
    code = {"add": capi.OP_ADD, "mul": capi.OP_MUL, "silu": capi.OP_SILU, "silu_mul": capi.OP_SILU_MUL}[op]
    capi.call("vvh_eltwise", code, do.ptr, dx.ptr, dy.ptr, n, d, None)
    capi.sync()
    assert nerr(down(do, d, (n,)), oracle.eltwise(op, x, y)) <= TOL[d]


@pytest.mark.parametrize("d", [F32, F16])
@pytest.mark.parametrize("rows,n", [(1, 896), (3, 1536), (128, 1000), (2, 5), (2, 4864), (1, 8960), (3, 2055)])
def test_rms_norm(gpu, oracle, rows, n, d):
    print(f"[case] rms_norm rows={rows} n={n} dtype={d}", flush=True)
    rng = np.random.default_rng(rows * n)
    dx, x = up(rng.normal(0, 1, (rows, n)), d)
    w, dw = mirror(rng.normal(1, 0.1, n))
    do = capi.DevBuf(rows * n * np.dtype(npd(d)).itemsize)
    capi.call("vvh_rms_norm", do.ptr, dx.ptr, dw, rows, n, 1e-6, d, None)
    capi.sync()
    assert nerr(down(do, d, (rows, n)), oracle.rms_norm(x, w, 1e-6)) <= TOL[d]
    capi.call("vvh_mirror_release", w.ctypes.data)


@pytest.mark.parametrize("d", [F32, F16])
@pytest.mark.parametrize("rows,n", [(1, 7), (4, 1000), (1, 151936)])
def test_softmax(gpu, oracle, rows, n, d):
    print(f"[case] softmax rows={rows} n={n} dtype={d}", flush=True)
    dx, x = up(np.random.default_rng(n).normal(0, 3, (rows, n)), d)
    do = capi.DevBuf(rows * n * np.dtype(npd(d)).itemsize)
    capi.call("vvh_softmax", do.ptr, dx.ptr, rows, n, d, None)
    capi.sync()
    got, ref = down(do, d, (rows, n)), oracle.softmax(x)
    # The reference sums n exponentials one after another in fp32; over long
    # rows its own rounding exceeds the bound, so the GPU result must then be
    # at least as close as the reference to the exact (fp64) softmax.
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    exact = e / e.sum(axis=1, keepdims=True)
    assert nerr(got, ref) <= TOL[d] or nerr(got, exact) <= max(TOL[d], nerr(ref, exact))


ROPE = [(1, 14, 2, 64, 0, 1e6), (1, 14, 2, 64, 4095, 1e6), (5, 12, 2, 128, 30000, 1e6), (3, 4, 4, 32, 7, 1e4)]


@pytest.mark.parametrize("d", [F32, F16])
@pytest.mark.parametrize("S,H,KVH,D,pos,theta", ROPE)
def test_rope(gpu, oracle, S, H, KVH, D, pos, theta, d):
    print(f"[case] rope S={S} H={H} KVH={KVH} D={D} pos={pos} dtype={d}", flush=True)
    rng = np.random.default_rng(pos + S)
    dq, q = up(rng.normal(0, 1, (S, H, D)), d)
    dk, k = up(rng.normal(0, 1, (S, KVH, D)), d)
    capi.call("vvh_rope", dq.ptr, dk.ptr, S, H, KVH, D, pos, theta, d, None)
    capi.sync()
    rq, rk = oracle.rope(q, k, pos, theta)
    assert nerr(down(dq, d, (S, H, D)), rq) <= TOL[d]
    assert nerr(down(dk, d, (S, KVH, D)), rk) <= TOL[d]


@pytest.mark.parametrize("d", [F32, F16])
def test_embedding(gpu, d):
    V, Hd = 1000, 896
    table, dt = mirror(np.random.default_rng(1).normal(0, 1, (V, Hd)))
    do = capi.DevBuf(Hd * 4)
    for tok in (0, 37, V - 1):
        capi.call("vvh_embedding", do.ptr, dt, tok, Hd, V, d, None)
        capi.sync()
        np.testing.assert_array_equal(down(do, d, (Hd,)), table[tok].astype(npd(d)).astype(np.float32))
    assert capi.status_of("vvh_embedding", do.ptr, dt, V, Hd, V, d, None) == 1  # token out of range
    capi.call("vvh_mirror_release", table.ctypes.data)


# n_q = 1 rows with head_dim % 8 == 0, head_dim <= 128 and <= 16 query heads
# per kv head take a decode kernel: fp16 with head_dim 64 or 128 the
# matrix-core one (one block of 4 waves up to 256 keys, of 8 waves up to 512,
# split blocks merged in the same launch beyond: one key, a one-key tail,
# 16 heads per kv head, spans of several chunks per wave), everything else
# the lane kernel (one chunk, two chunks with one key in the second, many
# chunks, a span beyond the general kernel's limit, blocks of several
# sub-chunks with a one-key tail, and head dims 8 to 40, whose merge blocks
# fold up to 64 groups of partials); the rest take the general kernel.
ATT = [(1, 1, 14, 2, 64), (1, 100, 14, 2, 64), (1, 256, 14, 2, 64), (1, 257, 14, 2, 64), (1, 4096, 14, 2, 64),
       (1, 1000, 32, 8, 128), (1, 700, 16, 1, 64), (1, 513, 12, 12, 40), (1, 40000, 2, 1, 64), (1, 20001, 4, 1, 64),
       (4, 10, 12, 2, 128), (3, 5, 4, 4, 32), (1, 16000, 2, 1, 64), (2, 7, 16, 2, 256), (1, 300, 4, 2, 256),
       (1, 300, 4, 2, 36), (1, 3000, 8, 2, 16), (1, 30000, 4, 1, 8), (1, 1200, 16, 4, 32), (1, 512, 14, 2, 64),
       (1, 450, 28, 4, 128), (1, 65, 12, 2, 128), (1, 513, 16, 1, 128)]


@pytest.mark.parametrize("d", [F32, F16])
@pytest.mark.parametrize("n_q,len0,H,KVH,D", ATT)
def test_attention(gpu, oracle, n_q, len0, H, KVH, D, d):
    print(f"[case] attention n_q={n_q} len0={len0} H={H} KVH={KVH} D={D} dtype={d}", flush=True)
    T = len0 + n_q - 1
    rng = np.random.default_rng(T + H)
    dq, q = up(rng.normal(0, 1, (n_q, H, D)), d)
    dk, k = up(rng.normal(0, 1, (T, KVH, D)), d)
    dv, v = up(rng.normal(0, 1, (T, KVH, D)), d)
    do = capi.DevBuf(n_q * H * D * np.dtype(npd(d)).itemsize)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    capi.call("vvh_attention", do.ptr, dq.ptr, dk.ptr, dv.ptr, n_q, len0, H, KVH, D, scale, d, None)
    capi.sync()
    got = down(do, d, (n_q, H * D))
    if not (n_q == 1 and D % 8 == 0 and D <= 128 and H // KVH <= 16):  # the general kernel's span limit
        assert capi.status_of("vvh_attention", do.ptr, dq.ptr, dk.ptr, dv.ptr, n_q, 16001, H, KVH, D, scale, d,
                              None) == 7
    for s in range(n_q):
        ref = oracle.causal_attention(q, k, v, s, len0 + s, scale)
        assert nerr(got[s], ref) <= TOL[d], f"query {s}"


@pytest.mark.parametrize("nbytes,off", [(256, 0), (4096 * 2, 0), (250, 0), (256, 2), (1, 0)])
def test_kv_append(gpu, nbytes, off):
    """The KV append's two copies in one launch: 16-byte chunks when every
    pointer and the size allow it, bytes otherwise; rows around the
    destination range stay untouched."""
    rng = np.random.default_rng(nbytes + off)
    k = rng.integers(0, 256, nbytes + 32, dtype=np.uint8)
    v = rng.integers(0, 256, nbytes + 32, dtype=np.uint8)
    dk, dv = capi.DevBuf.from_array(k), capi.DevBuf.from_array(v)
    kc0 = rng.integers(0, 256, 3 * nbytes + 64, dtype=np.uint8)
    vc0 = rng.integers(0, 256, 3 * nbytes + 64, dtype=np.uint8)
    kc, vc = capi.DevBuf.from_array(kc0), capi.DevBuf.from_array(vc0)
    at = nbytes + 16 + off
    capi.call("vvh_kv_append", kc.addr(at), vc.addr(at), dk.addr(off), dv.addr(off), nbytes, None)
    capi.sync()
    ek, ev = kc0.copy(), vc0.copy()
    ek[at:at + nbytes] = k[off:off + nbytes]
    ev[at:at + nbytes] = v[off:off + nbytes]
    np.testing.assert_array_equal(kc.to_array(np.uint8, ek.shape), ek)
    np.testing.assert_array_equal(vc.to_array(np.uint8, ev.shape), ev)
    assert capi.status_of("vvh_kv_append", kc.ptr, None, dk.ptr, dv.ptr, 16, None) == 1  # null pointer
    capi.call("vvh_kv_append", kc.ptr, vc.ptr, dk.ptr, dv.ptr, 0, None)  # nothing to copy


def test_attention_split_calls_in_a_row(gpu, oracle):
    """Split decode calls back to back on one stream, with different block
    counts: each merges its own partials (the per-kv-head arrival counters
    are back at zero after every call), the outputs match the oracle."""
    H, KVH, D = 14, 2, 64
    T = 9000
    rng = np.random.default_rng(11)
    dq, q = up(rng.normal(0, 1, (1, H, D)), F16)
    dk, k = up(rng.normal(0, 1, (T, KVH, D)), F16)
    dv, v = up(rng.normal(0, 1, (T, KVH, D)), F16)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    lens = (4096, 1500, 9000, 700, 4096)
    outs = [capi.DevBuf(H * D * 2) for _ in lens]
    for n, do in zip(lens, outs):
        print(f"[case] split attention len={n}", flush=True)
        capi.call("vvh_attention", do.ptr, dq.ptr, dk.ptr, dv.ptr, 1, n, H, KVH, D, scale, F16, None)
    capi.sync()
    for n, do in zip(lens, outs):
        ref = oracle.causal_attention(q, k, v, 0, n, scale)
        assert nerr(down(do, F16, (H * D,)), ref) <= TOL[F16], f"len {n}"


@pytest.mark.parametrize("d", [F32, F16])
def test_attention_unaligned_cache(gpu, oracle, d):
    """A k pointer off 16-byte alignment takes the general kernel; same results."""
    n, H, KVH, D = 300, 14, 2, 64
    es = np.dtype(npd(d)).itemsize
    rng = np.random.default_rng(5)
    dq, q = up(rng.normal(0, 1, (1, H, D)), d)
    kh = rng.normal(0, 1, (n, KVH, D)).astype(npd(d))
    dk = capi.DevBuf(kh.nbytes + 16)
    capi.call("vvh_memcpy_h2d", dk.addr(es), kh.ctypes.data, kh.nbytes)
    dv, v = up(rng.normal(0, 1, (n, KVH, D)), d)
    do = capi.DevBuf(H * D * es)
    scale = 1.0 / np.sqrt(D)
    capi.call("vvh_attention", do.ptr, dq.ptr, dk.addr(es), dv.ptr, 1, n, H, KVH, D, scale, d, None)
    capi.sync()
    ref = oracle.causal_attention(q, kh.astype(np.float32), v, 0, n, scale)
    assert nerr(down(do, d, (H * D,)), ref) <= TOL[d]


# K % 8 == 0 takes the 16-byte-load kernel (K = 8, K past one 2048-wide
# round of loads), K = 130 the element-wise one
DENSE = [(1, 896, 896), (3, 1000, 130), (7, 40, 4864), (1, 151936, 896), (2, 64, 8), (5, 300, 2056),
         # the streaming form (M <= 4, N >= 16384): a row tail (16390 % 16), a k tail
         # inside the last 128-byte step (904), a single step (64), M = 3 and 4
         (2, 16390, 904), (4, 20000, 64), (3, 16384, 1000)]


@pytest.mark.parametrize("d,wd", [(F32, F32), (F16, F16), (F16, F32), (F32, F16)])
@pytest.mark.parametrize("M,N,K", DENSE)
def test_dense(gpu, oracle, M, N, K, d, wd):
    print(f"[case] dense M={M} N={N} K={K} dtype={d} wdtype={wd}", flush=True)
    rng = np.random.default_rng(N + K + M)
    w = rng.normal(0, 0.05, (N, K)).astype(np.float32)
    wmir, dw = mirror(w, wd)
    weff = w.astype(np.float16).astype(np.float32) if wd == F16 else w  # what the device holds
    b, db = mirror(rng.normal(0, 0.1, N))
    dx, x = up(rng.normal(0, 1, (M, K)), d)
    res = M % 2 == 1
    dr, r = up(rng.normal(0, 1, (M, N)), d)
    do = capi.DevBuf(M * N * np.dtype(npd(d)).itemsize)
    capi.call("vvh_dense", do.ptr, dx.ptr, dw, wd, db, dr.ptr if res else None, M, N, K, d, None)
    capi.sync()
    ref = oracle.linear(x, weff, b, r if res else None)
    assert nerr(down(do, d, (M, N)), ref) <= TOL[d]
    for a in (wmir, b):
        capi.call("vvh_mirror_release", a.ctypes.data)


def test_dense_in_place_residual(gpu, oracle):
    """linear_add with out == residual (transformer.h:165-166 calls it so)."""
    M, N, K = 2, 64, 96
    rng = np.random.default_rng(9)
    w, dw = mirror(rng.normal(0, 0.1, (N, K)))
    dx, x = up(rng.normal(0, 1, (M, K)), F32)
    dr, r = up(rng.normal(0, 1, (M, N)), F32)
    capi.call("vvh_dense", dr.ptr, dx.ptr, dw, F32, None, dr.ptr, M, N, K, F32, None)
    capi.sync()
    assert nerr(down(dr, F32, (M, N)), oracle.linear(x, w, None, r)) <= TOL[F32]
    capi.call("vvh_mirror_release", w.ctypes.data)


@pytest.mark.parametrize("d", [F32, F16])
def test_matmul(gpu, oracle, d):
    rng = np.random.default_rng(4)
    dA, A = up(rng.normal(0, 1, (5, 70)), d)
    B, dB = mirror(rng.normal(0, 1, (70, 33)))
    do = capi.DevBuf(5 * 33 * 4)
    capi.call("vvh_matmul", do.ptr, dA.ptr, dB, 5, 33, 70, d, None)
    capi.sync()
    assert nerr(down(do, d, (5, 33)), oracle.matmul(A, B)) <= TOL[d]
    capi.call("vvh_mirror_release", B.ctypes.data)


def test_argmax(gpu):
    rng = np.random.default_rng(5)
    di = capi.DevBuf(4)
    # one block (n <= 2048), a second block of one element, many blocks, and
    # more than 1024 blocks' worth (blocks then take more than 2048 each)
    for n in (1, 1000, 2048, 2049, 151936, 5_000_001):
        x = rng.normal(0, 1, n).astype(np.float32)
        cases = [x]
        if n > 10:
            t = x.copy()
            t[[3, n - 2, n // 2]] = 50.0  # ties across blocks: the first index wins, as std::max_element
            cases.append(t)
            t = x.copy()
            t[-1] = 60.0  # the maximum in the last element
            cases.append(t)
            cases.append(np.full(n, -np.inf, np.float32))  # all equal: index 0
        for a in cases:
            dx = capi.DevBuf.from_array(a)
            capi.call("vvh_argmax", dx.ptr, n, di.ptr, None)
            capi.sync()
            assert int(di.to_array(np.int32, (1,))[0]) == int(np.argmax(a))


def test_mirror_f32_and_f16(gpu):
    a = np.random.default_rng(6).normal(0, 1, 1001).astype(np.float32)
    _, d32 = mirror(a, F32)
    _, d16 = mirror(a, F16)
    b32 = np.empty(1001, np.float32)
    b16 = np.empty(1001, np.float16)
    capi.call("vvh_memcpy_d2h", b32.ctypes.data, d32, 1001 * 4)
    capi.call("vvh_memcpy_d2h", b16.ctypes.data, d16, 1001 * 2)
    np.testing.assert_array_equal(b32, a)
    np.testing.assert_array_equal(b16, a.astype(np.float16))
    _, again = mirror(a, F32)
    assert again == d32  # same host array, same length: the cached copy
    capi.call("vvh_mirror_release", a.ctypes.data)
    assert capi.status_of("vvh_mirror_release", a.ctypes.data) == 6
