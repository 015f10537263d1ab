"""The fused decode operators against the unfused sequences they replace.

vvh_linear_q8_dev_in (RMSNorm or SiLU-mul as the input stage of a decode
linear), vvh_plan_set_input_op (the same for a grouped q/k/v plan) and
vvh_rope_append (RoPE writing the KV-cache rows) and vvh_attention_parts +
vvh_linear_q8_dev_attn (attention merged in the o projection's input stage)
compute exactly what the reference's separate calls compute (transformer.h:133-160, 176-185): rms_norm
then linear, silu_mul then linear, rope then KVCache::append.  Each stage
rounds as the standalone kernel, so every comparison here is bit-exact; the
standalone kernels themselves are checked against the oracle in
test_gpu_ops.py and test_gpu_parity.py.  Whole decode steps of the fused
harness must reproduce the unfused step's logits exactly.
"""
import contextlib
import ctypes

import numpy as np
import pytest

from vvllm_amd import capi
from vvllm_amd import qwen2_decode as qd

pytestmark = pytest.mark.gpu
F16, F32 = capi.F16, capi.F32


@contextlib.contextmanager
def dot_kernel():
    """The unfused reference on k_dot, the family the input stages run on
    (automatic dispatch takes it only up to M = 2)."""
    capi.set_kernel(capi.KERNEL_DOT)
    try:
        yield
    finally:
        capi.set_kernel(capi.KERNEL_AUTO)


def q8_weight(rng, N, K):
    q = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = (rng.random(N, dtype=np.float32) * 0.02 + 0.001).astype(np.float32)
    return capi.DevBuf.from_array(q), capi.DevBuf.from_array(s)


@pytest.mark.parametrize("M,N,K", [(1, 896, 896), (2, 130, 896), (4, 64, 1536), (1, 9728, 896), (3, 17, 4864),
                                   (1, 640, 4864)])
def test_rms_norm_stage(gpu, M, N, K):
    print(f"[case] rms_norm stage M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + N + K)
    x = rng.normal(0, 3, (M, K)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    res = rng.normal(0, 1, (M, N)).astype(np.float16)
    dq, ds = q8_weight(rng, N, K)
    dx, dw, db = capi.DevBuf.from_array(x), capi.DevBuf.from_array(w), capi.DevBuf.from_array(bias)
    dn = capi.DevBuf(M * K * 2)
    ref, got = capi.DevBuf.from_array(res), capi.DevBuf.from_array(res)
    eps = 1e-6
    capi.call("vvh_rms_norm", dn.ptr, dx.ptr, dw.ptr, M, K, eps, F16, None)
    with dot_kernel():  # the stage runs on k_dot: compare with the same family
        capi.call("vvh_linear_q8_dev", ref.ptr, dn.ptr, dq.ptr, ds.ptr, db.ptr, ref.ptr, M, N, K, F16, F16, None)
    capi.call("vvh_linear_q8_dev_in", got.ptr, dx.ptr, dq.ptr, ds.ptr, db.ptr, got.ptr, M, N, K, F16, F16,
              capi.IN_RMS_NORM, dw.ptr, eps, None)
    a, b = ref.to_array(np.float16, (M, N)), got.to_array(np.float16, (M, N))
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), float(np.abs(a.astype(np.float32) - b).max())


@pytest.mark.parametrize("M,N,K", [(1, 896, 4864), (2, 100, 4864), (3, 64, 896), (4, 48, 2048)])
@pytest.mark.parametrize("outd", [F16, F32])
def test_silu_mul_stage(gpu, M, N, K, outd):
    print(f"[case] silu_mul stage M={M} N={N} K={K} out={outd}", flush=True)
    rng = np.random.default_rng(M + N + K + outd)
    gu = rng.normal(0, 2, (M, 2 * K)).astype(np.float16)
    dq, ds = q8_weight(rng, N, K)
    dgu = capi.DevBuf.from_array(gu)
    ob = 2 if outd == F16 else 4
    dg = capi.DevBuf(M * K * 2)
    ref, got = capi.DevBuf(M * N * ob), capi.DevBuf(M * N * ob)
    for m in range(M):  # the standalone operator, row by row as the model calls it
        capi.call("vvh_eltwise", capi.OP_SILU_MUL, dg.addr(m * K * 2), dgu.addr(m * 4 * K), dgu.addr(m * 4 * K + 2 * K),
                  K, F16, None)
    with dot_kernel():
        capi.call("vvh_linear_q8_dev", ref.ptr, dg.ptr, dq.ptr, ds.ptr, None, None, M, N, K, F16, outd, None)
    capi.call("vvh_linear_q8_dev_in", got.ptr, dgu.ptr, dq.ptr, ds.ptr, None, None, M, N, K, F16, outd,
              capi.IN_SILU_MUL, None, 0.0, None)
    u = np.uint16 if outd == F16 else np.uint32
    assert np.array_equal(ref.to_array(u, (M, N)), got.to_array(u, (M, N)))


def test_input_stage_limits(gpu):
    """Shapes the stage cannot serve are refused, never computed another way."""
    rng = np.random.default_rng(5)
    dq, ds = q8_weight(rng, 64, 896)
    dx, dw, out = capi.DevBuf(8 * 896 * 4), capi.DevBuf(896 * 4 + 16), capi.DevBuf(8 * 64 * 4)
    unsupported, invalid = 7, 1

    def st(M, act, in_op, w, K=896):
        return capi.status_of("vvh_linear_q8_dev_in", out.ptr, dx.ptr, dq.ptr, ds.ptr, None, None, M, 64, K, act,
                              act, in_op, w, 1e-6, None)
    assert st(5, F16, capi.IN_RMS_NORM, dw.ptr) == unsupported       # M > 4
    assert st(1, F32, capi.IN_RMS_NORM, dw.ptr) == unsupported       # fp32 activations
    assert st(1, F16, capi.IN_RMS_NORM, dw.ptr + 4) == invalid       # misaligned norm weights
    assert st(1, F16, capi.IN_RMS_NORM, None) == invalid             # no norm weights
    assert st(1, F16, 3, dw.ptr) == invalid                          # unknown stage
    assert st(1, F16, capi.IN_RMS_NORM, dw.ptr, K=888) == unsupported  # K % 16 != 0


@pytest.mark.parametrize("S,pos", [(1, 0), (1, 37), (3, 5)])
@pytest.mark.parametrize("act", [F16, F32], ids=["f16", "f32"])
def test_rope_append(gpu, S, pos, act):
    print(f"[case] rope_append S={S} pos={pos} act={act}", flush=True)
    H, KVH, D, cap = 14, 2, 64, 48
    dt = np.float16 if act == F16 else np.float32
    rng = np.random.default_rng(S * 100 + pos + act)
    q = rng.normal(0, 1, (S, H, D)).astype(dt)
    k = rng.normal(0, 1, (S, KVH, D)).astype(dt)
    v = rng.normal(0, 1, (S, KVH, D)).astype(dt)
    cache = rng.normal(0, 1, (cap, KVH, D)).astype(dt)
    es = np.dtype(dt).itemsize
    row = KVH * D * es
    # unfused: rope in place, then copy the rows into the caches
    q1, k1, v1 = (capi.DevBuf.from_array(a) for a in (q, k, v))
    kc1, vc1 = capi.DevBuf.from_array(cache), capi.DevBuf.from_array(cache)
    capi.call("vvh_rope", q1.ptr, k1.ptr, S, H, KVH, D, pos, 1e6, act, None)
    capi.call("vvh_memcpy_d2d_async", kc1.addr(pos * row), k1.ptr, S * row, None)
    capi.call("vvh_memcpy_d2d_async", vc1.addr(pos * row), v1.ptr, S * row, None)
    # fused
    q2, k2, v2 = (capi.DevBuf.from_array(a) for a in (q, k, v))
    kc2, vc2 = capi.DevBuf.from_array(cache), capi.DevBuf.from_array(cache)
    capi.call("vvh_rope_append", q2.ptr, k2.ptr, v2.ptr, kc2.ptr, vc2.ptr, S, H, KVH, D, pos, 1e6, act, None)
    u = np.uint16 if act == F16 else np.uint32
    for a, b, shape in ((q1, q2, q.shape), (k1, k2, k.shape), (kc1, kc2, cache.shape), (vc1, vc2, cache.shape)):
        assert np.array_equal(a.to_array(u, shape), b.to_array(u, shape))


def test_plan_input_stage(gpu):
    """q/k/v as one grouped launch reading rms_norm(x) through the plan's
    input stage: equal to the plan over the normed rows."""
    rng = np.random.default_rng(9)
    K = 896
    x = rng.normal(0, 2, (1, K)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    dx, dw, dn = capi.DevBuf.from_array(x), capi.DevBuf.from_array(w), capi.DevBuf(K * 2)
    capi.call("vvh_rms_norm", dn.ptr, dx.ptr, dw.ptr, 1, K, 1e-6, F16, None)
    shapes = [896, 128, 128]
    ws = [q8_weight(rng, N, K) for N in shapes]
    outs = {}
    for name, src in (("ref", dn), ("fused", dx)):
        bufs = [capi.DevBuf(N * 2) for N in shapes]
        probs = [capi.Q8Problem(out=b.ptr, inp=src.ptr, residual=None, weight=q.ptr, scales=s.ptr, bias=None,
                                M=1, N=N, K=K) for b, (q, s), N in zip(bufs, ws, shapes)]
        h = ctypes.c_uint64()
        capi.call("vvh_plan_create", (capi.Q8Problem * 3)(*probs), 3, F16, F16, ctypes.byref(h))
        try:
            if name == "fused":
                capi.call("vvh_plan_set_input_op", h.value, capi.IN_RMS_NORM, dw.ptr, 1e-6)
            capi.call("vvh_plan_run", h.value, None)
            outs[name] = [b.to_array(np.uint16, (N,)) for b, N in zip(bufs, shapes)]
        finally:
            capi.call("vvh_plan_destroy", h.value)
    for a, b in zip(outs["ref"], outs["fused"]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("M,inter,K,bias,outd,stage", [(1, 4864, 896, False, F16, True), (1, 136, 256, True, F16, False),
                                                        (3, 512, 896, True, F32, True), (4, 8, 1536, False, F16, False),
                                                        (2, 8960, 1536, False, F16, True),
                                                        (6, 512, 896, True, F16, False), (8, 72, 2048, False, F32, False),
                                                        # 17 tiles with the stage: the last block's idle tiles
                                                        (1, 136, 256, True, F16, True), (2, 40, 512, True, F32, True)])
def test_plan_glu_epilogue(gpu, M, inter, K, bias, outd, stage):
    """gate/up as a plan with the SiLU-gated epilogue (and the RMSNorm input
    stage): bit for bit the plain plan's [gate | up] rows through
    vvh_eltwise(SILU_MUL)."""
    print(f"[case] glu epilogue M={M} inter={inter} K={K} bias={bias} outd={outd} stage={stage}", flush=True)
    rng = np.random.default_rng(M + inter + K)
    N = 2 * inter
    x = rng.normal(0, 2, (M, K)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    q, s = q8_weight(rng, N, K)
    b = capi.DevBuf.from_array(rng.normal(0, 0.1, N).astype(np.float32)) if bias else None
    dx, dw = capi.DevBuf.from_array(x), capi.DevBuf.from_array(w)
    es = 2 if outd == F16 else 4
    full, ref, got = capi.DevBuf(M * N * es), capi.DevBuf(M * inter * es), capi.DevBuf(M * inter * es)

    def plan(out, glu):
        pr = capi.Q8Problem(out=out.ptr, inp=dx.ptr, residual=None, weight=q.ptr, scales=s.ptr,
                            bias=b.ptr if b else None, M=M, N=N, K=K)
        h = ctypes.c_uint64()
        with dot_kernel():  # several rows with many tiles would take k_skinny
            capi.call("vvh_plan_create", (capi.Q8Problem * 1)(pr), 1, F16, outd, ctypes.byref(h))
        kern = ctypes.c_int()
        capi.call("vvh_plan_kernel", h.value, ctypes.byref(kern))
        assert kern.value == capi.KERNEL_DOT
        if stage:
            capi.call("vvh_plan_set_input_op", h.value, capi.IN_RMS_NORM, dw.ptr, 1e-6)
        if glu:
            capi.call("vvh_plan_set_glu", h.value, 0)
        capi.call("vvh_plan_run", h.value, None)
        capi.call("vvh_plan_destroy", h.value)

    plan(full, False)
    for m in range(M):  # row m of the plain plan: [gate | up] of inter each
        capi.call("vvh_eltwise", capi.OP_SILU_MUL, ref.addr(m * inter * es), full.addr(m * N * es),
                  full.addr((m * N + inter) * es), inter, outd, None)
    plan(got, True)
    capi.sync()
    u = np.uint16 if outd == F16 else np.uint32
    assert np.array_equal(ref.to_array(u, (M, inter)), got.to_array(u, (M, inter)))


def test_plan_glu_limits(gpu):
    rng = np.random.default_rng(4)
    K = 256
    x, y = capi.DevBuf(K * 2), capi.DevBuf(64 * 2)
    q, s = q8_weight(rng, 40, K)

    def status(N, res=False, rope=False):
        pr = capi.Q8Problem(out=y.ptr, inp=x.ptr, residual=y.ptr if res else None, weight=q.ptr, scales=s.ptr,
                            bias=None, M=1, N=N, K=K)
        h = ctypes.c_uint64()
        capi.call("vvh_plan_create", (capi.Q8Problem * 1)(pr), 1, F16, F16, ctypes.byref(h))
        try:
            return capi.status_of("vvh_plan_set_glu", h.value, 0), capi.status_of("vvh_plan_set_glu", h.value, 5)
        finally:
            capi.call("vvh_plan_destroy", h.value)

    assert status(32) == (0, 1)    # index 5 names no problem
    assert status(40)[0] == 7      # inter % 8 != 0
    assert status(32, res=True)[0] == 1


def _qkv_plan(bufs, src, ws, M, K, outd):
    probs = [capi.Q8Problem(out=b.ptr, inp=src.ptr, residual=None, weight=q.ptr, scales=s.ptr, bias=bb.ptr,
                            M=M, N=N, K=K) for b, (q, s, bb, N) in zip(bufs, ws)]
    h = ctypes.c_uint64()
    capi.call("vvh_plan_create", (capi.Q8Problem * 3)(*probs), 3, F16, outd, ctypes.byref(h))
    assert capi.plan_kernel(h.value) == "dot"
    return h.value


# tab: positions of the plan's cosine/sine table (vvh_plan_set_rope_table;
# 0 = not called, the table holds position 0 only); runs whose rows all fall
# inside it read the table, the others work the values out
@pytest.mark.parametrize("M,H,KVH,D,pos,outd,stage,tab", [
    (1, 14, 2, 64, 511, F16, True, 2048),  # Qwen2.5-0.5B, as the fused decode step runs it
    (1, 14, 2, 64, 511, F16, True, 0),
    (1, 14, 2, 64, 0, F16, False, 0),      # position 0: the default table
    (2, 4, 4, 128, 37, F16, True, 38),     # two positions in one run, MHA, head_dim 128; row 1 past the table
    (1, 8, 2, 32, 1000, F32, False, 1001),  # fp32 outputs and caches, head_dim 32; the table's last position
    (2, 12, 2, 128, 5, F32, True, 7),
    (5, 4, 2, 64, 100, F16, False, 4096),  # 5-8 rows: the MFMA dot path's 8-row operands
    (8, 8, 2, 128, 3, F32, False, 11),
    (8, 8, 2, 128, 3, F32, False, 0),
    (1, 3, 1, 32, 9, F16, True, 0),        # head_dim 32 and 48: tile counts that leave idle tiles in the last block
    (1, 5, 1, 48, 3, F16, True, 64),
])
def test_plan_rope_epilogue(gpu, M, H, KVH, D, pos, outd, stage, tab):
    """RoPE and the K/V cache append as the epilogue of the q/k/v plan
    (vvh_plan_set_rope, vvh_plan_run_pos) against the plan's plain run
    followed by vvh_rope_append, bit for bit: q, k, v and both caches."""
    print(f"[case] plan rope M={M} H={H} KVH={KVH} D={D} pos={pos} out={outd} stage={stage} tab={tab}", flush=True)
    rng = np.random.default_rng(M * 1000 + H * 10 + D + pos)
    K, theta, eps, cap = 896, 1e6, 1e-6, pos + M + 3
    dt = np.float16 if outd == F16 else np.float32
    x = rng.normal(0, 2, (M, K)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    dx, dw = capi.DevBuf.from_array(x), capi.DevBuf.from_array(w)
    shapes = [H * D, KVH * D, KVH * D]
    ws = []
    for N in shapes:
        q, s = q8_weight(rng, N, K)
        ws.append((q, s, capi.DevBuf.from_array(rng.normal(0, 0.1, N).astype(np.float32)), N))
    cache = rng.normal(0, 1, (cap, KVH * D)).astype(dt)
    results = {}
    for mode in ("ref", "fused"):
        bufs = [capi.DevBuf(M * N * np.dtype(dt).itemsize) for N in shapes]
        kc, vc = capi.DevBuf.from_array(cache), capi.DevBuf.from_array(cache)
        h = _qkv_plan(bufs, dx, ws, M, K, outd)
        try:
            if stage:
                capi.call("vvh_plan_set_input_op", h, capi.IN_RMS_NORM, dw.ptr, eps)
            if mode == "ref":
                capi.call("vvh_plan_run", h, None)
                capi.call("vvh_rope_append", bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, kc.ptr, vc.ptr, M, H, KVH, D, pos,
                          theta, outd, None)
            else:
                capi.call("vvh_plan_set_rope", h, 0, 1, 2, D, theta, kc.ptr, vc.ptr)
                if tab:
                    capi.call("vvh_plan_set_rope_table", h, tab)
                capi.call("vvh_plan_run_pos", h, pos, None)
            capi.sync()
        finally:
            capi.call("vvh_plan_destroy", h)
        u = np.uint16 if outd == F16 else np.uint32
        results[mode] = [b.to_array(u, (M * N,)) for b, N in zip(bufs, shapes)] + \
                        [kc.to_array(u, cache.shape), vc.to_array(u, cache.shape)]
    for name, a, b in zip(("q", "k", "v", "k_cache", "v_cache"), results["ref"], results["fused"]):
        assert np.array_equal(a, b), name


def test_plan_rope_table_replaced(gpu):
    """A table set, then the epilogue set again (the table back to position
    0), then a longer table: each run equals the plain run + vvh_rope_append,
    and runs read whichever table the plan holds at the time."""
    print("[case] plan rope table replaced", flush=True)
    rng = np.random.default_rng(17)
    M, H, KVH, D, K, theta = 1, 4, 2, 64, 256, 1e4
    x = rng.normal(0, 1, (M, K)).astype(np.float16)
    dx = capi.DevBuf.from_array(x)
    shapes = [H * D, KVH * D, KVH * D]
    ws = []
    for N in shapes:
        q, s = q8_weight(rng, N, K)
        ws.append((q, s, capi.DevBuf.from_array(rng.normal(0, 0.1, N).astype(np.float32)), N))
    cap = 300
    cache = rng.normal(0, 1, (cap, KVH * D)).astype(np.float16)
    ref_b = [capi.DevBuf(M * N * 2) for N in shapes]
    ref_kc, ref_vc = capi.DevBuf.from_array(cache), capi.DevBuf.from_array(cache)
    hr = _qkv_plan(ref_b, dx, ws, M, K, F16)
    bufs = [capi.DevBuf(M * N * 2) for N in shapes]
    kc, vc = capi.DevBuf.from_array(cache), capi.DevBuf.from_array(cache)
    h = _qkv_plan(bufs, dx, ws, M, K, F16)
    try:
        capi.call("vvh_plan_set_rope", h, 0, 1, 2, D, theta, kc.ptr, vc.ptr)
        capi.call("vvh_plan_set_rope_table", h, 64)
        # steps: (what to set before the run, position)
        for setup, pos in ((None, 10), ("rope", 10), ("rope", 0), ("table", 200), (None, 299), (None, 63)):
            if setup == "rope":
                capi.call("vvh_plan_set_rope", h, 0, 1, 2, D, theta, kc.ptr, vc.ptr)
            elif setup == "table":
                capi.call("vvh_plan_set_rope_table", h, 256)
            capi.call("vvh_plan_run", hr, None)
            capi.call("vvh_rope_append", ref_b[0].ptr, ref_b[1].ptr, ref_b[2].ptr, ref_kc.ptr, ref_vc.ptr, M, H, KVH,
                      D, pos, theta, F16, None)
            capi.call("vvh_plan_run_pos", h, pos, None)
            capi.sync()
            for name, a, b in zip(("q", "k", "v"), ref_b, bufs):
                assert np.array_equal(a.to_array(np.uint16, (a.nbytes // 2,)), b.to_array(np.uint16, (b.nbytes // 2,))), \
                    (setup, pos, name)
            for name, a, b in (("k_cache", ref_kc, kc), ("v_cache", ref_vc, vc)):
                assert np.array_equal(a.to_array(np.uint16, cache.shape), b.to_array(np.uint16, cache.shape)), \
                    (setup, pos, name)
    finally:
        capi.call("vvh_plan_destroy", h)
        capi.call("vvh_plan_destroy", hr)


def test_plan_rope_limits(gpu):
    """The RoPE epilogue is refused where it cannot apply."""
    rng = np.random.default_rng(3)
    K = 256
    dx = capi.DevBuf.from_array(rng.normal(0, 1, (1, K)).astype(np.float16))
    ws = [(*q8_weight(rng, N, K), capi.DevBuf(N * 4), N) for N in (128, 64, 64)]
    bufs = [capi.DevBuf(N * 2) for N in (128, 64, 64)]
    kc, vc = capi.DevBuf(64 * 2 * 4), capi.DevBuf(64 * 2 * 4)
    h = _qkv_plan(bufs, dx, ws, 1, K, F16)
    try:
        st = lambda *a: capi.status_of("vvh_plan_set_rope", h, *a)
        invalid, unsupported = 1, 7
        assert st(0, 1, 1, 32, 1e6, kc.ptr, vc.ptr) == invalid         # k and v the same problem
        assert st(0, 1, 5, 32, 1e6, kc.ptr, vc.ptr) == invalid         # no problem 5
        assert st(0, 1, 2, 24, 1e6, kc.ptr, vc.ptr) == unsupported     # head_dim % 16 != 0
        assert st(0, 1, 2, 48, 1e6, kc.ptr, vc.ptr) == invalid         # 128 rows are not whole heads of 48
        assert st(0, 1, 2, 32, 0.0, kc.ptr, vc.ptr) == invalid         # theta
        assert st(0, 1, 2, 32, 1e6, None, vc.ptr) == invalid           # no cache
        tab = lambda n: capi.status_of("vvh_plan_set_rope_table", h, n)
        assert tab(16) == invalid                                      # no RoPE epilogue yet
        assert st(0, 1, 2, 32, 1e6, kc.ptr, vc.ptr) == 0
        assert tab(0) == invalid and tab((1 << 20) + 1) == invalid     # positions
        assert tab(16) == 0 and tab(1 << 20) == 0
    finally:
        capi.call("vvh_plan_destroy", h)


# (len0, H, KVH, D): spans of 1 to 512 keys (4 parts up to 256, else 8),
# grouped and plain heads, head_dim 64 and 128, K = H * D up to 1024
ATTN_PARTS_CASES = [(1, 14, 2, 64), (2, 14, 2, 64), (63, 14, 2, 64), (64, 14, 2, 64), (65, 14, 2, 64),
                    (200, 14, 2, 64), (256, 14, 2, 64), (257, 14, 2, 64), (511, 14, 2, 64), (512, 14, 2, 64),
                    (100, 4, 4, 128), (384, 8, 2, 128), (512, 16, 1, 64), (300, 8, 1, 128)]


@pytest.mark.parametrize("len0,H,KVH,D", ATTN_PARTS_CASES)
@pytest.mark.parametrize("outd", [F16, F32], ids=["f16out", "f32out"])
def test_attention_parts_o_projection(gpu, len0, H, KVH, D, outd):
    """vvh_attention_parts then vvh_linear_q8_dev_attn (o + bias + residual in
    place) against vvh_attention then vvh_linear_q8_dev on k_dot: the same
    bits."""
    print(f"[case] attention parts len0={len0} H={H} KVH={KVH} D={D} out={outd}", flush=True)
    rng = np.random.default_rng(len0 * 131 + H * 7 + D)
    K = N = H * D
    q = rng.normal(0, 1, (H, D)).astype(np.float16)
    kc = rng.normal(0, 1, (len0, KVH, D)).astype(np.float16)
    vc = rng.normal(0, 1, (len0, KVH, D)).astype(np.float16)
    dq, ds = q8_weight(rng, N, K)
    bias = capi.DevBuf.from_array(rng.normal(0, 0.1, N).astype(np.float32))
    res = rng.normal(0, 1, N).astype(np.float16 if outd == F16 else np.float32)
    dqv, dk, dv = capi.DevBuf.from_array(q), capi.DevBuf.from_array(kc), capi.DevBuf.from_array(vc)
    attn = capi.DevBuf(K * 2)
    ref, got = capi.DevBuf.from_array(res), capi.DevBuf.from_array(res)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    capi.call("vvh_attention", attn.ptr, dqv.ptr, dk.ptr, dv.ptr, 1, len0, H, KVH, D, scale, F16, None)
    with dot_kernel():
        capi.call("vvh_linear_q8_dev", ref.ptr, attn.ptr, dq.ptr, ds.ptr, bias.ptr, ref.ptr, 1, N, K, F16, outd, None)
    nf = 8 * H * (D + 4)
    parts = capi.DevBuf(nf * 4)
    n = ctypes.c_size_t()
    capi.call("vvh_attention_parts", parts.ptr, nf, ctypes.byref(n), dqv.ptr, dk.ptr, dv.ptr, len0, H, KVH, D,
              scale, F16, None)
    assert n.value == (4 if len0 <= 256 else 8)
    capi.call("vvh_linear_q8_dev_attn", got.ptr, parts.ptr, n.value, D, dq.ptr, ds.ptr, bias.ptr, got.ptr, N, K,
              outd, None)
    u = np.uint16 if outd == F16 else np.uint32
    a, b = ref.to_array(u, (N,)), got.to_array(u, (N,))
    assert np.array_equal(a, b), f"{int((a != b).sum())} of {N} outputs differ"


def test_attention_parts_limits(gpu):
    H, KVH, D = 14, 2, 64
    q, k, v = capi.DevBuf(H * D * 2), capi.DevBuf(600 * KVH * D * 2), capi.DevBuf(600 * KVH * D * 2)
    nf = 8 * H * (D + 4)
    parts = capi.DevBuf(nf * 4)
    n = ctypes.c_size_t()
    st = lambda *a: capi.status_of("vvh_attention_parts", *a)
    invalid, unsupported = 1, 7
    assert st(parts.ptr, nf, ctypes.byref(n), q.ptr, k.ptr, v.ptr, 513, H, KVH, D, 0.125, F16, None) == unsupported
    assert st(parts.ptr, nf, ctypes.byref(n), q.ptr, k.ptr, v.ptr, 100, H, KVH, D, 0.125, F32, None) == unsupported
    assert st(parts.ptr, nf, ctypes.byref(n), q.ptr, k.ptr, v.ptr, 100, 12, 2, 96, 0.125, F16, None) == unsupported
    assert st(parts.ptr, nf - 1, ctypes.byref(n), q.ptr, k.ptr, v.ptr, 300, H, KVH, D, 0.125, F16, None) == invalid
    assert st(parts.ptr, nf, None, q.ptr, k.ptr, v.ptr, 100, H, KVH, D, 0.125, F16, None) == invalid
    assert st(parts.ptr, nf, ctypes.byref(n), q.ptr, k.ptr, v.ptr, 0, H, KVH, D, 0.125, F16, None) == invalid
    assert st(parts.ptr, nf, ctypes.byref(n), q.ptr, k.ptr, v.ptr, 300, H, KVH, D, 0.125, F16, None) == 0
    assert n.value == 8
    rng = np.random.default_rng(5)
    dq, ds = q8_weight(rng, 896, 896)
    out = capi.DevBuf(896 * 2)
    so = lambda *a: capi.status_of("vvh_linear_q8_dev_attn", *a)
    assert so(out.ptr, parts.ptr, 0, D, dq.ptr, ds.ptr, None, None, 896, 896, F16, None) == invalid
    assert so(out.ptr, parts.ptr, 9, D, dq.ptr, ds.ptr, None, None, 896, 896, F16, None) == invalid
    assert so(out.ptr, parts.ptr, 8, 60, dq.ptr, ds.ptr, None, None, 896, 896, F16, None) == invalid
    assert so(out.ptr, parts.ptr, 8, 112, dq.ptr, ds.ptr, None, None, 896, 896, F16, None) == invalid  # not 2^n
    big_q, big_s = q8_weight(rng, 16, 1536)
    assert so(out.ptr, parts.ptr, 8, 64, big_q.ptr, big_s.ptr, None, None, 16, 1536, F16, None) == unsupported
    assert so(out.ptr, parts.ptr, 8, D, dq.ptr, ds.ptr, None, None, 896, 896, F16, None) == 0


def fused_vs_unfused(cfg, head, steps, max_ctx):
    models = [qd.Model(cfg, act=F16, lm_head=head, max_ctx=max_ctx, seed=11, fused=f) for f in (False, True)]
    try:
        assert models[1].calls_per_step() < models[0].calls_per_step()
        tok = 3
        for pos in range(steps):
            print(f"[case] fused step {cfg.hidden}x{cfg.layers} head={head} pos={pos}", flush=True)
            logits = []
            for m in models:
                m.step(tok, pos)
                logits.append(m.logits_host())
            assert np.array_equal(logits[0].view(np.uint32), logits[1].view(np.uint32)), \
                f"pos {pos}: max difference {float(np.abs(logits[0] - logits[1]).max()):.3e}"
            toks = [m.next_token() for m in models]
            assert toks[0] == toks[1]
            tok = toks[0]
    finally:
        for m in models:
            m.close()


@pytest.mark.parametrize("head", ["dense", "int8"])
def test_fused_step_small(gpu, head):
    fused_vs_unfused(qd.Config(hidden=128, heads=4, kv_heads=2, inter=256, layers=2, vocab=512), head, 10, 16)


@pytest.mark.parametrize("head", ["dense", "int8"])
def test_fused_step_qwen25_05b_shapes(gpu, head):
    fused_vs_unfused(qd.QWEN25_05B, head, 2, 8)


@pytest.mark.parametrize("P", [255, 256, 511, 600])
def test_fused_step_late_positions(gpu, P):
    """One step at a late position of a filled KV cache, Qwen2.5-0.5B shapes:
    spans of 256 and 512 keys take the attention parts merged in the o
    projection (4 and 8 parts), 257 the 8-part form with a short last chunk,
    601 vvh_attention (the span over several blocks); the logits equal the
    unfused step's bit for bit."""
    cfg, max_ctx = qd.QWEN25_05B, 1024
    models = [qd.Model(cfg, act=F16, lm_head="int8", max_ctx=max_ctx, seed=13, fused=f) for f in (False, True)]
    try:
        print(f"[case] fused step late position {P}", flush=True)
        logits = []
        for m in models:
            m.fill_kv(5)
            m.step(3, P)
            logits.append(m.logits_host())
        assert np.array_equal(logits[0].view(np.uint32), logits[1].view(np.uint32)), \
            f"max difference {float(np.abs(logits[0] - logits[1]).max()):.3e}"
    finally:
        for m in models:
            m.close()
