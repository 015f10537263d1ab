"""HIP graph capture of the int8 linear path, of the split decode attention
and of a whole fused decode step (launch-overhead removal by graph capture
of the decode step).

A decode plan, a several-row decode call, a GEMM and a split-K GEMM are
issued on one stream, captured into a graph and replayed several times, with
eager work and synchronisation between the replays.  Every replay must give
exactly the eager results: the kernels are deterministic and the captured
calls allocate nothing (the split-K workspace of the stream is grown by an
eager call before capture).
"""
import ctypes

import numpy as np
import pytest

from vvllm_amd import capi
from vvllm_amd import qwen2_decode as qd

pytestmark = pytest.mark.gpu

F16, F32 = capi.F16, capi.F32


def _hip():
    for name in ("libamdhip64.so.7", "libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
        try:
            return ctypes.CDLL(name)
        except OSError:
            continue
    raise OSError("libamdhip64 not found")


def _check(st, what):
    assert st == 0, f"{what} failed with hipError {st}"


def test_graph_replay_matches_eager(gpu, oracle):
    hip = _hip()
    V = ctypes.c_void_p
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(V)]
    hip.hipStreamSynchronize.argtypes = [V]
    hip.hipStreamBeginCapture.argtypes = [V, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [V, ctypes.POINTER(V)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(V), V, V, V, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [V, V]
    hip.hipGraphExecDestroy.argtypes = [V]
    hip.hipGraphDestroy.argtypes = [V]
    hip.hipStreamDestroy.argtypes = [V]
    stream = V()
    _check(hip.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")

    rng = np.random.default_rng(99)
    keep, outs = [], []

    def problem(M, N, K, bias):
        w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
        q, s = oracle.quantize_per_channel(w)
        x = rng.normal(0, 1, (M, K)).astype(np.float16)
        b = rng.normal(0, 0.01, N).astype(np.float32) if bias else None
        d = dict(q=capi.DevBuf.from_array(q), s=capi.DevBuf.from_array(s), x=capi.DevBuf.from_array(x),
                 b=capi.DevBuf.from_array(b) if bias else None, y=capi.DevBuf(M * N * 2), M=M, N=N, K=K)
        keep.append(d)
        outs.append(d)
        return d

    # a decode plan (M = 1, q/k/v-like), a 4-row decode call, a GEMM, a split-K GEMM
    plan_ds = [problem(1, 896, 896, True), problem(1, 128, 896, True), problem(1, 4864, 896, False)]
    probs = [capi.Q8Problem(out=d["y"].ptr, inp=d["x"].ptr, residual=None, weight=d["q"].ptr, scales=d["s"].ptr,
                            bias=d["b"].ptr if d["b"] else None, M=1, N=d["N"], K=d["K"]) for d in plan_ds]
    arr = (capi.Q8Problem * len(probs))(*probs)
    plan = ctypes.c_uint64()
    capi.call("vvh_plan_create", arr, len(probs), F16, F16, ctypes.byref(plan))
    singles = [problem(4, 896, 896, True), problem(64, 512, 896, False), problem(64, 896, 4864, False)]

    def issue():
        capi.call("vvh_plan_run", plan.value, stream)
        for d in singles:
            capi.call("vvh_linear_q8_dev", d["y"].ptr, d["x"].ptr, d["q"].ptr, d["s"].ptr,
                      d["b"].ptr if d["b"] else None, None, d["M"], d["N"], d["K"], F16, F16, stream)

    def results():
        return [d["y"].to_array(np.uint16, (d["M"], d["N"])) for d in outs]

    issue()  # eager (also grows the split-K workspace of this stream)
    _check(hip.hipStreamSynchronize(stream), "sync")
    eager = results()
    zero = np.zeros(max(d["M"] * d["N"] for d in outs), np.uint16)

    graph, gexec = V(), V()
    _check(hip.hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")
    issue()
    _check(hip.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
    _check(hip.hipGraphInstantiate(ctypes.byref(gexec), graph, None, None, 0), "hipGraphInstantiate")
    scratch = capi.DevBuf(4096 * 4)
    for rep in range(3):
        for d in outs:  # clear the outputs, so each replay must write them again
            capi.call("vvh_memcpy_h2d", d["y"].ptr, zero.ctypes.data, d["M"] * d["N"] * 2)
        capi.call("vvh_fill_normal", scratch.ptr, F32, 4096, rep, 0.0, 1.0, None)  # eager work between replays
        capi.sync()
        print(f"[case] graph replay {rep}", flush=True)
        _check(hip.hipGraphLaunch(gexec, stream), "hipGraphLaunch")
        _check(hip.hipStreamSynchronize(stream), "sync")
        for i, (a, b) in enumerate(zip(eager, results())):
            np.testing.assert_array_equal(a, b, err_msg=f"replay {rep}, output {i}")
    hip.hipGraphExecDestroy(gexec)
    hip.hipGraphDestroy(graph)
    capi.call("vvh_plan_destroy", plan.value)
    hip.hipStreamDestroy(stream)


def test_graph_survives_workspace_growth(gpu, oracle):
    """A graph captured with a split-K GEMM keeps working after a larger
    split-K call on the same stream has grown the stream's workspace: the
    outgrown buffer, whose address the graph holds, is kept, not freed."""
    hip = _hip()
    V = ctypes.c_void_p
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(V)]
    hip.hipStreamSynchronize.argtypes = [V]
    hip.hipStreamBeginCapture.argtypes = [V, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [V, ctypes.POINTER(V)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(V), V, V, V, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [V, V]
    hip.hipGraphExecDestroy.argtypes = [V]
    hip.hipGraphDestroy.argtypes = [V]
    hip.hipStreamDestroy.argtypes = [V]
    stream = V()
    _check(hip.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
    rng = np.random.default_rng(7)

    def problem(M, N, K):
        w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
        q, s = oracle.quantize_per_channel(w)
        x = rng.normal(0, 1, (M, K)).astype(np.float16)
        return dict(q=capi.DevBuf.from_array(q), s=capi.DevBuf.from_array(s), x=capi.DevBuf.from_array(x),
                    y=capi.DevBuf(M * N * 2), M=M, N=N, K=K)

    def run(d):
        capi.call("vvh_linear_q8_dev", d["y"].ptr, d["x"].ptr, d["q"].ptr, d["s"].ptr, None, None,
                  d["M"], d["N"], d["K"], F16, F16, stream)

    def out(d):
        return d["y"].to_array(np.uint16, (d["M"], d["N"]))

    small = problem(64, 896, 4864)   # split-K, a few MB of partial planes
    large = problem(512, 896, 4864)  # split-K, about 11 MB: grows the workspace
    assert "split" in capi.gemm_variant(64, 896, 4864) and "split" in capi.gemm_variant(512, 896, 4864)
    capi.call("vvh_workspace_release", stream)  # start from no workspace on this stream
    run(small)
    _check(hip.hipStreamSynchronize(stream), "sync")
    eager_small = out(small)
    graph, gexec = V(), V()
    _check(hip.hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")
    run(small)
    _check(hip.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
    _check(hip.hipGraphInstantiate(ctypes.byref(gexec), graph, None, None, 0), "hipGraphInstantiate")
    run(large)  # eager: grows the workspace past the captured buffer
    _check(hip.hipStreamSynchronize(stream), "sync")
    eager_large = out(large)
    zero = np.zeros(64 * 896, np.uint16)
    for rep in range(3):
        capi.call("vvh_memcpy_h2d", small["y"].ptr, zero.ctypes.data, zero.nbytes)
        print(f"[case] replay after workspace growth {rep}", flush=True)
        _check(hip.hipGraphLaunch(gexec, stream), "hipGraphLaunch")
        _check(hip.hipStreamSynchronize(stream), "sync")
        np.testing.assert_array_equal(out(small), eager_small, err_msg=f"replay {rep}")
        run(large)  # eager work on the grown workspace between replays
        _check(hip.hipStreamSynchronize(stream), "sync")
        np.testing.assert_array_equal(out(large), eager_large, err_msg=f"large after replay {rep}")
    hip.hipGraphExecDestroy(gexec)
    hip.hipGraphDestroy(graph)
    capi.call("vvh_workspace_release", stream)
    hip.hipStreamDestroy(stream)


def test_graph_split_attention(gpu, oracle):
    """Split decode attention (blocks merged in the same launch through
    per-kv-head arrival counters) captured into a graph and replayed, with
    eager split calls on the same stream between the replays: every replay
    matches the eager outputs bit for bit, so the counters are back at zero
    after every call, captured or not."""
    hip = _hip()
    V = ctypes.c_void_p
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(V)]
    hip.hipStreamSynchronize.argtypes = [V]
    hip.hipStreamBeginCapture.argtypes = [V, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [V, ctypes.POINTER(V)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(V), V, V, V, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [V, V]
    hip.hipGraphExecDestroy.argtypes = [V]
    hip.hipGraphDestroy.argtypes = [V]
    hip.hipStreamDestroy.argtypes = [V]
    stream = V()
    _check(hip.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
    H, KVH, D, T = 14, 2, 64, 6000
    rng = np.random.default_rng(21)
    q = capi.DevBuf.from_array(rng.normal(0, 1, (H, D)).astype(np.float16))
    k = capi.DevBuf.from_array(rng.normal(0, 1, (T, KVH, D)).astype(np.float16))
    v = capi.DevBuf.from_array(rng.normal(0, 1, (T, KVH, D)).astype(np.float16))
    scale = float(1.0 / np.sqrt(np.float32(D)))
    lens = (6000, 300, 2500)  # split, one block, split with fewer blocks
    outs = [capi.DevBuf(H * D * 2) for _ in lens]

    def issue(bufs):
        for n, o in zip(lens, bufs):
            capi.call("vvh_attention", o.ptr, q.ptr, k.ptr, v.ptr, 1, n, H, KVH, D, scale, F16, stream)

    issue(outs)  # eager: sizes the stream's workspace and sets up its counters
    _check(hip.hipStreamSynchronize(stream), "sync")
    eager = [o.to_array(np.uint16, (H * D,)) for o in outs]
    graph, gexec = V(), V()
    _check(hip.hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")
    issue(outs)
    _check(hip.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
    _check(hip.hipGraphInstantiate(ctypes.byref(gexec), graph, None, None, 0), "hipGraphInstantiate")
    others = [capi.DevBuf(H * D * 2) for _ in lens]
    zero = np.zeros(H * D, np.uint16)
    for rep in range(3):
        for o in outs:
            capi.call("vvh_memcpy_h2d", o.ptr, zero.ctypes.data, zero.nbytes)
        print(f"[case] split attention replay {rep}", flush=True)
        _check(hip.hipGraphLaunch(gexec, stream), "hipGraphLaunch")
        _check(hip.hipStreamSynchronize(stream), "sync")
        for i, (a, o) in enumerate(zip(eager, outs)):
            np.testing.assert_array_equal(o.to_array(np.uint16, (H * D,)), a, err_msg=f"replay {rep}, len {lens[i]}")
        issue(others)  # eager split calls between the replays
        _check(hip.hipStreamSynchronize(stream), "sync")
        for i, (a, o) in enumerate(zip(eager, others)):
            np.testing.assert_array_equal(o.to_array(np.uint16, (H * D,)), a, err_msg=f"eager {rep}, len {lens[i]}")
    hip.hipGraphExecDestroy(gexec)
    hip.hipGraphDestroy(graph)
    capi.call("vvh_workspace_release", stream)
    hip.hipStreamDestroy(stream)


@pytest.mark.parametrize("pos", [200, 511])
def test_graph_fused_decode_step(gpu, pos):
    """A whole fused decode step (RMSNorm stages, RoPE + cache epilogue, the
    attention as per-wave parts merged in the o projection, SiLU-gated
    epilogue), small Qwen2-shaped model, captured at one position and
    replayed three times with eager steps on the same stream between the
    replays: every replay's logits equal the eager step's bit for bit."""
    hip = _hip()
    V = ctypes.c_void_p
    for f, args in (("hipStreamCreate", [ctypes.POINTER(V)]), ("hipStreamSynchronize", [V]),
                    ("hipStreamBeginCapture", [V, ctypes.c_int]), ("hipStreamEndCapture", [V, ctypes.POINTER(V)]),
                    ("hipGraphInstantiate", [ctypes.POINTER(V), V, V, V, ctypes.c_size_t]),
                    ("hipGraphLaunch", [V, V]), ("hipGraphExecDestroy", [V]), ("hipGraphDestroy", [V]),
                    ("hipStreamDestroy", [V])):
        getattr(hip, f).argtypes = args
    stream = V()
    _check(hip.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
    cfg = qd.Config(hidden=512, heads=8, kv_heads=2, inter=1024, layers=2, vocab=2048)
    m = qd.Model(cfg, act=F16, lm_head="int8", max_ctx=pos + 1, seed=5, fused=True)
    try:
        m.fill_kv(9)
        print(f"[case] fused decode step graph at position {pos}", flush=True)
        m.step(3, pos, stream.value)  # eager: sizes the stream's workspace
        _check(hip.hipStreamSynchronize(stream), "sync")
        eager = m.logits_host().view(np.uint32).copy()
        graph, gexec = V(), V()
        _check(hip.hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")
        m.step(3, pos, stream.value)
        _check(hip.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
        _check(hip.hipGraphInstantiate(ctypes.byref(gexec), graph, None, None, 0), "hipGraphInstantiate")
        for rep in range(3):
            capi.call("vvh_fill_normal", m.logits32.ptr, F32, cfg.vocab, rep, 0.0, 1.0, stream.value)
            _check(hip.hipGraphLaunch(gexec, stream), "hipGraphLaunch")
            _check(hip.hipStreamSynchronize(stream), "sync")
            np.testing.assert_array_equal(m.logits_host().view(np.uint32), eager, err_msg=f"replay {rep}")
            m.step(3, pos, stream.value)  # an eager step between the replays
            _check(hip.hipStreamSynchronize(stream), "sync")
            np.testing.assert_array_equal(m.logits_host().view(np.uint32), eager, err_msg=f"eager {rep}")
        hip.hipGraphExecDestroy(gexec)
        hip.hipGraphDestroy(graph)
    finally:
        m.close()
        capi.call("vvh_workspace_release", stream.value)
        hip.hipStreamDestroy(stream)
