"""End-to-end decode steps on the GPU (vvllm_amd.qwen2_decode) against a CPU
forward pass built from the oracle's operators in the order of
transformer_forward (include/vvllm/model/transformer.h:126-189).

In fp16 mode the CPU forward rounds every activation to fp16 where the device
stores one, so both sides see the same data flow.  Logits are compared with a
normalized max error (fp32: 1e-3, fp16: 2e-2, over every layer of the step),
and the greedy token must match whenever the top-two margin of the CPU logits
is wider than that error.
"""
import numpy as np
import pytest

from vvllm_amd import capi
from vvllm_amd import qwen2_decode as qd

pytestmark = pytest.mark.gpu

TOL = {capi.F32: 1e-3, capi.F16: 2e-2}


def cpu_step(oracle, W, cfg, token, pos, cache, fp16, int8_head):
    r = (lambda a: a.astype(np.float16).astype(np.float32)) if fp16 else (lambda a: np.asarray(a, np.float32))
    H, KVH, D, I = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.inter
    scale = float(1.0 / np.sqrt(np.float32(D)))
    x = r(W["table"][token])
    for l, L in enumerate(W["layers"]):
        n = r(oracle.rms_norm(x[None], L["ln1"], cfg.eps))
        q = r(oracle.linear_q8(n, L["q"][0], L["q"][1], L["q"][2]))
        k = r(oracle.linear_q8(n, L["k"][0], L["k"][1], L["k"][2]))
        v = r(oracle.linear_q8(n, L["v"][0], L["v"][1], L["v"][2]))
        q3, k3 = oracle.rope(q.reshape(1, H, D), k.reshape(1, KVH, D), pos, cfg.theta)
        q, k = r(q3), r(k3)
        cache[l][0][pos], cache[l][1][pos] = k.ravel(), v.ravel()
        kc = cache[l][0][: pos + 1].reshape(pos + 1, KVH, D)
        vc = cache[l][1][: pos + 1].reshape(pos + 1, KVH, D)
        attn = r(oracle.causal_attention(q, kc, vc, 0, pos + 1, scale))
        x = r(oracle.linear_q8(attn[None], L["o"][0], L["o"][1], None, x[None]))[0]
        n = r(oracle.rms_norm(x[None], L["ln2"], cfg.eps))
        gu = r(oracle.linear_q8(n, L["gu"][0], L["gu"][1]))[0]
        g = r(oracle.eltwise("silu_mul", gu[:I], gu[I:]))
        x = r(oracle.linear_q8(g[None], L["down"][0], L["down"][1], None, x[None]))[0]
    f = r(oracle.rms_norm(x[None], W["final_norm"], cfg.eps))
    if int8_head:
        return oracle.linear_q8(f, W["head"][0], W["head"][1])[0]
    table = W["table"].astype(np.float16).astype(np.float32) if fp16 else W["table"]
    return r(oracle.linear(f, table)[0])


def run(oracle, cfg, act, head, steps, max_ctx, first=3):
    m = qd.Model(cfg, act=act, lm_head=head, max_ctx=max_ctx, seed=11)
    try:
        W = m.host_weights()
        cache = [(np.zeros((max_ctx, cfg.kv_dim), np.float32), np.zeros((max_ctx, cfg.kv_dim), np.float32))
                 for _ in range(cfg.layers)]
        tok = first
        for pos in range(steps):
            print(f"[case] decode {cfg.hidden}x{cfg.layers} act={act} head={head} pos={pos}", flush=True)
            m.step(tok, pos)
            got = m.logits_host()
            nxt = m.next_token()
            ref = cpu_step(oracle, W, cfg, tok, pos, cache, act == capi.F16, head == "int8")
            err = float(np.abs(got - ref).max() / np.abs(ref).max())
            assert err <= TOL[act], f"pos {pos}: normalized logits error {err:.2e}"
            top2 = np.sort(ref)[-2:]
            if top2[1] - top2[0] > 2 * err * np.abs(ref).max():
                assert nxt == int(np.argmax(ref)), f"pos {pos}: greedy token differs"
            assert nxt == int(np.argmax(got))
            tok = nxt  # both sides continue from the device's token
    finally:
        m.close()


SMALL = qd.Config(hidden=128, heads=4, kv_heads=2, inter=256, layers=2, vocab=512)


@pytest.mark.parametrize("head", ["dense", "int8"])
@pytest.mark.parametrize("act", [capi.F32, capi.F16], ids=["f32", "f16"])
def test_decode_small_model(gpu, oracle, act, head):
    run(oracle, SMALL, act, head, steps=12, max_ctx=32)


@pytest.mark.parametrize("head", ["dense", "int8"])
def test_decode_qwen25_05b_shapes(gpu, oracle, head):
    """Two steps at the real Qwen2.5-0.5B shapes (24 layers, vocab 151936)."""
    run(oracle, qd.QWEN25_05B, capi.F16, head, steps=2, max_ctx=16)


@pytest.mark.parametrize("P", [511, 700])
@pytest.mark.parametrize("fused", [False, True], ids=["unfused", "fused"])
def test_decode_late_position(gpu, oracle, fused, P):
    """One step at a late position of a filled KV cache, Qwen2.5-0.5B shapes:
    511 as bench.py times it (512 keys: the MFMA decode attention with one
    8-wave block per kv head, 8 chunks of 64 keys) and 700 (11 chunks: the
    span split over several blocks per kv head, merged in the same launch by
    the last block to arrive), which the short steps above never reach.  The
    cache rows the step reads are copied back from the device, so the CPU
    forward attends to the same context."""
    cfg, max_ctx = qd.QWEN25_05B, 1024
    m = qd.Model(cfg, act=capi.F16, lm_head="int8", max_ctx=max_ctx, seed=13, fused=fused)
    try:
        m.fill_kv(5)
        capi.sync()
        W = m.host_weights()
        cache = [(L["kc"].to_array(np.float16, (max_ctx, cfg.kv_dim)).astype(np.float32),
                  L["vc"].to_array(np.float16, (max_ctx, cfg.kv_dim)).astype(np.float32)) for L in m.layers]
        print(f"[case] decode late position {P} fused={fused}", flush=True)
        m.step(3, P)
        got = m.logits_host()
        ref = cpu_step(oracle, W, cfg, 3, P, cache, True, True)
        err = float(np.abs(got - ref).max() / np.abs(ref).max())
        assert err <= TOL[capi.F16], f"pos {P}: normalized logits error {err:.2e}"
    finally:
        m.close()
