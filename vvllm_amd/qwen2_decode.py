"""A Qwen2-shaped decode step on one MI355X, issued over the C ABI.

One step is the operator sequence of transformer_forward
(include/vvllm/model/transformer.h:126-189) for one token:

    embedding (fp32) -> [fp16 conversion] ->
    per layer: rms_norm -> q/k/v (one grouped int8 launch) -> rope ->
               K/V append -> causal attention -> o (+ residual, in place) ->
               rms_norm -> gate_up (int8) -> silu_mul -> down (+ residual, in place)
    -> final rms_norm -> LM head -> argmax

with every weight, the KV cache and every activation resident in HBM, all
launches queued on one stream (so a whole step can be captured in a HIP
graph).  The LM head is the tied embedding either as a dense linear (fp16
copy of the table in fp16 mode, like BackendCUDA) or as int8 per-channel
codes through linear_q8 (the int8 LM head).

fused=True (fp16 only) issues the same arithmetic in fewer launches: the
RMSNorms before q/k/v and gate_up run in the input stage of those plans
(vvh_plan_set_input_op), RoPE and the K/V cache rows are the epilogue of the
q/k/v plan (vvh_plan_set_rope, vvh_plan_run_pos; its cosines and sines
come from a per-plan table, vvh_plan_set_rope_table), the SiLU-mul is the
epilogue of the gate_up plan (vvh_plan_set_glu), attention over spans of up
to 512 positions runs as per-wave parts (vvh_attention_parts) that the o
projection merges in its input stage (vvh_linear_q8_dev_attn), and the
embedding row is gathered straight to fp16.  Each stage rounds exactly as the standalone
operator, so the logits equal the unfused step's.  The final norm stays a
launch of its own: every block of the LM head would repeat it.

The model is synthetic (seeded N(0, 0.02) weights, no checkpoint); it is the
measurement and end-to-end parity harness of this library's operators.  The
drop-in boundary for the reference's own model code is BackendHIP.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import capi

F16, F32 = capi.F16, capi.F32


@dataclass(frozen=True)
class Config:
    hidden: int
    heads: int
    kv_heads: int
    inter: int
    layers: int
    vocab: int
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim


# Qwen2.5-0.5B (src/config/config_test.cc:22-33 of the reference)
QWEN25_05B = Config(hidden=896, heads=14, kv_heads=2, inter=4864, layers=24, vocab=151936)

# Longest span that vvh_attention_parts takes (one block of 8 waves of 64
# keys per kv head in the one-launch kernel).
ATTN_PARTS_MAX_SPAN = 512


class _Q8:
    """int8 codes + fp32 scales (+ fp32 bias) of one projection, in HBM,
    quantized on the device from seeded N(0, 0.02) fp32 weights (or from
    `src`, a device fp32 [N, K] array)."""

    def __init__(self, tmp, N, K, seed, bias, src=None):
        self.N, self.K = N, K
        self.q = capi.DevBuf(N * K)
        self.s = capi.DevBuf(N * 4)
        if src is None:
            if tmp.nbytes < N * K * 4:
                raise ValueError(f"weight scratch of {tmp.nbytes} bytes is too small for {N} x {K} fp32 weights")
            capi.call("vvh_fill_normal", tmp.ptr, F32, N * K, seed, 0.0, 0.02, None)
            src = tmp
        capi.call("vvh_quantize_per_channel", src.ptr, N, K, self.q.ptr, self.s.ptr, None)
        self.b = None
        if bias:
            self.b = capi.DevBuf(N * 4)
            capi.call("vvh_fill_normal", self.b.ptr, F32, N, seed + 1, 0.0, 0.01, None)


class Model:
    def __init__(self, cfg: Config, act: int = F16, lm_head: str = "dense", max_ctx: int = 2048, seed: int = 0,
                 fused: bool = False):
        assert lm_head in ("dense", "int8")
        if fused and act != F16:
            raise ValueError("the fused step needs fp16 activations")
        self.cfg, self.act, self.lm_head, self.max_ctx, self.fused = cfg, act, lm_head, max_ctx, fused
        c = cfg
        es = 2 if act == F16 else 4
        self.es = es
        big = max(c.inter * 2 * c.hidden, c.vocab * c.hidden)
        tmp = capi.DevBuf(big * 4)
        rng = np.random.default_rng(seed)
        # embedding table (tied LM head), fp32 as the reference keeps it
        self.table = capi.DevBuf(c.vocab * c.hidden * 4)
        capi.call("vvh_fill_normal", self.table.ptr, F32, c.vocab * c.hidden, seed + 7, 0.0, 0.02, None)
        self.table16 = None
        if lm_head == "dense" and act == F16:
            self.table16 = capi.DevBuf(c.vocab * c.hidden * 2)
            capi.call("vvh_convert", self.table16.ptr, F16, self.table.ptr, F32, c.vocab * c.hidden, None)
        self.head = None
        if lm_head == "int8":  # the tied table quantized per vocabulary row
            self.head = _Q8(tmp, c.vocab, c.hidden, 0, False, src=self.table)
        self.norms_host = []
        self.layers = []
        for l in range(c.layers):
            s0 = seed + 100 * (l + 1)
            ln1 = (1.0 + 0.1 * rng.standard_normal(c.hidden)).astype(np.float32)
            ln2 = (1.0 + 0.1 * rng.standard_normal(c.hidden)).astype(np.float32)
            self.norms_host.append((ln1, ln2))
            L = dict(ln1=capi.DevBuf.from_array(ln1), ln2=capi.DevBuf.from_array(ln2),
                     q=_Q8(tmp, c.hidden, c.hidden, s0 + 1, True), k=_Q8(tmp, c.kv_dim, c.hidden, s0 + 3, True),
                     v=_Q8(tmp, c.kv_dim, c.hidden, s0 + 5, True), o=_Q8(tmp, c.hidden, c.hidden, s0 + 7, False),
                     gu=_Q8(tmp, 2 * c.inter, c.hidden, s0 + 9, False),
                     down=_Q8(tmp, c.hidden, c.inter, s0 + 11, False),
                     kc=capi.DevBuf(max_ctx * c.kv_dim * es), vc=capi.DevBuf(max_ctx * c.kv_dim * es))
            self.layers.append(L)
        self.final_host = (1.0 + 0.1 * rng.standard_normal(c.hidden)).astype(np.float32)
        self.final_norm = capi.DevBuf.from_array(self.final_host)
        del tmp
        # activations
        self.x32 = capi.DevBuf(c.hidden * 4)
        self.x = capi.DevBuf(c.hidden * es)
        self.norm_out = capi.DevBuf(c.hidden * es)
        self.q = capi.DevBuf(c.hidden * es)
        self.k_new = capi.DevBuf(c.kv_dim * es)
        self.v_new = capi.DevBuf(c.kv_dim * es)
        self.attn = capi.DevBuf(c.hidden * es)
        self.gu = capi.DevBuf(2 * c.inter * es)
        self.gate = capi.DevBuf(c.inter * es)
        self.final = capi.DevBuf(c.hidden * es)
        self.logits = capi.DevBuf(c.vocab * es)
        self.logits32 = capi.DevBuf(c.vocab * 4)
        self.token = capi.DevBuf(4)
        # one grouped launch per layer for q/k/v (they share the input: the
        # normed rows, or in the fused step the residual stream through the
        # plan's RMSNorm input stage)
        self.plans = []
        src = self.x if fused else self.norm_out
        for L in self.layers:
            probs = [capi.Q8Problem(out=o.ptr, inp=src.ptr, residual=None, weight=p.q.ptr,
                                    scales=p.s.ptr, bias=p.b.ptr, M=1, N=p.N, K=p.K)
                     for o, p in ((self.q, L["q"]), (self.k_new, L["k"]), (self.v_new, L["v"]))]
            arr = (capi.Q8Problem * 3)(*probs)
            h = ctypes.c_uint64()
            capi.call("vvh_plan_create", arr, 3, act, act, ctypes.byref(h))
            self.plans.append(h.value)
            if fused:
                capi.call("vvh_plan_set_input_op", h.value, capi.IN_RMS_NORM, L["ln1"].ptr, c.eps)
                # RoPE and the K/V cache rows in the plan's epilogue (problems 0, 1, 2 = q, k, v)
                capi.call("vvh_plan_set_rope", h.value, 0, 1, 2, c.head_dim, c.theta, L["kc"].ptr, L["vc"].ptr)
                # cosine/sine of every position the cache holds, read by the epilogue
                capi.call("vvh_plan_set_rope_table", h.value, max_ctx)
        # fused: attention over spans of at most ATTN_PARTS_MAX_SPAN positions
        # as per-wave parts (vvh_attention_parts), merged in the o projection's
        # input stage (vvh_linear_q8_dev_attn): the same row as vvh_attention
        # with the keys spread over more CUs; longer spans keep vvh_attention
        self.parts = None
        self.nparts = ctypes.c_size_t()
        if fused and c.head_dim in (64, 128) and c.heads // c.kv_heads <= 16 and c.hidden <= 1024:
            self.parts_floats = 8 * c.heads * (c.head_dim + 4)
            self.parts = capi.DevBuf(self.parts_floats * 4)
        self.mlp_plans = []
        # fused: gate/up as a one-problem plan that reads the residual stream
        # through the post-attention RMSNorm and writes silu(gate) * up
        if fused:
            for L in self.layers:
                g = L["gu"]
                pr = capi.Q8Problem(out=self.gate.ptr, inp=self.x.ptr, residual=None, weight=g.q.ptr,
                                    scales=g.s.ptr, bias=None, M=1, N=2 * c.inter, K=c.hidden)
                arr = (capi.Q8Problem * 1)(pr)
                h = ctypes.c_uint64()
                capi.call("vvh_plan_create", arr, 1, act, act, ctypes.byref(h))
                self.mlp_plans.append(h.value)
                capi.call("vvh_plan_set_input_op", h.value, capi.IN_RMS_NORM, L["ln2"].ptr, c.eps)
                capi.call("vvh_plan_set_glu", h.value, 0)

    def fill_kv(self, seed: int = 0) -> None:
        """Seeded N(0, 1) rows in every layer's whole KV cache (a stand-in
        context, for timing a step at a given position)."""
        n = self.max_ctx * self.cfg.kv_dim
        for l, L in enumerate(self.layers):
            capi.call("vvh_fill_normal", L["kc"].ptr, self.act, n, seed + 2 * l, 0.0, 1.0, None)
            capi.call("vvh_fill_normal", L["vc"].ptr, self.act, n, seed + 2 * l + 1, 0.0, 1.0, None)

    def calls_per_step(self) -> int:
        """C-ABI calls per step (fp32 attention over more than one block and
        the argmax over the vocabulary launch two kernels each)."""
        c = self.cfg
        head = 1 if self.lm_head == "int8" or self.act == F32 else 2
        if self.fused:
            return 1 + 5 * c.layers + 1 + head + 1
        return (2 if self.act == F16 else 1) + 10 * c.layers + 1 + head + 1

    def close(self):
        for h in self.plans + self.mlp_plans:
            capi.call("vvh_plan_destroy", h)
        self.plans, self.mlp_plans = [], []

    # ---- one decode step -------------------------------------------------
    def step(self, token: int, pos: int, stream=None) -> None:
        """Queues one step for `token` at position `pos` on `stream`; the
        greedy next token lands in self.token (int32, device)."""
        c, a = self.cfg, self.act
        if pos >= self.max_ctx:
            raise ValueError(f"position {pos} beyond the KV cache ({self.max_ctx})")
        call = capi.call
        if a == F16 and self.fused:  # the table row rounded to fp16 once, in the gather
            call("vvh_embedding", self.x.ptr, self.table.ptr, token, c.hidden, c.vocab, F16, stream)
        elif a == F16:  # as BackendCUDA: the fp32 row, then the cast
            call("vvh_embedding", self.x32.ptr, self.table.ptr, token, c.hidden, c.vocab, F32, stream)
            call("vvh_convert", self.x.ptr, F16, self.x32.ptr, F32, c.hidden, stream)
        else:
            call("vvh_embedding", self.x.ptr, self.table.ptr, token, c.hidden, c.vocab, F32, stream)
        scale = float(1.0 / np.sqrt(np.float32(c.head_dim)))
        kvb = c.kv_dim * self.es
        if self.fused:
            self._fused_layers(pos, scale, stream)
        else:
            for L, plan in zip(self.layers, self.plans):
                call("vvh_rms_norm", self.norm_out.ptr, self.x.ptr, L["ln1"].ptr, 1, c.hidden, c.eps, a, stream)
                call("vvh_plan_run", plan, stream)
                call("vvh_rope", self.q.ptr, self.k_new.ptr, 1, c.heads, c.kv_heads, c.head_dim, pos, c.theta, a,
                     stream)
                call("vvh_kv_append", L["kc"].ptr + pos * kvb, L["vc"].ptr + pos * kvb, self.k_new.ptr,
                     self.v_new.ptr, kvb, stream)
                call("vvh_attention", self.attn.ptr, self.q.ptr, L["kc"].ptr, L["vc"].ptr, 1, pos + 1, c.heads,
                     c.kv_heads, c.head_dim, scale, a, stream)
                o = L["o"]
                call("vvh_linear_q8_dev", self.x.ptr, self.attn.ptr, o.q.ptr, o.s.ptr, None, self.x.ptr, 1,
                     c.hidden, c.hidden, a, a, stream)
                call("vvh_rms_norm", self.norm_out.ptr, self.x.ptr, L["ln2"].ptr, 1, c.hidden, c.eps, a, stream)
                g = L["gu"]
                call("vvh_linear_q8_dev", self.gu.ptr, self.norm_out.ptr, g.q.ptr, g.s.ptr, None, None, 1,
                     2 * c.inter, c.hidden, a, a, stream)
                call("vvh_eltwise", capi.OP_SILU_MUL, self.gate.ptr, self.gu.ptr, self.gu.ptr + c.inter * self.es,
                     c.inter, a, stream)
                d = L["down"]
                call("vvh_linear_q8_dev", self.x.ptr, self.gate.ptr, d.q.ptr, d.s.ptr, None, self.x.ptr, 1,
                     c.hidden, c.inter, a, a, stream)
        call("vvh_rms_norm", self.final.ptr, self.x.ptr, self.final_norm.ptr, 1, c.hidden, c.eps, a, stream)
        if self.lm_head == "int8":
            h = self.head
            call("vvh_linear_q8_dev", self.logits32.ptr, self.final.ptr, h.q.ptr, h.s.ptr, None, None, 1, c.vocab,
                 c.hidden, a, F32, stream)
        elif a == F16:
            call("vvh_dense", self.logits.ptr, self.final.ptr, self.table16.ptr, F16, None, None, 1, c.vocab,
                 c.hidden, F16, stream)
            call("vvh_convert", self.logits32.ptr, F32, self.logits.ptr, F16, c.vocab, stream)
        else:
            call("vvh_dense", self.logits32.ptr, self.final.ptr, self.table.ptr, F32, None, None, 1, c.vocab,
                 c.hidden, F32, stream)
        call("vvh_argmax", self.logits32.ptr, c.vocab, self.token.ptr, stream)

    def _fused_layers(self, pos: int, scale: float, stream) -> None:
        """The layers of the fused step: 5 launches per layer (q/k/v with
        RMSNorm in and RoPE + cache rows out, attention, o, gate/up with
        RMSNorm in and SiLU-mul out, down) instead of 10."""
        c, a, call = self.cfg, self.act, capi.call
        for L, plan, mlp in zip(self.layers, self.plans, self.mlp_plans):
            # q/k/v of rms_norm(x, ln1), RoPE'd, k and v rows written to the cache
            call("vvh_plan_run_pos", plan, pos, stream)
            o = L["o"]
            if self.parts is not None and pos + 1 <= ATTN_PARTS_MAX_SPAN:
                # attention parts, then o (+ residual) of their merge
                call("vvh_attention_parts", self.parts.ptr, self.parts_floats, ctypes.byref(self.nparts),
                     self.q.ptr, L["kc"].ptr, L["vc"].ptr, pos + 1, c.heads, c.kv_heads, c.head_dim, scale, a,
                     stream)
                call("vvh_linear_q8_dev_attn", self.x.ptr, self.parts.ptr, self.nparts.value, c.head_dim, o.q.ptr,
                     o.s.ptr, None, self.x.ptr, c.hidden, c.hidden, a, stream)
            else:
                call("vvh_attention", self.attn.ptr, self.q.ptr, L["kc"].ptr, L["vc"].ptr, 1, pos + 1, c.heads,
                     c.kv_heads, c.head_dim, scale, a, stream)
                call("vvh_linear_q8_dev", self.x.ptr, self.attn.ptr, o.q.ptr, o.s.ptr, None, self.x.ptr, 1,
                     c.hidden, c.hidden, a, a, stream)
            # silu(gate) * up of rms_norm(x, ln2) in one launch
            call("vvh_plan_run", mlp, stream)
            d = L["down"]
            call("vvh_linear_q8_dev", self.x.ptr, self.gate.ptr, d.q.ptr, d.s.ptr, None, self.x.ptr, 1, c.hidden,
                 c.inter, a, a, stream)

    def next_token(self) -> int:
        capi.sync()
        return int(self.token.to_array(np.int32, (1,))[0])

    def logits_host(self) -> np.ndarray:
        capi.sync()
        return self.logits32.to_array(np.float32, (self.cfg.vocab,))

    # ---- host copies for an external check ---------------------------------
    def host_weights(self) -> dict:
        """Every weight as numpy arrays (codes, scales, biases, norms, table)."""
        c = self.cfg

        def q8(p):
            q = p.q.to_array(np.int8, (p.N, p.K))
            s = p.s.to_array(np.float32, (p.N,))
            b = p.b.to_array(np.float32, (p.N,)) if p.b else None
            return q, s, b

        out = {"table": self.table.to_array(np.float32, (c.vocab, c.hidden)), "final_norm": self.final_host,
               "layers": []}
        if self.head is not None:
            out["head"] = q8(self.head)
        for L, (ln1, ln2) in zip(self.layers, self.norms_host):
            out["layers"].append(dict(ln1=ln1, ln2=ln2, **{k: q8(L[k]) for k in ("q", "k", "v", "o", "gu", "down")}))
        return out


def main(argv=None) -> int:
    """Runs decode steps of the synthetic Qwen2.5-0.5B-shaped model at one
    position of a filled KV cache (e.g. under rocprofv3 --kernel-trace):

        python -m vvllm_amd.qwen2_decode --lm-head int8 --position 511 --steps 5
    """
    import argparse
    import time

    ap = argparse.ArgumentParser(description=main.__doc__)
    ap.add_argument("--lm-head", choices=("dense", "int8"), default="int8")
    ap.add_argument("--act", choices=("f16", "f32"), default="f16")
    ap.add_argument("--position", type=int, default=511)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--fused", action="store_true", help="input stages and RoPE + KV append (fp16)")
    a = ap.parse_args(argv)
    capi.init(0)
    m = Model(QWEN25_05B, act=F16 if a.act == "f16" else F32, lm_head=a.lm_head, max_ctx=a.position + 1, seed=3,
              fused=a.fused)
    m.fill_kv(5)
    m.step(1, a.position)
    capi.sync()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        m.step(1, a.position)
    tok = m.next_token()
    el = (time.perf_counter() - t0) / a.steps
    print(f"{a.steps} steps at position {a.position} ({a.lm_head} LM head, {a.act}{', fused' if a.fused else ''}): "
          f"{el * 1e6:.0f} us/step "
          f"launched from Python, next token {tok}", flush=True)
    m.close()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
