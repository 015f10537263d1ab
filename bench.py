"""Benchmark of the INT8 per-channel linear path on one MI355X.

Headline: the full Qwen2.5-0.5B decode projection
set at M=1 -- per layer q 896->896 (+bias), k 896->128 (+bias), v 896->128
(+bias), o 896->896 (+residual, in place), gate 896->4864, up 896->4864,
down 4864->896 (+residual, in place) -- for 24 layers of independent seeded
int8 per-channel weights, fp16 activations and outputs, fp32 accumulation.

A step is one pass over the 168 projections, issued as one grouped launch
(vvh_plan_run) over weights already resident in HBM.  Three replicas of the
whole set (3 x 360 MB) are rotated step by step so that no step finds its
weights in the 256 MB Infinity Cache.  `value` is algorithmic HBM bytes per
step / measured step time (GB/s); the algorithmic bytes of one projection are
N*K (codes) + 4N (scales) + 4N (bias) + 2K (activation row) + 2N (output)
+ 2N (residual read).  Timing: W untimed warm-up steps, then K steps
bracketed by device synchronisation and HIP events on the stream the kernels
run on.

Also reported (same JSON line, key "extras"): the same set with the other
decode kernel families; in model order (q/k/v grouped, o, gate+up grouped,
down: 96 launches per step), launched from Python and captured in a HIP
graph; per-call times of each projection (24 single calls captured in a
graph, replayed); the LM-head GEMV, prefill GEMM TFLOPS
(configs[3]) and the Qwen2.5-1.5B M sweep; and the reference CPU
path (BackendCPU::linear_q8 compiled from the reference's sources,
oracle/_ref) timed single-threaded on a bounded sample of the same workload.

All inputs are synthetic (vvh_fill_normal + the device quantizer).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from vvllm_amd import capi  # noqa: E402

F16, F32 = capi.F16, capi.F32
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, AMD public spec
MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 MFMA, AMD public spec

QWEN05 = dict(hidden=896, kv=128, inter=4864, layers=24)
# (name, N, K, bias, residual)
def layer_projs(h, kv, inter):
    return [("q", h, h, True, False), ("k", kv, h, True, False), ("v", kv, h, True, False),
            ("o", h, h, False, True), ("gate", inter, h, False, False), ("up", inter, h, False, False),
            ("down", h, inter, False, True)]


def algo_bytes(M, N, K, bias, residual, act_bytes=2, out_bytes=2):
    return N * K + 4 * N + (4 * N if bias else 0) + M * K * act_bytes + M * N * out_bytes + \
        (M * N * out_bytes if residual else 0)


# ---------------------------------------------------------------------------
# HIP events on the null stream (the stream every launch below uses)
# ---------------------------------------------------------------------------
class HipEvents:
    """HIP events, streams and graphs through ctypes (timing plumbing only)."""

    def __init__(self):
        for name in ("libamdhip64.so.7", "libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
            try:
                self.hip = ctypes.CDLL(name)
                break
            except OSError:
                continue
        h, V = self.hip, ctypes.c_void_p
        h.hipEventCreate.argtypes = [ctypes.POINTER(V)]
        h.hipEventRecord.argtypes = [V, V]
        h.hipEventSynchronize.argtypes = [V]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), V, V]
        h.hipEventDestroy.argtypes = [V]
        h.hipStreamCreate.argtypes = [ctypes.POINTER(V)]
        h.hipStreamSynchronize.argtypes = [V]
        h.hipStreamBeginCapture.argtypes = [V, ctypes.c_int]
        h.hipStreamEndCapture.argtypes = [V, ctypes.POINTER(V)]
        h.hipGraphInstantiate.argtypes = [ctypes.POINTER(V), V, V, V, ctypes.c_size_t]
        h.hipGraphLaunch.argtypes = [V, V]
        h.hipGraphDestroy.argtypes = [V]
        h.hipGraphExecDestroy.argtypes = [V]

    def create(self):
        e = ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e, stream=None):
        assert self.hip.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b):
        assert self.hip.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def stream(self):
        s = ctypes.c_void_p()
        assert self.hip.hipStreamCreate(ctypes.byref(s)) == 0
        return s

    def graph(self, stream, fn):
        """Captures fn(stream) into an instantiated graph; the captured graph
        itself is destroyed once instantiated.  The caller releases the
        executable graph with drop()."""
        g, ge = ctypes.c_void_p(), ctypes.c_void_p()
        assert self.hip.hipStreamBeginCapture(stream, 0) == 0
        fn(stream)
        assert self.hip.hipStreamEndCapture(stream, ctypes.byref(g)) == 0
        try:
            assert self.hip.hipGraphInstantiate(ctypes.byref(ge), g, None, None, 0) == 0
        finally:
            assert self.hip.hipGraphDestroy(g) == 0
        return ge

    def launch(self, ge, stream):
        assert self.hip.hipGraphLaunch(ge, stream) == 0

    def drop(self, *graphs):
        """Destroys executable graphs (after the work queued from them ends)."""
        capi.sync()
        for ge in graphs:
            assert self.hip.hipGraphExecDestroy(ge) == 0

    def destroy(self, *events):
        for e in events:
            assert self.hip.hipEventDestroy(e) == 0


def timed(ev, fn, reps, stream=None):
    """Average ms per call of fn(i) over reps calls, HIP events around the loop
    on the stream the work runs on."""
    capi.sync()
    a, b = ev.create(), ev.create()
    try:
        ev.record(a, stream)
        for i in range(reps):
            fn(i)
        ev.record(b, stream)
        ms = ev.elapsed_ms(a, b)
        capi.sync()
    finally:
        ev.destroy(a, b)
    return ms / reps


# ---------------------------------------------------------------------------
# device-resident synthetic workload
# ---------------------------------------------------------------------------
class Arena:
    """One device allocation carved into 256-byte aligned pieces."""

    def __init__(self, nbytes):
        self.buf = capi.DevBuf(nbytes)
        self.off = 0

    def take(self, nbytes):
        p = self.buf.ptr + self.off
        self.off += (nbytes + 255) // 256 * 256
        assert self.off <= self.buf.nbytes
        return p


def arena_size(items):
    return sum((n + 255) // 256 * 256 for n in items)


ROTATE_BYTES = 1 << 30  # more than the 256 MB MALL: every timed call reads its weights from HBM


def check_scratch(tmp_w, N, K):
    """Raises before any device call when the fp32 weight scratch `tmp_w`
    (anything with .ptr and .nbytes, e.g. a capi.DevBuf) cannot hold the
    N x K fp32 weights that vvh_fill_normal writes into it."""
    need = N * K * 4
    nbytes = getattr(tmp_w, "nbytes", None)
    if nbytes is None or not getattr(tmp_w, "ptr", None):
        raise TypeError("the weight scratch must be a device buffer with .ptr and .nbytes")
    if need > nbytes:
        raise ValueError(f"weight scratch of {nbytes} bytes is too small for {N} x {K} fp32 weights ({need} bytes)")


def rotation(tmp_w, M, N, K, bias, res, seed, act=F16, outd=F16, max_reps=4096):
    """Replicas of one projection's weights (codes, scales, bias), enough that
    cycling through them moves >= ROTATE_BYTES of weights, in one arena; the
    activation and output rows are shared, as in a model step, where the
    previous operator has just written them.  tmp_w: the fp32 weight scratch
    (a capi.DevBuf of at least N * K * 4 bytes).  Returns (arena, linears)."""
    check_scratch(tmp_w, N, K)
    ab, ob = (2 if act == F16 else 4), (2 if outd == F16 else 4)
    wsz = [N * K, 4 * N] + ([4 * N] if bias else [])
    per = arena_size(wsz)
    n = max(2, min(max_reps, -(-ROTATE_BYTES // per)))
    ar = Arena(per * n + arena_size([M * K * ab, M * N * ob]))
    x, y = ar.take(M * K * ab), ar.take(M * N * ob)
    capi.call("vvh_fill_normal", x, act, M * K, seed + 2, 0.0, 1.0, None)
    capi.call("vvh_fill_normal", y, outd, M * N, seed + 3, 0.0, 1.0, None)
    return ar, [Linear(ar, tmp_w, M, N, K, bias, res, seed + 5 * r, act, outd, xy=(x, y)) for r in range(n)]


GRAPH_CALLS = 64  # calls captured per HIP graph in graph_rotation


def graph_rotation(ev, lins, stream, min_calls=60):
    """ms per call over the replicas in `lins`, each called once per pass,
    the calls captured in HIP graphs of at most GRAPH_CALLS calls on `stream`
    and replayed: what a model step pays per call on the GPU, without the
    host's launch time (a Python call costs several microseconds, more than
    a small projection's kernel).  Every replica runs once on `stream`
    before capture (this sizes the stream's workspace) and one replayed pass
    precedes the timed passes."""
    for l in lins:
        l.run(stream)
    capi.sync()
    graphs = [ev.graph(stream, lambda st, c=lins[i:i + GRAPH_CALLS]: [l.run(st) for l in c])
              for i in range(0, len(lins), GRAPH_CALLS)]

    def one_pass(_i):
        for g in graphs:
            ev.launch(g, stream)

    try:
        one_pass(0)
        passes = max(2, -(-min_calls // len(lins)))
        return timed(ev, one_pass, passes, stream) / len(lins)
    finally:
        ev.drop(*graphs)


def timed_rotation(ev, lins, steps, stream=None):
    """ms per call over `steps` calls that rotate through `lins`, after one
    warm-up pass over all of them (so no timed call finds its operands in
    the MALL from the set-up writes)."""
    for l in lins:
        l.run(stream)
    n = len(lins)
    return timed(ev, lambda i: lins[(i + 1) % n].run(stream), steps, stream)


class Linear:
    """One quantized projection resident in HBM with its input/output rows."""

    def __init__(self, arena, tmp_w, M, N, K, bias, residual, seed, act=F16, outd=F16, xy=None):
        """tmp_w: the device scratch (a capi.DevBuf) that holds the N x K fp32
        weights before quantization; xy: (x, y) device pointers to share
        instead of rows of its own."""
        check_scratch(tmp_w, N, K)
        self.M, self.N, self.K, self.has_bias, self.has_res = M, N, K, bias, residual
        self.act, self.outd = act, outd
        ab, ob = (2 if act == F16 else 4), (2 if outd == F16 else 4)
        self.w = arena.take(N * K)
        self.s = arena.take(4 * N)
        self.b = arena.take(4 * N) if bias else None
        capi.call("vvh_fill_normal", tmp_w.ptr, F32, N * K, seed, 0.0, 0.02, None)
        capi.call("vvh_quantize_per_channel", tmp_w.ptr, N, K, self.w, self.s, None)
        if bias:
            capi.call("vvh_fill_normal", self.b, F32, N, seed + 1, 0.0, 0.01, None)
        if xy is None:
            self.x = arena.take(M * K * ab)
            self.y = arena.take(M * N * ob)
            capi.call("vvh_fill_normal", self.x, act, M * K, seed + 2, 0.0, 1.0, None)
            capi.call("vvh_fill_normal", self.y, outd, M * N, seed + 3, 0.0, 1.0, None)
        else:
            self.x, self.y = xy
        self.bytes = algo_bytes(M, N, K, bias, residual, ab, ob)
        self.flops = 2 * M * N * K

    @staticmethod
    def sizes(M, N, K, bias, act=F16, outd=F16):
        ab, ob = (2 if act == F16 else 4), (2 if outd == F16 else 4)
        return [N * K, 4 * N] + ([4 * N] if bias else []) + [M * K * ab, M * N * ob]

    def problem(self):
        return capi.Q8Problem(out=self.y, inp=self.x, residual=self.y if self.has_res else None, weight=self.w,
                              scales=self.s, bias=self.b, M=self.M, N=self.N, K=self.K)

    def run(self, stream=None):
        capi.call("vvh_linear_q8_dev", self.y, self.x, self.w, self.s, self.b,
                  self.y if self.has_res else None, self.M, self.N, self.K, self.act, self.outd, stream)


def make_plan(linears, act=F16, outd=F16, kernel=capi.KERNEL_AUTO):
    arr = (capi.Q8Problem * len(linears))(*[l.problem() for l in linears])
    h = ctypes.c_uint64()
    capi.set_kernel(kernel)
    try:
        capi.call("vvh_plan_create", arr, len(linears), act, outd, ctypes.byref(h))
    finally:
        capi.set_kernel(capi.KERNEL_AUTO)
    return h.value


KERNEL_SYMBOL = {"dot": "k_dot_grouped<f16>", "stream": "k_stream<f16>", "skinny": "k_skinny_grouped<f16>"}


def build_decode_set(replicas, layers, projs, tmp_w, M=1):
    sets = []
    for r in range(replicas):
        sizes = []
        for _ in range(layers):
            for (_, N, K, bias, _res) in projs:
                sizes += Linear.sizes(M, N, K, bias)
        arena = Arena(arena_size(sizes))
        lins = []
        for l in range(layers):
            for pid, (name, N, K, bias, res) in enumerate(projs):
                seed = 0x5EED + 16 * l + pid + 100003 * r
                lins.append(Linear(arena, tmp_w, M, N, K, bias, res, seed))
        sets.append((arena, lins))
    capi.sync()
    return sets


# ---------------------------------------------------------------------------
# CPU baseline: reference BackendCPU::linear_q8 on the host, one thread
# ---------------------------------------------------------------------------
def bf16_layer_rows(projs, seed):
    """Host BF16 bit patterns of one layer's projection weights, N(0, 0.02)."""
    rng = np.random.default_rng(seed)
    out = []
    for name, N, K, bias, res in projs:
        w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
        out.append((name, N, K, (w.view(np.uint32) >> 16).astype(np.uint16)))
    return out


def cpu_ingest(projs):
    """Host path a BF16 checkpoint takes in the reference (widen to fp32, then
    quantize_per_channel) on one layer's weights, one thread: GB/s of BF16
    input."""
    from oracle import oracle as O
    if not O.available("port"):
        O.build(ref=False)
    rows = bf16_layer_rows(projs, 5)
    t0 = time.perf_counter()
    for _, N, K, bits in rows:
        O.ingest_bf16(bits)
    el = time.perf_counter() - t0
    nbytes = sum(b.nbytes for *_, b in rows)
    return {"GBps": round(nbytes / el / 1e9, 3), "seconds": round(el, 3), "bf16_bytes": nbytes,
            "sample": "one Qwen2.5-0.5B layer (q,k,v,o,gate,up,down), oracle restatement, one thread"}


def host_cpu():
    """Model name of the host CPU (lscpu's "Model name"), from /proc/cpuinfo."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(lins, budget_s):
    from oracle import oracle as O

    kind = "reference" if O.available("reference") else "port"
    if not O.available(kind):
        O.build(ref=False)
    host, host_keep = [], []
    for l in lins:
        q = np.empty((l.N, l.K), np.int8)
        capi.call("vvh_memcpy_d2h", q.ctypes.data, l.w, q.nbytes)
        s = np.empty(l.N, np.float32)
        capi.call("vvh_memcpy_d2h", s.ctypes.data, l.s, s.nbytes)
        b = None
        if l.b:
            b = np.empty(l.N, np.float32)
            capi.call("vvh_memcpy_d2h", b.ctypes.data, l.b, b.nbytes)
        x16 = np.empty((1, l.K), np.float16)
        capi.call("vvh_memcpy_d2h", x16.ctypes.data, l.x, x16.nbytes)
        r = np.zeros((1, l.N), np.float32) if l.has_res else None
        host.append((x16.astype(np.float32), q, s, b, r, l))
    # the reference takes fp32 activations/outputs (widened fp16 inputs are exact);
    # call its entry points directly with preallocated buffers
    lib = O._lib(kind)
    pre = "ref_" if kind == "reference" else "orc_"
    f_lin, f_add = getattr(lib, pre + "linear_q8"), getattr(lib, pre + "linear_q8_add")
    calls = []
    for x, q, s, b, r, l in host:
        y = r if r is not None else np.empty((1, l.N), np.float32)
        bp = None if b is None else b.ctypes.data
        if r is not None:  # linear_q8_add in place, as the model calls it
            calls.append((f_add, (y.ctypes.data, x.ctypes.data, q.ctypes.data, s.ctypes.data, bp, y.ctypes.data,
                                  1, l.N, l.K)))
        else:
            calls.append((f_lin, (y.ctypes.data, x.ctypes.data, q.ctypes.data, s.ctypes.data, bp, 1, l.N, l.K)))
        host_keep.append(y)
    per_pass = sum(algo_bytes(1, l.N, l.K, l.has_bias, l.has_res, 4, 4) for *_, l in host)
    # one thread pinned to one core (the reference's CPU path is single-threaded),
    # as `taskset -c <core>` would; the process's own affinity is restored after
    allowed = sorted(os.sched_getaffinity(0))
    core = allowed[0]
    os.sched_setaffinity(0, {core})
    try:
        def one_pass():
            t = time.perf_counter()
            for f, a in calls:
                f(*a)
            return time.perf_counter() - t

        one_pass()  # warm-up: first touch of the host copies, caches, clocks
        times, t0 = [], time.perf_counter()
        while len(times) < 20 or time.perf_counter() - t0 < budget_s:
            times.append(one_pass())
        el = time.perf_counter() - t0
        ingest = cpu_ingest(layer_projs(896, 128, 4864))
    finally:
        os.sched_setaffinity(0, set(allowed))
    med = float(np.median(times))
    return dict(value=round(per_pass / med / 1e9, 3), unit="GB/s", cores=1, kind=kind,
                host_cpu=host_cpu(), nproc=os.cpu_count(), cpus_allowed=len(allowed), pinned_core=core,
                ms_per_step=round(med * 1e3, 3), ms_per_step_mean=round(el / len(times) * 1e3, 3),
                timed_passes=len(times), ingest_host_path=ingest,
                sample=(f"one warm-up pass, then {len(times)} timed passes (the median reported) of the 24-layer "
                        f"decode projection set (168 linear_q8 calls, same int8 weights as the GPU run, fp32 "
                        f"activations) in {el:.1f} s, one thread pinned to core {core}; "
                        + ("reference BackendCPU::linear_q8 compiled from its sources -O2 -mavx2 -mfma"
                           if kind == "reference" else "oracle restatement of BackendCPU::linear_q8")))


# ---------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replicas", type=int, default=3)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--workload", choices=("decode", "prefill", "lm-head", "vendor-gemm", "copy", "configs",
                                           "dense-head", "decode-ops"),
                    default="decode",
                    help="decode: configs[1] (the headline line); prefill: configs[3] gate/up GEMM only; "
                         "lm-head: configs[2] alone; "
                         "vendor-gemm: the int8 GEMM beside the vendor fp16 GEMM on the prefill shapes; "
                         "copy: a 256 MiB device-to-device copy, the calibration of the HBM traffic counters; "
                         "configs: every configs[3] and configs[4] (M = 1, 16, 256) shape, bracketed for "
                         "rocprofv3 (see --trace-configs); dense-head: the dense fp16 tied LM head (vvh_dense); "
                         "decode-ops: each operator of the fused decode step alone (graph replay)")
    ap.add_argument("--trace-configs", metavar="KERNEL_TRACE_CSV",
                    help="summarise the rocprofv3 kernel trace of a --workload configs run per shape and kernel "
                         "(needs --configs-json, the run's JSON line; --pmc adds counter CSVs); no GPU is used")
    ap.add_argument("--configs-json", metavar="FILE", help="the JSON line printed by --workload configs")
    ap.add_argument("--pmc", nargs="*", metavar="COUNTER_CSV", help="rocprofv3 --pmc CSVs of the same workload")
    ap.add_argument("--markdown", action="store_true", help="--trace-configs: also print a markdown table")
    ap.add_argument("--max-replicas", type=int, default=4096,
                    help="--workload configs: at most this many weight replicas per shape (counter runs, where "
                         "every set-up kernel is serialised, use few)")
    ap.add_argument("--prefill-m", type=int, default=512)
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="summarise a rocprofv3 --kernel-trace CSV of a bench run: the dispatches of the kernel "
                         "named by --kernel after the first --skip of them (the warm-up steps); no GPU is used")
    ap.add_argument("--kernel", default="k_dot_grouped", help="substring of the kernel name (--trace-summary)")
    ap.add_argument("--skip", type=int, default=None, help="dispatches to skip (--trace-summary; default --warmup)")
    ap.add_argument("--count", type=int, default=None,
                    help="dispatches to summarise after the skipped ones (--trace-summary; default --steps)")
    ap.add_argument("--bytes", type=float, default=360339456.0,
                    help="algorithmic bytes per dispatch (--trace-summary; default: the headline step)")
    args = ap.parse_args()
    if args.trace_summary:
        return trace_summary(args)
    if args.trace_configs:
        return configs_summary(args)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build targets one MI355X; the int8 linear path is measured on one GPU "
              "(multi-GPU sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.workload == "vendor-gemm":
        import torch  # torch's own HIP runtime must start before this library's (else it sees no GPU)
        torch.cuda.init()
    name = capi.init(0)
    ev = HipEvents()
    if args.workload == "prefill":
        return prefill_main(args, ev, name)
    if args.workload == "lm-head":
        return lm_head_main(args, ev, name)
    if args.workload == "vendor-gemm":
        return vendor_gemm_main(args, ev)
    if args.workload == "copy":
        return copy_main(args, ev)
    if args.workload == "configs":
        return configs_main(args, ev)
    if args.workload == "dense-head":
        return dense_head_main(args, ev)
    if args.workload == "decode-ops":
        return decode_ops_main(args, ev)
    h, kv, inter, L = QWEN05["hidden"], QWEN05["kv"], QWEN05["inter"], QWEN05["layers"]
    projs = layer_projs(h, kv, inter)
    tmp_w = capi.DevBuf(max(inter * h, 151936 * 896, 8960 * 1536) * 4)

    t_setup = time.perf_counter()
    sets = build_decode_set(args.replicas, L, projs, tmp_w)
    plans = [make_plan(lins) for _, lins in sets]
    step_bytes = sum(l.bytes for l in sets[0][1])
    print(f"[bench] {name}: {args.replicas} x {len(sets[0][1])} projections, "
          f"{step_bytes / 1e6:.1f} MB/step, setup {time.perf_counter() - t_setup:.1f}s", file=sys.stderr, flush=True)

    def step(i):
        capi.call("vvh_plan_run", plans[i % len(plans)], None)

    for i in range(args.warmup):
        step(i)
    ms = timed(ev, lambda i: step(args.warmup + i), args.steps)
    value = step_bytes / (ms * 1e-3) / 1e9
    launches = ctypes.c_int()
    capi.call("vvh_plan_launches", plans[0], ctypes.byref(launches))
    kern = capi.plan_kernel(plans[0])
    print(f"[bench] {kern} step {ms * 1e3:.1f} us, {value:.0f} GB/s", file=sys.stderr, flush=True)

    traffic = None
    tfile = os.path.join(ROOT, "profiles", "traffic_decode_set.json")
    if os.path.exists(tfile):
        t = json.load(open(tfile))
        # measured on the kernel family this run uses (the file names the full instantiation)
        if t.get("kernel", "").split("<")[0] == KERNEL_SYMBOL.get(kern, "?").split("<")[0]:
            traffic = t.get("hbm_bytes_per_launch")

    result = {
        "metric": "linear_q8 GEMV µs + HBM GB/s at Qwen2.5-0.5B shapes; prefill GEMM TFLOPS",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x f16 activations, f32 accumulate",
        "data": "synthetic (seeded N(0,0.02) fp32 weights quantized per channel on device; N(0,1) fp16 activations)",
        "config": {"workload": "configs[1]: Qwen2.5-0.5B decode projection set, 24 layers x "
                               "{q,k,v,o,gate,up,down}, M=1, one grouped launch per step",
                   "M": 1, "layers": L, "projections_per_step": len(sets[0][1]),
                   "algorithmic_bytes_per_step": step_bytes, "weight_replicas_rotated": args.replicas,
                   "launches_per_step": launches.value, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": KERNEL_SYMBOL.get(kern, kern), "achieved": round(value, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
    }

    if not args.no_extras:
        result["extras"] = extras(ev, sets, projs, tmp_w, args)
    if not args.no_cpu:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(sets[0][1], args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


def trace_summary(args):
    """Timed dispatches of one kernel in a rocprofv3 kernel trace: count,
    mean / median / min / max duration, and algorithmic bytes / mean
    against the HBM peak, as one JSON line."""
    import csv
    import statistics
    rows = [r for r in csv.DictReader(open(args.trace_summary)) if args.kernel in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    skip = args.warmup if args.skip is None else args.skip
    count = args.steps if args.count is None else args.count
    rows_all = len(rows)
    rows = rows[:skip + count]
    d = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows[skip:]]
    if not d:
        print(json.dumps({"error": f"no dispatch of {args.kernel!r} after {skip}"}))
        return
    mean = sum(d) / len(d)
    span = (int(rows[-1]["End_Timestamp"]) - int(rows[skip]["Start_Timestamp"])) / 1e3 / len(d)
    print(json.dumps({"kernel": rows[0]["Kernel_Name"][:120], "dispatches": rows_all, "skipped": skip,
                      "timed": len(d), "mean_us": round(mean, 3), "median_us": round(statistics.median(d), 3),
                      "min_us": round(min(d), 3), "max_us": round(max(d), 3),
                      "span_per_dispatch_us": round(span, 3),
                      "GBps_at_mean": round(args.bytes / (mean * 1e-6) / 1e9, 1),
                      "hbm_frac_at_mean": round(args.bytes / (mean * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}))


def kernel_name(M, N, K, outd=F16):
    """Kernel family of an fp16 linear_q8 call, with the GEMM variant spelled out."""
    k = capi.kernel_choice(M, N, K, F16, outd)
    return capi.gemm_variant(M, N, K) if k == "gemm" else k


def prefill_main(args, ev, name):
    """configs[3] gate/up GEMM alone (M = --prefill-m, N = 4864, K = 896, fp16
    in and out): one JSON line in TFLOP/s against the fp16 MFMA peak.
    Replicas of the weights rotate (>= 1 GiB, see rotation()); the kernel
    runs on the null stream, where the HIP events are recorded."""
    M, N, K = args.prefill_m, QWEN05["inter"], QWEN05["hidden"]
    tmp_w = capi.DevBuf(N * K * 4)
    _ar, lins = rotation(tmp_w, M, N, K, False, False, 900)
    for i in range(args.warmup):
        lins[i % len(lins)].run()
    ms = timed_rotation(ev, lins, args.steps)
    tf = lins[0].flops / (ms * 1e-3) / 1e12
    kern = kernel_name(M, N, K)
    print(f"[bench] {name}: prefill gate/up M={M} {ms * 1e3:.2f} us, {tf:.0f} TFLOP/s ({kern})",
          file=sys.stderr, flush=True)
    print(json.dumps({
        "metric": "linear_q8 GEMV µs + HBM GB/s at Qwen2.5-0.5B shapes; prefill GEMM TFLOPS",
        "value": round(tf, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 weights x f16 activations, f32 accumulate",
        "data": "synthetic (seeded N(0,0.02) fp32 weights quantized per channel on device; N(0,1) fp16 activations)",
        "config": {"workload": f"configs[3]: prefill gate/up GEMM, M={M}, N={N}, K={K}, fp16 out",
                   "M": M, "N": N, "K": K, "flops_per_step": lins[0].flops, "replicas_rotated": len(lins),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": kern, "achieved": round(tf, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None},
        "cpu_baseline": None}), flush=True)


def lm_head_main(args, ev, name):
    """configs[2] alone: the LM-head GEMV (M=1, K=896, N=151936, fp16
    activations, fp32 logits), 8 weight replicas rotated (>= 1 GiB), calls
    launched back to back on the null stream (each call, about 25 us, is
    longer than its launch) and timed with HIP events: one JSON line in GB/s
    against the HBM peak."""
    N, K = 151936, QWEN05["hidden"]
    tmp_w = capi.DevBuf(N * K * 4)
    _ar, heads = rotation(tmp_w, 1, N, K, False, False, 777, F16, F32)
    for i in range(args.warmup):
        heads[i % len(heads)].run()
    ms = timed(ev, lambda i: heads[i % len(heads)].run(), args.steps)
    b = heads[0].bytes
    gbs = b / (ms * 1e-3) / 1e9
    print(f"[bench] {name}: lm head {ms * 1e3:.2f} us, {gbs:.0f} GB/s", file=sys.stderr, flush=True)
    print(json.dumps({
        "metric": "linear_q8 GEMV µs + HBM GB/s at Qwen2.5-0.5B shapes; prefill GEMM TFLOPS",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 weights x f16 activations, f32 accumulate",
        "data": "synthetic (seeded N(0,0.02) fp32 weights quantized per channel on device; N(0,1) fp16 activations)",
        "config": {"workload": f"configs[2]: LM-head GEMV, M=1, N={N}, K={K}, fp32 logits",
                   "M": 1, "N": N, "K": K, "algorithmic_bytes_per_step": b, "replicas_rotated": len(heads),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "k_dot<float>", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": None}), flush=True)


# The per-shape profiling workload: BASELINE.json configs[3] (both MLP shapes at
# M = 128, 512, 2048) and configs[4] (the Qwen2.5-1.5B shapes at M = 1, 16, 256),
# fp16 activations and outputs; the down projections add their residual in place
# (as the model calls them, include/vvllm/model/transformer.h:187-188).
CONFIG_SHAPES = [(f"c3_{nm}_M{M}", M, N, K, res) for M in (128, 512, 2048)
                 for nm, N, K, res in (("gate_up", 4864, 896, False), ("down", 896, 4864, True))] + \
                [(f"c4_{nm}_M{M}", M, N, K, False) for M in (1, 16, 256)
                 for nm, N, K in (("qo", 1536, 1536), ("kv", 256, 1536), ("gate_up", 8960, 1536), ("down", 1536, 8960))]


def separator(buf):
    """A kernel that no linear_q8 call uses (vvh_argmax over 1 value, which
    runs k_sample_part): it brackets each shape's timed calls in a rocprofv3
    kernel trace."""
    capi.call("vvh_argmax", buf.ptr, 1, buf.ptr + 64, None)


def configs_main(args, ev):
    """Every configs[3] / configs[4] shape, one after the other: weight replicas
    rotated (>= 1 GiB, as rotation()), one untimed pass over them, then
    --steps calls launched one by one on the null stream between two
    separator kernels.  Under rocprofv3 --kernel-trace (or --pmc) the calls
    of shape i are the dispatches between separators 2i and 2i+1; run
    bench.py --trace-configs on that trace for the per-kernel durations.  The
    JSON line gives each shape's kernel, algorithmic bytes and flops and the
    HIP-event time per call (launches from Python: the host's launch rate
    bounds the small shapes; the kernel durations come from the trace)."""
    tmp = capi.DevBuf(8960 * 1536 * 4)
    sep = capi.DevBuf(256)
    capi.call("vvh_fill_normal", sep.ptr, F32, 1, 1, 0.0, 1.0, None)
    out = {}
    for name, M, N, K, res in CONFIG_SHAPES:
        print(f"[bench] {name}: set-up", file=sys.stderr, flush=True)
        _ar, lins = rotation(tmp, M, N, K, False, res, 900, max_reps=args.max_replicas)
        for l in lins:
            l.run()
        capi.sync()
        separator(sep)
        ms = timed(ev, lambda i: lins[i % len(lins)].run(), args.steps)
        separator(sep)
        capi.sync()
        l = lins[0]
        out[name] = {"M": M, "N": N, "K": K, "residual": res, "kernel": kernel_name(M, N, K),
                     "calls": args.steps, "bytes": l.bytes, "flops": l.flops, "us_events": round(ms * 1e3, 3),
                     "replicas_rotated": len(lins)}
        print(f"[bench] {name}: {ms * 1e3:.2f} us/call (events) {out[name]['kernel']}", file=sys.stderr, flush=True)
        del lins, _ar
    print(json.dumps({"workload": "configs", "order": [s[0] for s in CONFIG_SHAPES], "shapes": out}), flush=True)


def configs_summary(args):
    """Per-shape kernel durations of a --workload configs run from its
    rocprofv3 kernel trace (and counters from --pmc traces of the same
    workload): the dispatches between separator pairs, grouped by kernel;
    per call the algorithmic bytes and flops over the summed kernel means.
    One JSON line; with --markdown, a table as well."""
    import csv
    import statistics
    meta = json.load(open(args.configs_json))
    order = meta["order"]

    def segments(rows, key):
        rows.sort(key=key)
        segs, cur, open_ = [], None, False
        prev_sep = False
        for r in rows:
            is_sep = "k_sample_part" in r["Kernel_Name"]  # vvh_argmax's kernel
            if is_sep and not prev_sep:
                if open_:
                    segs.append(cur)
                    open_ = False
                else:
                    cur, open_ = [], True
            elif not is_sep and open_:
                cur.append(r)
            prev_sep = is_sep
        return segs

    rows = list(csv.DictReader(open(args.trace_configs)))
    segs = segments(rows, lambda r: int(r["Start_Timestamp"]))
    if len(segs) != len(order):
        print(json.dumps({"error": f"{len(segs)} bracketed segments for {len(order)} shapes"}))
        return
    counters = {}
    for path in args.pmc or []:
        crow = list(csv.DictReader(open(path)))
        # one row per (dispatch, counter): order dispatches by id
        by_disp = {}
        for r in crow:
            d = by_disp.setdefault(int(r["Dispatch_Id"]), {"Kernel_Name": r["Kernel_Name"], "c": {}})
            d["c"][r["Counter_Name"]] = d["c"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        disp = [{"Kernel_Name": v["Kernel_Name"], "id": k, "c": v["c"]} for k, v in by_disp.items()]
        for name, seg in zip(order, segments(disp, lambda r: r["id"])):
            for r in seg:
                kshort = r["Kernel_Name"].split("(")[0][:90]
                acc = counters.setdefault(name, {}).setdefault(kshort, {})
                for cn, cv in r["c"].items():
                    acc.setdefault(cn, []).append(cv)
    out = {}
    for name, seg in zip(order, segs):
        sh = meta["shapes"][name]
        ks = {}
        for r in seg:
            kshort = r["Kernel_Name"].split("(")[0][:90]
            ks.setdefault(kshort, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        kern = {}
        per_call = 0.0
        for k, d in ks.items():
            mean = sum(d) / len(d)
            per_call += mean * len(d) / sh["calls"]
            kern[k] = {"dispatches": len(d), "mean_us": round(mean, 3), "median_us": round(statistics.median(d), 3),
                       "min_us": round(min(d), 3), "max_us": round(max(d), 3)}
            c = counters.get(name, {}).get(k)
            if c:
                kern[k]["counters_mean"] = {cn: round(sum(v) / len(v), 1) for cn, v in c.items()}
        out[name] = {**sh, "kernels": kern, "kernel_us_per_call": round(per_call, 3),
                     "GBps": round(sh["bytes"] / (per_call * 1e-6) / 1e9, 1),
                     "hbm_frac": round(sh["bytes"] / (per_call * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "TFLOPS": round(sh["flops"] / (per_call * 1e-6) / 1e12, 1),
                     "mfma_frac": round(sh["flops"] / (per_call * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    print(json.dumps({"configs": out}))
    if args.markdown:
        print("\n| Shape | Kernel | Calls | Mean µs | Median µs | Bytes | GB/s | HBM frac | TFLOP/s | MFMA frac |")
        print("|---|---|---|---|---|---|---|---|---|---|")
        for name in order:
            o = out[name]
            for i, (k, v) in enumerate(o["kernels"].items()):
                head = (f"| {name} | `{k}` | {v['dispatches']} | {v['mean_us']} | {v['median_us']} | ")
                if i == 0:
                    print(head + f"{o['bytes']} | {o['GBps']} | {o['hbm_frac']} | {o['TFLOPS']} | {o['mfma_frac']} |")
                else:
                    print(head + "| | | | |")


def dense_head_main(args, ev):
    """The tied LM head as the reference computes it (a dense linear over the
    fp16 embedding table, transformer.h:202-203 -> backend_cuda.cc:171-179):
    vvh_dense, M = 1, N = 151936, K = 896, fp16 weights, activations and
    logits; 4 replicas of the 272 MB table rotated (1.09 GB), calls launched
    one by one on the null stream (each is longer than its launch) and timed
    with HIP events.  One JSON line in GB/s against the HBM peak."""
    N, K, reps = 151936, QWEN05["hidden"], 4
    tables = [capi.DevBuf(N * K * 2) for _ in range(reps)]
    for i, t in enumerate(tables):
        capi.call("vvh_fill_normal", t.ptr, F16, N * K, 40 + i, 0.0, 0.02, None)
    x, y = capi.DevBuf(K * 2), capi.DevBuf(N * 2)
    capi.call("vvh_fill_normal", x.ptr, F16, K, 7, 0.0, 1.0, None)
    run = lambda i: capi.call("vvh_dense", y.ptr, x.ptr, tables[i % reps].ptr, F16, None, None, 1, N, K, F16, None)
    for i in range(max(args.warmup, reps)):
        run(i)
    ms = timed(ev, run, args.steps)
    b = N * K * 2 + K * 2 + N * 2
    gbs = b / (ms * 1e-3) / 1e9
    print(f"[bench] dense fp16 LM head {ms * 1e3:.2f} us, {gbs:.0f} GB/s", file=sys.stderr, flush=True)
    print(json.dumps({"workload": "dense fp16 LM head (vvh_dense, M=1, N=151936, K=896)", "us": round(ms * 1e3, 3),
                      "GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": b,
                      "steps": args.steps, "replicas_rotated": reps}), flush=True)


def decode_ops_main(args, ev):
    """Each operator of the fused Qwen2.5-0.5B decode step alone: its 24
    per-layer calls (the model's own buffers and plans, position 511 of a
    filled KV cache) captured in one HIP graph and replayed; µs per call,
    a graph node included.  Beside them: a near-empty kernel, the one-launch
    attention and the o projection on its row, the gate/up plan without its
    stage or epilogue, with either alone, and the same problem as one k_dot
    call.  One JSON line."""
    from vvllm_amd import qwen2_decode as qd
    c, P, a = qd.QWEN25_05B, 511, F16
    m = qd.Model(c, act=a, lm_head="int8", max_ctx=P + 1, seed=3, fused=True)
    m.fill_kv(5)
    st = ev.stream()
    for _ in range(3):
        m.step(1, P, st)
    capi.sync()
    call, scale, n = capi.call, float(1.0 / np.sqrt(np.float32(c.head_dim))), ctypes.c_size_t()

    def gu_plan(L, rms, glu):
        g = m.layers[L]["gu"]
        pr = capi.Q8Problem(out=(m.gate if glu else m.gu).ptr, inp=m.x.ptr, residual=None, weight=g.q.ptr,
                            scales=g.s.ptr, bias=None, M=1, N=2 * c.inter, K=c.hidden)
        h = ctypes.c_uint64()
        call("vvh_plan_create", (capi.Q8Problem * 1)(pr), 1, a, a, ctypes.byref(h))
        if rms:
            call("vvh_plan_set_input_op", h.value, capi.IN_RMS_NORM, m.layers[L]["ln2"].ptr, c.eps)
        if glu:
            call("vvh_plan_set_glu", h.value, 0)
        return h.value

    extra = {k: [gu_plan(L, *f) for L in range(c.layers)] for k, f in
             (("rms", (True, False)), ("glu", (False, True)), ("plain", (False, False)))}

    def attn_parts(L, s):
        Ld = m.layers[L]
        call("vvh_attention_parts", m.parts.ptr, m.parts_floats, ctypes.byref(n), m.q.ptr, Ld["kc"].ptr,
             Ld["vc"].ptr, P + 1, c.heads, c.kv_heads, c.head_dim, scale, a, s)

    def o_merge(L, s):
        o = m.layers[L]["o"]
        call("vvh_linear_q8_dev_attn", m.x.ptr, m.parts.ptr, n.value, c.head_dim, o.q.ptr, o.s.ptr, None, m.x.ptr,
             c.hidden, c.hidden, a, s)

    def attention(L, s):
        Ld = m.layers[L]
        call("vvh_attention", m.attn.ptr, m.q.ptr, Ld["kc"].ptr, Ld["vc"].ptr, 1, P + 1, c.heads, c.kv_heads,
             c.head_dim, scale, a, s)

    def lin(name, out, inp, res, N, K):
        def f(L, s):
            w = m.layers[L][name]
            call("vvh_linear_q8_dev", out.ptr, inp.ptr, w.q.ptr, w.s.ptr, None, res.ptr if res else None, 1, N, K,
                 a, a, s)
        return f

    ops = [("near-empty kernel (one-element fill)",
            lambda L, s: call("vvh_fill_normal", m.token.ptr, F32, 1, 1, 0.0, 1.0, s)),
           ("q/k/v plan (RMSNorm stage, RoPE + K/V append)", lambda L, s: call("vvh_plan_run_pos", m.plans[L], P, s)),
           ("attention parts", attn_parts),
           ("o + attention merge stage", o_merge),
           ("gate/up plan (RMSNorm stage, SiLU-gated)", lambda L, s: call("vvh_plan_run", m.mlp_plans[L], s)),
           ("down (+ residual)", lin("down", m.x, m.gate, m.x, c.hidden, c.inter)),
           ("one-launch attention (vvh_attention)", attention),
           ("o (+ residual) on that row", lin("o", m.x, m.attn, m.x, c.hidden, c.hidden)),
           ("gate/up plan, RMSNorm stage only", lambda L, s: call("vvh_plan_run", extra["rms"][L], s)),
           ("gate/up plan, SiLU-gated epilogue only", lambda L, s: call("vvh_plan_run", extra["glu"][L], s)),
           ("gate/up plan, neither", lambda L, s: call("vvh_plan_run", extra["plain"][L], s)),
           ("gate/up as one k_dot call", lin("gu", m.gu, m.norm_out, None, 2 * c.inter, c.hidden))]
    out = {}
    for name, f in ops:
        for L in range(c.layers):
            f(L, st)
        capi.sync()
        g = ev.graph(st, lambda s_: [f(L, s_) for L in range(c.layers)])
        for _ in range(3):
            ev.launch(g, st)
        ms = timed(ev, lambda i: ev.launch(g, st), max(args.steps, 10), st)
        ev.drop(g)
        out[name] = round(ms * 1e3 / c.layers, 3)
        print(f"[bench] {name}: {out[name]:.2f} us per call", file=sys.stderr, flush=True)
    for h in extra["rms"] + extra["glu"] + extra["plain"]:
        call("vvh_plan_destroy", h)
    m.close()
    print(json.dumps({"workload": "fused decode step operators, Qwen2.5-0.5B shapes, position 511, 24 layer calls "
                                  "per graph", "us_per_call": out}), flush=True)


def copy_main(args, ev):
    """Calibration of rocprofv3's FETCH_SIZE / WRITE_SIZE: one 256 MiB
    device-to-device copy per step (hipMemcpyAsync, __amd_rocclr_copyBuffer),
    which reads and writes exactly 256 MiB.  Run under rocprofv3 --pmc, the
    counters per copy dispatch against 262144 KiB give the scale factors that
    turn the decode kernel's counters into HBM bytes."""
    nbytes = 256 << 20
    src, dst = capi.DevBuf(nbytes), capi.DevBuf(nbytes)
    capi.call("vvh_fill_normal", src.ptr, F32, nbytes // 4, 1, 0.0, 1.0, None)
    for _ in range(args.warmup):
        capi.call("vvh_memcpy_d2d_async", dst.ptr, src.ptr, nbytes, None)
    ms = timed(ev, lambda i: capi.call("vvh_memcpy_d2d_async", dst.ptr, src.ptr, nbytes, None), args.steps)
    rate = 2 * nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({"workload": "copy calibration", "bytes_read": nbytes, "bytes_written": nbytes,
                      "ms_per_copy": round(ms, 4), "GB_per_s_read_plus_write": round(rate, 1)}), flush=True)


VENDOR_SHAPES = [("gate_up", 128, 4864, 896), ("gate_up", 512, 4864, 896), ("gate_up", 2048, 4864, 896),
                 ("down", 512, 896, 4864), ("down", 2048, 896, 4864), ("gate_up_1.5b", 256, 8960, 1536)]


def vendor_gemm_main(args, ev):
    """Calibration: for each prefill shape, this library's int8 GEMM
    (linear_q8, fp16 activations and output) and the vendor fp16 GEMM
    (torch.matmul on fp16 weights, hipBLASLt) on the same M, N, K, one after
    the other.  The vendor GEMM streams 2 bytes per weight and converts
    nothing; it is the library speed of the same problem on this GPU.  The
    kernel durations come from rocprofv3 --kernel-trace run over this
    workload; the HIP-event times printed here include Python launch gaps
    for the vendor calls (one torch call per launch)."""
    import torch
    out = {}
    tmp_w = capi.DevBuf(8960 * 1536 * 4)
    for name, M, N, K in VENDOR_SHAPES:
        reps = []
        for r in range(2):
            ar = Arena(arena_size(Linear.sizes(M, N, K, False)))
            reps.append((ar, Linear(ar, tmp_w, M, N, K, False, name.startswith("down"), 900 + r)))
        for i in range(args.warmup):
            reps[i % 2][1].run()
        ms = timed(ev, lambda i: reps[i % 2][1].run(), args.steps)
        del reps
        As = [torch.randn(M, K, device="cuda", dtype=torch.float16) for _ in range(2)]
        Ws = [torch.randn(N, K, device="cuda", dtype=torch.float16) for _ in range(8)]  # 8 x N x K x 2 bytes
        for i in range(args.warmup):
            torch.matmul(As[i % 2], Ws[i % 8].t())
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(args.steps):
            torch.matmul(As[i % 2], Ws[i % 8].t())
        b.record()
        torch.cuda.synchronize()
        vms = a.elapsed_time(b) / args.steps
        del As, Ws
        fl = 2 * M * N * K
        out[f"{name}_M{M}"] = {"M": M, "N": N, "K": K, "kernel": kernel_name(M, N, K),
                               "int8_us_events": round(ms * 1e3, 2),
                               "int8_TFLOPS": round(fl / (ms * 1e-3) / 1e12, 1),
                               "vendor_fp16_us_events_incl_launch_gaps": round(vms * 1e3, 2)}
        print(f"[bench] {name} M={M}: int8 {ms * 1e3:.2f} us, vendor fp16 {vms * 1e3:.2f} us (events)",
              file=sys.stderr, flush=True)
    print(json.dumps({"workload": "vendor-gemm calibration", "shapes": out}), flush=True)


def extras(ev, sets, projs, tmp_w, args):
    out = {}
    L = QWEN05["layers"]
    step_bytes = sum(l.bytes for l in sets[0][1])
    # (0) the same grouped step with the other decode kernel families
    for fam, kern in (("skinny", capi.KERNEL_SKINNY), ("stream", capi.KERNEL_STREAM)):
        alt = [make_plan(lins, kernel=kern) for _, lins in sets]
        for i in range(5):
            capi.call("vvh_plan_run", alt[i % len(alt)], None)
        ms = timed(ev, lambda i: capi.call("vvh_plan_run", alt[i % len(alt)], None), max(args.steps // 2, 20))
        out[f"decode_set_{fam}"] = {"kernel": KERNEL_SYMBOL[capi.plan_kernel(alt[0])], "ms_per_step": round(ms, 5),
                                    "GBps": round(step_bytes / (ms * 1e-3) / 1e9, 2)}
        for h in alt:
            capi.call("vvh_plan_destroy", h)
    # (1) model order: q/k/v grouped, o, gate+up grouped, down -> 4 launches/layer
    order_plans = []
    for _, lins in sets:
        seq = []
        for l in range(L):
            q, k, v, o, g, u, d = lins[7 * l: 7 * l + 7]
            seq += [("plan", make_plan([q, k, v])), ("lin", o), ("plan", make_plan([g, u])), ("lin", d)]
        order_plans.append(seq)

    def model_step_on(seq, stream):
        for kind, item in seq:
            if kind == "plan":
                capi.call("vvh_plan_run", item, stream)
            else:
                item.run(stream)

    def model_step(i):
        model_step_on(order_plans[i % len(order_plans)], None)

    for i in range(5):
        model_step(i)
    reps = max(args.steps // 4, 20)
    ms = timed(ev, model_step, reps)
    out["model_order"] = {"launches_per_step": 4 * L, "ms_per_step": round(ms, 5),
                          "GBps": round(step_bytes / (ms * 1e-3) / 1e9, 2),
                          "note": "launched one by one from Python: the host launch rate bounds it"}
    print(f"[bench] model order {ms * 1e3:.1f} us", file=sys.stderr, flush=True)

    # the same 96 launches captured in a HIP graph per replica (GPU-side time,
    # with the per-kernel launch floor of a graph replay)
    stream = ev.stream()
    graphs = [ev.graph(stream, lambda st, seq=seq: model_step_on(seq, st)) for seq in order_plans]
    for i in range(5):
        ev.launch(graphs[i % len(graphs)], stream)
    ms = timed(ev, lambda i: ev.launch(graphs[i % len(graphs)], stream), reps, stream)
    ev.drop(*graphs)
    for seq in order_plans:
        for kind, item in seq:
            if kind == "plan":
                capi.call("vvh_plan_destroy", item)
    out["model_order_graph"] = {"launches_per_step": 4 * L, "ms_per_step": round(ms, 5),
                                "GBps": round(step_bytes / (ms * 1e-3) / 1e9, 2)}
    print(f"[bench] model order (graph) {ms * 1e3:.1f} us", file=sys.stderr, flush=True)

    # (2) per-call time of each projection: its 24 single calls (one per layer)
    # captured in a graph per replica, replayed; us per call = replay / 24
    nproj = len(projs)
    calls = {}
    for pi, (name, N, K, bias, res) in enumerate(projs):
        pg = [ev.graph(stream, lambda st, lins=lins: [lins[7 * l + pi].run(st) for l in range(L)])
              for _, lins in sets]
        for i in range(3):
            ev.launch(pg[i % len(pg)], stream)
        ms = timed(ev, lambda i: ev.launch(pg[i % len(pg)], stream), 30, stream)
        ev.drop(*pg)
        us = ms * 1e3 / L
        b = algo_bytes(1, N, K, bias, res)
        calls[name] = {"N": N, "K": K, "us": round(us, 2), "GBps": round(b / (us * 1e-6) / 1e9, 1),
                       "kernel": capi.kernel_choice(1, N, K, F16, F16)}
    out["per_call_graph"] = calls

    # (3) LM head GEMV, configs[2]: K=896, N=151936, fp16 act, fp32 logits
    N, K = 151936, 896
    _ar, heads = rotation(tmp_w, 1, N, K, False, False, 777, F16, F32)
    us = graph_rotation(ev, heads, stream) * 1e3
    b = heads[0].bytes
    out["lm_head"] = {"N": N, "K": K, "replicas_rotated": len(heads), "us": round(us, 2),
                      "GBps": round(b / (us * 1e-6) / 1e9, 1),
                      "hbm_frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                      "kernel": capi.kernel_choice(1, N, K, F16, F32)}
    del heads, _ar
    print(f"[bench] lm head {us:.1f} us", file=sys.stderr, flush=True)

    # (4) prefill GEMM, configs[3]
    gemm = {}
    for M in (128, 512, 2048):
        for name, N, K, res in (("gate_up", QWEN05["inter"], QWEN05["hidden"], False),
                                ("down", QWEN05["hidden"], QWEN05["inter"], True)):
            _ar, reps = rotation(tmp_w, M, N, K, False, res, 900)
            us = graph_rotation(ev, reps, stream) * 1e3
            tf = reps[0].flops / (us * 1e-6) / 1e12
            del reps, _ar
            gemm[f"{name}_M{M}"] = {"M": M, "N": N, "K": K, "us": round(us, 2), "TFLOPS": round(tf, 1),
                                    "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                                    "kernel": kernel_name(M, N, K)}
    out["prefill_gemm"] = gemm
    print(f"[bench] gemm M512 gate_up {gemm['gate_up_M512']['us']} us", file=sys.stderr, flush=True)

    # (4b) fp32 activations (the reference's default mode) on the prefill
    # shapes: the dispatched kernel (the MFMA GEMM on split fp16 high/low
    # parts from M = 32) beside the fp32 VALU kernel forced, across the
    # crossover
    f32 = {}
    for M in (8, 16, 32, 64, 128, 512, 2048):
        for name, N, K, res in (("gate_up", QWEN05["inter"], QWEN05["hidden"], False),
                                ("down", QWEN05["hidden"], QWEN05["inter"], True)):
            if name == "down" and M not in (32, 512, 2048):
                continue
            _ar, reps = rotation(tmp_w, M, N, K, False, res, 950, F32, F32)
            row = {"M": M, "N": N, "K": K, "kernel": capi.kernel_choice(M, N, K, F32, F32)}
            for fam, kern in (("auto", capi.KERNEL_AUTO), ("gemm", capi.KERNEL_GEMM),
                              ("gemv_f32", capi.KERNEL_GEMV_F32)):
                capi.set_kernel(kern)
                try:
                    us = graph_rotation(ev, reps, stream) * 1e3
                finally:
                    capi.set_kernel(capi.KERNEL_AUTO)
                row[f"{fam}_us"] = round(us, 2)
                row[f"{fam}_TFLOPS"] = round(reps[0].flops / (us * 1e-6) / 1e12, 1)
            del reps, _ar
            f32[f"{name}_M{M}"] = row
    out["prefill_gemm_f32"] = f32
    print(f"[bench] fp32 gemm M512 gate_up {f32['gate_up_M512']['auto_us']} us "
          f"(fp32 VALU kernel {f32['gate_up_M512']['gemv_f32_us']} us)", file=sys.stderr, flush=True)

    # (4c) the decode families side by side at small M (fp16), Qwen2.5-1.5B
    # shapes: the measurement behind the crossovers of the dispatcher
    fams = {}
    for name, N, K in (("qo", 1536, 1536), ("gate_up", 8960, 1536), ("down", 1536, 8960)):
        for M in (1, 2, 4, 8, 16, 32):
            _ar, reps = rotation(tmp_w, M, N, K, False, False, 1300)
            row = {"auto": kernel_name(M, N, K)}
            for fam, kern in (("dot", capi.KERNEL_DOT), ("skinny", capi.KERNEL_SKINNY),
                              ("stream", capi.KERNEL_STREAM), ("gemm", capi.KERNEL_GEMM)):
                if capi.load().vvh_linear_q8_choice(M, N, K, F16, F16) < 0:
                    continue
                capi.set_kernel(kern)
                try:
                    if capi.kernel_choice(M, N, K, F16, F16) != fam:
                        continue
                    row[f"{fam}_us"] = round(graph_rotation(ev, reps, stream) * 1e3, 2)
                finally:
                    capi.set_kernel(capi.KERNEL_AUTO)
            del reps, _ar
            fams[f"{name}_M{M}"] = row
    out["decode_families"] = fams

    # (5) Qwen2.5-1.5B shapes, M sweep
    sweep = {}
    for M in (1, 4, 16, 64, 256):
        for name, N, K in (("qo", 1536, 1536), ("kv", 256, 1536), ("gate_up", 8960, 1536), ("down", 1536, 8960)):
            _ar, reps = rotation(tmp_w, M, N, K, False, False, 1300)
            us = graph_rotation(ev, reps, stream) * 1e3
            l = reps[0]
            del reps, _ar
            sweep[f"{name}_M{M}"] = {"us": round(us, 2), "GBps": round(l.bytes / (us * 1e-6) / 1e9, 1),
                                     "TFLOPS": round(l.flops / (us * 1e-6) / 1e12, 2),
                                     "kernel": kernel_name(M, N, K)}
    out["qwen15_sweep"] = sweep

    # (6) weight ingestion: host BF16 rows of 4 layers quantized into device mirrors
    layers = [bf16_layer_rows(projs, 100 + l) for l in range(4)]
    nbytes = sum(b.nbytes for rows in layers for *_, b in rows)
    scales = [[np.empty(N, np.float32) for _, N, K, _b in rows] for rows in layers]
    h = ctypes.c_uint64()
    handles = []
    t0 = time.perf_counter()
    for rows, sc in zip(layers, scales):
        for (_, N, K, bits), s_ in zip(rows, sc):
            capi.call("vvh_weight_ingest", bits.ctypes.data, capi.BF16, None, N, K, s_.ctypes.data, ctypes.byref(h))
            handles.append(h.value)
    el = time.perf_counter() - t0
    for hv in handles:
        capi.call("vvh_weight_release", hv)
    out["weight_ingest"] = {"layers": 4, "bf16_bytes": nbytes, "seconds": round(el, 4),
                            "GBps": round(nbytes / el / 1e9, 2),
                            "note": "host BF16 rows (pageable numpy memory) -> pinned staging -> device quantizer; "
                                    "wall time including the host copies"}
    print(f"[bench] weight ingest {nbytes / el / 1e9:.1f} GB/s", file=sys.stderr, flush=True)

    # (7) a whole decode step at Qwen2.5-0.5B shapes: every operator of
    # transformer_forward on the device (vvllm_amd.qwen2_decode), at position
    # 511 of a filled KV cache, launched from Python and replayed from a graph;
    # "fused": the same arithmetic with the norms and SiLU-mul in the input
    # stage of the following linear and RoPE writing the KV cache (identical
    # logits, fewer launches)
    from vvllm_amd import qwen2_decode as qd
    e2e = {}
    for head, fused in (("dense", False), ("int8", False), ("dense", True), ("int8", True)):
        m = qd.Model(qd.QWEN25_05B, act=F16, lm_head=head, max_ctx=1024, seed=3, fused=fused)
        m.fill_kv(5)
        P = 511
        for i in range(3):
            m.step(1, P)
        ms_eager = timed(ev, lambda i: m.step(1, P), 10)
        m.step(1, P, stream)  # sizes the capture stream's workspace before capture
        capi.sync()
        g = ev.graph(stream, lambda st: m.step(1, P, st))
        for i in range(3):
            ev.launch(g, stream)
        ms_graph = timed(ev, lambda i: ev.launch(g, stream), 50, stream)
        ev.drop(g)
        e2e[f"{head}_lm_head" + ("_fused" if fused else "")] = {"calls_per_step": m.calls_per_step(), "position": P,
                                  "us_per_token_graph": round(ms_graph * 1e3, 1),
                                  "tok_per_s_graph": round(1e3 / ms_graph, 1),
                                  "us_per_token_python_launches": round(ms_eager * 1e3, 1)}
        m.close()
        del m
        print(f"[bench] decode step ({head} LM head{', fused' if fused else ''}) {ms_graph * 1e3:.0f} us graph, "
              f"{ms_eager * 1e3:.0f} us eager", file=sys.stderr, flush=True)
    e2e["note"] = ("synthetic Qwen2.5-0.5B-shaped model (seeded weights), fp16 activations, int8 linears, greedy "
                   "argmax on the device; GPU time per token, no host sampling or tokenizer")
    out["decode_step"] = e2e
    return out


if __name__ == "__main__":
    main()
