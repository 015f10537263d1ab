"""GPU parity of the linear_q8 path against the CPU oracle, through the C ABI.

Bars: int8 codes and scales bit-exact; normalized max
error max|y - r| / max|r| <= 1e-4 for fp32 activations and <= 2e-3 for fp16
activations (or fp16 outputs), where r is the oracle (the reference's
BackendCPU::linear_q8 restated, oracle/oracle.c) on the same inputs; fp16
activations are handed to the oracle widened to fp32, which is exact.

Every kernel family is forced over shapes that hit its edges (K tails,
N % 16 != 0, M around the 16-row crossover, K == 0, misaligned pointers), and
the automatic dispatch is run at every BASELINE.json config shape.
"""
import ctypes
import functools
import os

import numpy as np
import pytest

from vvllm_amd import capi

pytestmark = pytest.mark.gpu

F32, F16 = capi.F32, capi.F16
TOL_F32, TOL_F16 = 1e-4, 2e-3
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@functools.lru_cache(maxsize=None)
def weights(N, K, seed, oracle_mod):
    rng = np.random.default_rng(seed)
    w = rng.normal(0.0, 0.02, (N, K)).astype(np.float32)
    q, s = oracle_mod.quantize_per_channel(w)
    b = rng.normal(0.0, 0.01, N).astype(np.float32)
    return q, s, b


def npd(d):
    return np.float32 if d == F32 else np.float16


def run_case(oracle, M, N, K, act=F16, outd=F16, bias=True, res=None, kernel=capi.KERNEL_AUTO,
             seed=0, rows=None, x_offset=0):
    """res: None | "sep" | "inplace".  rows: subset of rows checked against
    the oracle (all rows when None).  x_offset: byte offset of the activation
    base (misalignment test)."""
    print(f"[case] M={M} N={N} K={K} act={act} out={outd} bias={bias} res={res} "
          f"kernel={capi.KERNEL_NAMES[kernel]} seed={seed}", flush=True)
    q, s, b = weights(N, K, seed, oracle)
    rng = np.random.default_rng(seed + 1000)
    x = rng.normal(0.0, 1.0, (M, K)).astype(np.float32).astype(npd(act))
    r = rng.normal(0.0, 1.0, (M, N)).astype(np.float32).astype(npd(outd)) if res else None
    d_q, d_s = capi.DevBuf.from_array(q), capi.DevBuf.from_array(s)
    d_b = capi.DevBuf.from_array(b) if bias else None
    d_x = capi.DevBuf(x.nbytes + 64)
    capi.call("vvh_memcpy_h2d", d_x.addr(x_offset), x.ctypes.data, x.nbytes) if x.nbytes else None
    d_r = capi.DevBuf.from_array(r) if res == "sep" else None
    d_y = capi.DevBuf.from_array(r) if res == "inplace" else capi.DevBuf(max(M * N * np.dtype(npd(outd)).itemsize, 1))
    capi.set_kernel(kernel)
    try:
        capi.linear_q8_dev(d_y, d_x.addr(x_offset), d_q, d_s, d_b, d_y if res == "inplace" else d_r,
                           M, N, K, act, outd)
        capi.sync()
    finally:
        capi.set_kernel(capi.KERNEL_AUTO)
    y = d_y.to_array(npd(outd), (M, N)).astype(np.float32)
    sel = np.arange(M) if rows is None else np.asarray(rows)
    ref = oracle.linear_q8(x[sel].astype(np.float32), q, s, b if bias else None,
                           None if r is None else r[sel].astype(np.float32))
    got = y[sel]
    scale = max(float(np.abs(ref).max()), 1e-30)
    err = float(np.abs(got - ref).max()) / scale
    tol = TOL_F32 if (act == F32 and outd == F32) else TOL_F16
    assert np.isfinite(got).all()
    assert err <= tol, f"normalized max error {err:.3e} > {tol:.0e}"
    if outd == F32:
        check_f32_bound(got, ref, x[sel], q, s, b if bias else None, None if r is None else r[sel], K)
    return err


def check_f32_bound(got, ref, x, q, s, b, r, K):
    """fp32 outputs carry no final fp16 rounding, so they are held to the
    fp32 accumulation bound of the oracle's own tests: both sides sum K exact
    (fp16 x int8) or once-rounded (fp32 x int8) products in fp32, so each is
    within K * 2^-24 * sum_k |x q| * scale of the exact value, plus the
    roundings of the epilogue (scale, bias, residual).  A lost k tail, a
    dropped term or fp16 partial sums exceed it by orders of magnitude."""
    mag = (np.abs(x.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * np.abs(s.astype(np.float64))
    extra = np.abs(ref.astype(np.float64))
    if b is not None:
        extra = extra + np.abs(b.astype(np.float64))
    if r is not None:
        extra = extra + np.abs(r.astype(np.float64))
    bound = 2.0 * K * 2.0 ** -24 * mag + 2.0 ** -22 * extra + 1e-30
    diff = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    worst = float((diff / bound).max()) if diff.size else 0.0
    assert worst <= 1.0, f"fp32 output off the fp32 accumulation bound by {worst:.2f}x"


# ---------------------------------------------------------------------------
# BASELINE.json configs, automatic dispatch
# ---------------------------------------------------------------------------
def test_config1_fp32_decode(gpu, oracle):
    """M=1, K=N=896, fp32 activations/outputs, bias."""
    assert capi.kernel_choice(1, 896, 896, F32, F32) == "gemv_f32"
    run_case(oracle, 1, 896, 896, F32, F32, bias=True, seed=11)


QWEN05_LAYER = [  # (name, N, K, bias, residual)
    ("q", 896, 896, True, None), ("k", 128, 896, True, None), ("v", 128, 896, True, None),
    ("o", 896, 896, False, "inplace"), ("gate", 4864, 896, False, None), ("up", 4864, 896, False, None),
    ("gate_up", 9728, 896, False, None), ("down", 896, 4864, False, "inplace"),
]


@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("proj", QWEN05_LAYER, ids=[p[0] for p in QWEN05_LAYER])
def test_config2_qwen05_decode(gpu, oracle, proj, outd):
    name, N, K, bias, res = proj
    seed = 200 + [p[0] for p in QWEN05_LAYER].index(name)  # fixed per projection: a failure replays
    run_case(oracle, 1, N, K, F16, outd, bias=bias, res=res, seed=seed)


def test_config3_lm_head(gpu, oracle):
    """M=1, K=896, N=151936, fp16 activations, fp32 logits."""
    run_case(oracle, 1, 151936, 896, F16, F32, bias=False, seed=33)


@pytest.mark.parametrize("M", [128, 512, 2048])
@pytest.mark.parametrize("shape", [(4864, 896), (896, 4864)], ids=["gate_up", "down"])
def test_config4_prefill(gpu, oracle, M, shape):
    N, K = shape
    rows = None if M <= 512 else [0, 1, 127, 128, 129, 511, 1023, 1024, 1500, 2046, 2047]
    run_case(oracle, M, N, K, F16, F16, bias=False, res="inplace" if K == 4864 else None, seed=44, rows=rows)


QWEN15 = [("qo", 1536, 1536), ("kv", 256, 1536), ("gate_up", 8960, 1536), ("down", 1536, 8960)]


@pytest.mark.parametrize("M", [1, 4, 16, 64, 256])
@pytest.mark.parametrize("proj", QWEN15, ids=[p[0] for p in QWEN15])
def test_config5_qwen15_sweep(gpu, oracle, proj, M):
    name, N, K = proj
    rows = None if M * N * K < 2e9 else list(range(0, M, 17))
    run_case(oracle, M, N, K, F16, F16, bias=(name == "kv"), seed=55, rows=rows)


# ---------------------------------------------------------------------------
# every kernel family over its edges
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("act,outd", [(F32, F32), (F16, F16), (F16, F32)])
@pytest.mark.parametrize("M,N,K", [(1, 3, 4), (1, 2, 2), (2, 17, 33), (3, 40, 100), (1, 5, 0), (4, 64, 896)])
def test_generic_kernel(gpu, oracle, M, N, K, act, outd):
    run_case(oracle, M, N, K, act, outd, bias=True, res="sep", kernel=capi.KERNEL_GENERIC, seed=M + N + K)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 9, 20])
@pytest.mark.parametrize("N,K", [(1, 16), (17, 80), (896, 896), (130, 4864)])
def test_gemv_f32_kernel(gpu, oracle, M, N, K):
    run_case(oracle, M, N, K, F32, F32, bias=True, res="inplace" if M % 2 else None,
             kernel=capi.KERNEL_GEMV_F32, seed=7 * M + N)


@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("M", [1, 2, 4, 7, 15, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("N,K", [(1, 16), (17, 48), (128, 896), (896, 4864), (300, 1040), (40, 128)])
def test_skinny_kernel(gpu, oracle, M, N, K, outd):
    """One 16-row MFMA operand of activations (M <= 16), or 2 and 4 groups of
    16 rows against each weight chunk (M = 17..64), ragged in every
    dimension; K = 128 at M = 64 is 16 KB of activations whose padded rows
    would not fit the LDS staging area (read through the caches instead)."""
    run_case(oracle, M, N, K, F16, outd, bias=bool(M % 2), res=["sep", "inplace", None][M % 3],
             kernel=capi.KERNEL_SKINNY, seed=3 * M + K)


@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("M", [1, 17, 64, 130, 300])
@pytest.mark.parametrize("N,K", [(17, 16), (128, 80), (896, 896), (250, 4864)])
def test_gemm_kernel(gpu, oracle, M, N, K, outd):
    run_case(oracle, M, N, K, F16, outd, bias=bool(M % 2), res=["sep", "inplace", None][M % 3],
             kernel=capi.KERNEL_GEMM, seed=5 * M + N)


@pytest.mark.parametrize("res", ["sep", "inplace"])
@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("M,N,K,variant", [(256, 768, 512, "k_gemm3 64x64"), (256, 4864, 512, "k_gemm3 64x128"),
                                           (2048, 2304, 128, "k_gemm3 128x192"), (300, 776, 256, "k_gemm3 64x64"),
                                           (300, 3500, 256, "k_gemm3 64x128"), (1024, 2176, 256, "k_gemm3 128x128"),
                                           (1000, 2200, 256, "k_gemm3 128x128")])
def test_gemm3_epilogue(gpu, oracle, M, N, K, variant, outd, res):
    """k_gemm3's epilogue with bias and residual together, on every tile
    shape the dispatch picks: tiles wholly inside the problem take the
    branch-free path, the others (M = 300 with N = 776 or 3500, M = 1000
    with N = 2200: partial rows and columns) the general one."""
    assert capi.gemm_variant(M, N, K) == variant
    rows = None if M <= 300 else [r for r in (0, 1, 63, 64, 127, 128, 1000, 1919, 1920) if r < M] + [M - 1]
    run_case(oracle, M, N, K, F16, outd, bias=True, res=res, kernel=capi.KERNEL_GEMM, seed=M + K, rows=rows)


def reduce_groups(M, N, splits):
    """Split groups per block of the split-K reduction (k_splitk_reduce8):
    4 or 2 when one group's blocks would be few (< 128) and carry 8+ or 4+
    splits each, else 1."""
    blocks1 = (M * (N // 8) + 255) // 256
    return 1 if blocks1 >= 128 else 4 if splits >= 8 else 2 if splits >= 4 else 1


@pytest.mark.parametrize("res", ["sep", "inplace", None])
@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("M,N,K,splits,groups", [(24, 1544, 8960, 10, 4), (56, 904, 4864, 11, 4), (72, 1032, 3072, 7, 2),
                                                 (100, 1000, 1536, 4, 2), (200, 1000, 1536, 3, 1)])
def test_splitk_reduce_groups(gpu, oracle, M, N, K, splits, groups, outd, res):
    """The split-K reduction with 4, 2 and 1 split groups per block: groups
    of unequal split counts (10 over 4: 2, 3, 2, 3; 11; 7 over 2: 3, 4) and a
    last block whose chunk count leaves threads of every group idle."""
    assert capi.gemm_variant(M, N, K) == f"k_gemm3 64x64 split {splits}"
    assert reduce_groups(M, N, splits) == groups
    assert (M * N // 8) % (256 // groups) != 0
    run_case(oracle, M, N, K, F16, outd, bias=bool(M % 3), res=res, kernel=capi.KERNEL_GEMM, seed=M + N + splits)


@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("M", [1, 2, 4, 5, 16])
@pytest.mark.parametrize("N,K", [(1, 512), (17, 592), (130, 896), (896, 4864), (300, 1040), (4099, 768)])
def test_stream_kernel(gpu, oracle, M, N, K, outd):
    """Persistent streaming decode forced on shapes with K tails (592, 1040),
    N % 16 != 0, a single tile, and the 8- and 12-deep pipelines."""
    run_case(oracle, M, N, K, F16, outd, bias=bool(M % 2), res=["sep", "inplace", None][(M + N) % 3],
             kernel=capi.KERNEL_STREAM, seed=11 * M + K)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 12, 16])
@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("N,K", [(1, 16), (17, 48), (128, 896), (896, 4864), (300, 1040), (4099, 592),
                                 (64, 20480), (33, 8960), (48, 2048)])
def test_dot_kernel(gpu, oracle, M, N, K, outd):
    """Dot-product decode (v_dot2 for M <= 2, MFMA for 3 <= M <= 16): K tails
    (48, 592, 1040), a single 16-code step, N % 16 != 0, activations too
    large for LDS (K = 20480 at M >= 2) and the ksplit reduction (few
    tiles)."""
    run_case(oracle, M, N, K, F16, outd, bias=bool(N % 2), res=["sep", "inplace", None][(N + K + M) % 3],
             kernel=capi.KERNEL_DOT, seed=13 * N + K + M)


def dot_x_reread_bytes(M, N, K):
    """Activation bytes a k_dot launch's 16-row tiles re-read (each tile
    reads all M rows); from 5 MB, launches that load the activations with
    the weights take them in whole lines through the wave's LDS tile, when
    their waves have at most 12 k steps each (48 at ksplit 4)."""
    return -(-N // 16) * M * K * 2


@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("M,N,K", [(16, 4099, 1040), (12, 896, 4864), (5, 8960, 1040), (4, 8960, 1536),
                                   (3, 8960, 1616), (16, 8960, 1536)])
def test_dot_activation_tile(gpu, oracle, M, N, K, outd):
    """k_dot's MFMA path with its activations loaded in whole lines and
    regathered through LDS (4-, 8- and 16-row instantiations; K tails of
    16 and 80 codes past a step at K = 1040 and 1616; N % 16 != 0)."""
    assert dot_x_reread_bytes(M, N, K) >= 5 << 20 and -(-K // 128) <= 48
    run_case(oracle, M, N, K, F16, outd, bias=bool(M % 2), res=["sep", "inplace", None][(N + M) % 3],
             kernel=capi.KERNEL_DOT, seed=17 * M + N)


def dot_split8(M, N, K, cus=256):
    """Whether a plain k_dot call runs blocks of 8 waves (k split 8): 9-16
    rows over at most one block per CU whose waves would have exactly 3 k
    steps each at k split 4 (K of 1025-1536)."""
    tiles = -(-N // 16)
    return 8 < M <= 16 and tiles <= cus and -(-(-(-K // 128)) // 4) == 3


@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("M,N,K", [(16, 1536, 1536), (9, 256, 1536), (12, 300, 1040), (13, 4095, 1152),
                                   (16, 4096, 1536), (11, 17, 1424)])
def test_dot_split8(gpu, oracle, M, N, K, outd):
    """k_dot's 8-wave blocks: one 16-row tile per block, its k steps over 8
    waves (waves past the k range idle), the 8 partial tiles added in wave
    order; N % 16 != 0, K tails of 16 and 16 + 64 codes, the activation
    tile (4096 x 1536 at M = 16 re-reads 12.6 MB of activations)."""
    assert dot_split8(M, N, K)
    assert capi.kernel_choice(M, N, K, F16, outd) == "dot"
    run_case(oracle, M, N, K, F16, outd, bias=bool(N % 2), res=["sep", "inplace", None][(M + N) % 3],
             kernel=capi.KERNEL_AUTO, seed=19 * M + K)


def test_decode_dispatch_on_device(gpu):
    assert capi.kernel_choice(1, 151936, 896, F16, F32) == "dot"
    assert capi.kernel_choice(1, 9728, 896, F16, F16) == "dot"
    assert capi.kernel_choice(2, 896, 896, F16, F16) == "dot"
    assert capi.kernel_choice(4, 896, 896, F16, F16) == "dot"
    assert capi.kernel_choice(4, 1536, 8960, F16, F16) == "dot"
    assert capi.kernel_choice(4, 9728, 896, F16, F16) == "dot"
    assert capi.kernel_choice(4, 17920, 1536, F16, F16) == "dot"
    assert capi.kernel_choice(5, 1536, 8960, F16, F16) == "dot"
    assert capi.kernel_choice(8, 896, 4864, F16, F16) == "dot"
    assert capi.kernel_choice(8, 17920, 1536, F16, F16) == "dot"
    assert capi.kernel_choice(8, 151936, 896, F16, F16) == "dot"
    assert capi.kernel_choice(16, 896, 4864, F16, F16) == "dot"
    assert capi.kernel_choice(9, 1536, 8960, F16, F16) == "dot"
    assert capi.kernel_choice(13, 1536, 8960, F16, F16) == "gemm"
    assert capi.kernel_choice(5, 151936, 896, F16, F16) == "dot"
    assert capi.kernel_choice(16, 4864, 896, F16, F16) == "dot"
    assert capi.kernel_choice(16, 17920, 1536, F16, F16) == "dot"
    assert capi.kernel_choice(11, 1536, 8960, F16, F16) == "gemm"
    assert capi.kernel_choice(64, 1152, 896, F16, F16) == "skinny"
    assert capi.kernel_choice(64, 1536, 1536, F16, F16) == "gemm"


@pytest.mark.parametrize("M,N,K,family", [(8, 17920, 1536, "dot"), (16, 17920, 1536, "dot"), (3, 17920, 1536, "dot"),
                                          (10, 1536, 8960, "dot"), (11, 1536, 8960, "gemm"), (4, 32768, 2048, "skinny"),
                                          (16, 896, 4864, "dot"), (13, 896, 4864, "dot"), (13, 1536, 8960, "gemm"),
                                          (9, 8960, 1536, "dot"), (16, 1536, 1536, "dot"), (16, 9728, 896, "dot"),
                                          (64, 1152, 896, "skinny"), (33, 1536, 1536, "skinny")])
def test_dispatch_edges_parity(gpu, oracle, M, N, K, family):
    """The automatic choice at the edges of the small-M dispatch rules, each
    against the oracle as dispatched (bias and residual on)."""
    assert capi.kernel_choice(M, N, K, F16, F16) == family
    run_case(oracle, M, N, K, F16, F16, bias=True, res="sep", kernel=capi.KERNEL_AUTO, seed=17 * M + N)


def random_shapes(n=40, seed=20261202):
    """Seeded shapes over the automatic dispatch: M across every small-M rule
    (1-17 rows) and into the GEMM, K up to 10240 with some K % 16 != 0 (the
    generic kernel), N up to 16 M codes per call, fp32 activations and fp32
    outputs, bias and residual (separate or in place) drawn per case."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.choice([1, 1, 2, 3, 4, 5, 6, 8, 9, 11, 12, 13, 16, 17, 24, 40, 96]))
        K = int(rng.integers(1, 641)) * 16
        if rng.random() < 0.12:
            K = max(1, K - int(rng.integers(1, 16)))
        N = int(rng.integers(1, 1 + min(40000, 16_000_000 // K)))
        act = F32 if rng.random() < 0.15 else F16
        outd = F32 if rng.random() < 0.4 else F16
        out.append((M, N, K, act, outd, bool(rng.random() < 0.6), ["sep", "inplace", None][int(rng.integers(3))]))
    return out


@pytest.mark.parametrize("i", range(40))
def test_auto_dispatch_random_shapes(gpu, oracle, i):
    """Whatever family the automatic dispatch picks for a seeded random shape
    (with its split count, ring depth, first stage and activation tile),
    against the oracle."""
    M, N, K, act, outd, bias, res = random_shapes()[i]
    run_case(oracle, M, N, K, act, outd, bias=bias, res=res, kernel=capi.KERNEL_AUTO, seed=1000 + i)


def test_random_shapes_cover_the_families():
    """The seeded draw reaches every family the automatic dispatch picks
    (the streaming kernel runs only when forced)."""
    fams = {capi.kernel_choice(M, N, K, act, outd) for M, N, K, act, outd, _, _ in random_shapes()}
    assert fams == {"dot", "gemm", "skinny", "generic", "gemv_f32"}


def test_misaligned_activations_fall_back(gpu, oracle):
    """A 2-byte-offset fp16 activation base cannot take 16-byte loads: the
    dispatcher must route it to the generic kernel and stay correct."""
    run_case(oracle, 1, 64, 896, F16, F16, x_offset=2, seed=9)
    run_case(oracle, 20, 64, 896, F16, F16, x_offset=2, seed=9)


# ---------------------------------------------------------------------------
# device quantizer: bit-exact codes and scales
# ---------------------------------------------------------------------------
def _quantize_dev(w):
    N, K = w.shape
    d_w = capi.DevBuf.from_array(w)
    d_q, d_s = capi.DevBuf(max(N * K, 1)), capi.DevBuf(N * 4)
    capi.call("vvh_quantize_per_channel", d_w.ptr, N, K, d_q.ptr, d_s.ptr, None)
    capi.sync()
    return d_q.to_array(np.int8, (N, K)), d_s.to_array(np.float32, (N,))


def test_device_quantizer_golden(gpu):
    d = np.load(os.path.join(GOLDEN, "quantize_ref.npz"))
    for name in sorted({k[2:-2] for k in d.files if k.endswith("_w")}):
        print(f"[case] quantize golden {name}", flush=True)
        q, s = _quantize_dev(d[f"q_{name}_w"])
        np.testing.assert_array_equal(q, d[f"q_{name}_codes"], err_msg=name)
        np.testing.assert_array_equal(s.view(np.uint32), d[f"q_{name}_scales"].view(np.uint32), err_msg=name)


@pytest.mark.parametrize("N,K,std", [(300, 1000, 0.02), (4864, 896, 0.02), (64, 5000, 3.0), (3, 1, 1.0)])
def test_device_quantizer_matches_oracle(gpu, oracle, N, K, std):
    print(f"[case] quantize N={N} K={K}", flush=True)
    rng = np.random.default_rng(N + K)
    w = rng.normal(0, std, (N, K)).astype(np.float32)
    w[0, : min(K, 3)] = [np.float32(127.0 * 0.5)] * min(K, 3)
    q, s = _quantize_dev(w)
    q_ref, s_ref = oracle.quantize_per_channel(w)
    np.testing.assert_array_equal(q, q_ref)
    np.testing.assert_array_equal(s.view(np.uint32), s_ref.view(np.uint32))


# ---------------------------------------------------------------------------
# weight mirror, plans, allocator, conversion, generator
# ---------------------------------------------------------------------------
def test_weight_mirror_handles(gpu, oracle):
    q, s, b = weights(896, 896, 21, oracle)
    q, s, b = q.copy(), s.copy(), b.copy()
    h = ctypes.c_uint64()
    capi.call("vvh_weight_register", q.ctypes.data, s.ctypes.data, b.ctypes.data, 896, 896, ctypes.byref(h))
    h2 = ctypes.c_uint64()
    capi.call("vvh_weight_register", q.ctypes.data, s.ctypes.data, b.ctypes.data, 896, 896, ctypes.byref(h2))
    assert h.value == h2.value  # same tuple -> same mirror
    found = ctypes.c_uint64()
    capi.call("vvh_weight_find", q.ctypes.data, ctypes.byref(found))
    assert found.value == h.value
    x = np.random.default_rng(1).normal(0, 1, (1, 896)).astype(np.float16)
    d_x, d_y = capi.DevBuf.from_array(x), capi.DevBuf(896 * 4)
    capi.call("vvh_linear_q8", d_y.ptr, d_x.ptr, h.value, None, 1, 896, 896, F16, F32, None)
    capi.sync()
    ref = oracle.linear_q8(x.astype(np.float32), q, s, b)
    y = d_y.to_array(np.float32, (1, 896))
    assert np.abs(y - ref).max() / np.abs(ref).max() <= TOL_F16
    # shape mismatch against the mirror is rejected
    assert capi.status_of("vvh_linear_q8", d_y.ptr, d_x.ptr, h.value, None, 1, 448, 896, F16, F32, None) == 1
    # same host pointer, different shape -> replaced mirror, new handle
    h3 = ctypes.c_uint64()
    capi.call("vvh_weight_register", q.ctypes.data, s.ctypes.data, None, 448, 896, ctypes.byref(h3))
    assert h3.value != h.value
    assert capi.status_of("vvh_linear_q8", d_y.ptr, d_x.ptr, h.value, None, 1, 896, 896, F16, F32, None) == 6
    capi.call("vvh_weight_release", h3.value)
    assert capi.status_of("vvh_weight_find", q.ctypes.data, ctypes.byref(found)) == 6


def test_grouped_plan_matches_single_calls(gpu, oracle):
    """One decode layer of Qwen2.5-0.5B (q/k/v with bias, o and down in place,
    gate and up) x 3 layers as one grouped launch."""
    rng = np.random.default_rng(77)
    probs, keep, checks = [], [], []
    for layer in range(3):
        for name, N, K, bias, res in QWEN05_LAYER:
            if name == "gate_up":
                continue
            q, s, b = weights(N, K, 100 + layer, oracle)
            x = rng.normal(0, 1, (1, K)).astype(np.float16)
            r = rng.normal(0, 1, (1, N)).astype(np.float16) if res else None
            d = dict(q=capi.DevBuf.from_array(q), s=capi.DevBuf.from_array(s),
                     b=capi.DevBuf.from_array(b) if bias else None, x=capi.DevBuf.from_array(x),
                     y=capi.DevBuf.from_array(r) if res else capi.DevBuf(N * 2))
            keep.append(d)
            p = capi.Q8Problem(out=d["y"].ptr, inp=d["x"].ptr, residual=d["y"].ptr if res else None,
                               weight=d["q"].ptr, scales=d["s"].ptr, bias=d["b"].ptr if bias else None,
                               M=1, N=N, K=K)
            probs.append(p)
            checks.append((d["y"], x, q, s, b if bias else None, r, N))
    arr = (capi.Q8Problem * len(probs))(*probs)
    plan = ctypes.c_uint64()
    capi.call("vvh_plan_create", arr, len(probs), F16, F16, ctypes.byref(plan))
    n = ctypes.c_int()
    capi.call("vvh_plan_launches", plan.value, ctypes.byref(n))
    assert n.value == 1
    assert capi.plan_kernel(plan.value) == "dot"  # every problem has M = 1
    print("[case] grouped plan run", flush=True)
    capi.call("vvh_plan_run", plan.value, None)
    capi.sync()
    for d_y, x, q, s, b, r, N in checks:
        y = d_y.to_array(np.float16, (1, N)).astype(np.float32)
        ref = oracle.linear_q8(x.astype(np.float32), q, s, b, None if r is None else r.astype(np.float32))
        assert np.abs(y - ref).max() / np.abs(ref).max() <= TOL_F16
    capi.call("vvh_plan_destroy", plan.value)


def _plan_case(oracle, specs, outd, kernel, seed, expect=None):
    """specs: list of (M, N, K, bias, res) with res in {None, "sep", "inplace"}.
    Builds one plan under the forced kernel family, runs it twice (the second
    run must give the same result: a plan is reusable) and checks every
    problem against the oracle.  Returns the plan's launch count."""
    rng = np.random.default_rng(seed)
    probs, checks, keep = [], [], []
    for i, (M, N, K, bias, res) in enumerate(specs):
        q, s, b = weights(N, K, seed + i, oracle)
        x = rng.normal(0, 1, (M, K)).astype(np.float16)
        r = rng.normal(0, 1, (M, N)).astype(npd(outd)) if res else None
        d = dict(q=capi.DevBuf.from_array(q), s=capi.DevBuf.from_array(s),
                 b=capi.DevBuf.from_array(b) if bias else None, x=capi.DevBuf.from_array(x),
                 r=capi.DevBuf.from_array(r) if res == "sep" else None)
        d["y"] = capi.DevBuf.from_array(r) if res == "inplace" else capi.DevBuf(M * N * np.dtype(npd(outd)).itemsize)
        keep.append(d)
        resid = d["y"].ptr if res == "inplace" else (d["r"].ptr if res == "sep" else None)
        probs.append(capi.Q8Problem(out=d["y"].ptr, inp=d["x"].ptr, residual=resid, weight=d["q"].ptr,
                                    scales=d["s"].ptr, bias=d["b"].ptr if bias else None, M=M, N=N, K=K))
        checks.append((d, x, q, s, b if bias else None, r, M, N, res))
    arr = (capi.Q8Problem * len(probs))(*probs)
    plan = ctypes.c_uint64()
    capi.set_kernel(kernel)
    try:
        capi.call("vvh_plan_create", arr, len(probs), F16, outd, ctypes.byref(plan))
    finally:
        capi.set_kernel(capi.KERNEL_AUTO)
    n = ctypes.c_int()
    capi.call("vvh_plan_launches", plan.value, ctypes.byref(n))
    assert capi.plan_kernel(plan.value) == (expect or capi.KERNEL_NAMES[kernel])
    for rep in range(2):
        for d, x, q, s, b, r, M, N, res in checks:
            if res == "inplace":  # restore the residual the previous run overwrote
                capi.call("vvh_memcpy_h2d", d["y"].ptr, r.ctypes.data, r.nbytes)
        print(f"[case] plan run {rep} kernel={capi.KERNEL_NAMES[kernel]} problems={len(specs)}", flush=True)
        capi.call("vvh_plan_run", plan.value, None)
        capi.sync()
        for d, x, q, s, b, r, M, N, res in checks:
            y = d["y"].to_array(npd(outd), (M, N)).astype(np.float32)
            ref = oracle.linear_q8(x.astype(np.float32), q, s, b, None if r is None else r.astype(np.float32))
            err = np.abs(y - ref).max() / np.abs(ref).max()
            assert err <= TOL_F16, (M, N, res, err)
    capi.call("vvh_plan_destroy", plan.value)
    return n.value


MIXED_PLAN = [(1, 896, 896, True, None), (1, 128, 896, True, None), (3, 130, 592, False, "sep"),
              (16, 300, 1040, True, "inplace"), (1, 896, 4864, False, "inplace"), (5, 17, 768, False, None),
              (1, 4864, 896, False, None), (2, 1, 512, True, "sep")]


@pytest.mark.parametrize("outd", [F16, F32])
@pytest.mark.parametrize("kernel", [capi.KERNEL_STREAM, capi.KERNEL_SKINNY], ids=["stream", "skinny_grouped"])
def test_mixed_plan_single_launch(gpu, oracle, kernel, outd):
    """Problems of different M, N, K, bias and residual forms in one launch of
    either decode kernel family."""
    assert _plan_case(oracle, MIXED_PLAN, outd, kernel, seed=300) == 1


DOT_PLAN = [(1, 896, 896, True, None), (1, 128, 896, True, None), (1, 130, 592, False, "sep"),
            (1, 300, 1040, True, "inplace"), (1, 896, 4864, False, "inplace"), (1, 17, 48, False, None),
            (1, 4864, 896, False, None), (1, 1, 512, True, "sep")]
DOT_PLAN_M4 = [(4, 896, 896, True, None), (2, 128, 896, True, "sep"), (3, 300, 1040, False, "inplace"),
               (1, 896, 4864, False, "inplace"), (4, 17, 48, True, None)]
DOT_PLAN_M8 = [(8, 896, 896, True, None), (5, 128, 896, True, "sep"), (7, 300, 1040, False, "inplace"),
               (6, 896, 4864, False, "inplace"), (1, 17, 48, True, None), (3, 130, 592, True, "sep")]
DOT_PLAN_M16 = [(16, 896, 896, True, None), (9, 128, 896, True, "sep"), (12, 300, 1040, False, "inplace"),
                (10, 896, 4864, False, "inplace"), (2, 17, 48, True, None), (16, 64, 20480, True, "sep")]


@pytest.mark.parametrize("outd", [F16, F32])
def test_dot_plan_single_launch(gpu, oracle, outd):
    assert _plan_case(oracle, DOT_PLAN, outd, capi.KERNEL_AUTO, seed=500, expect="dot") == 1


def test_dot_plan_several_rows(gpu, oracle):
    """k_dot_grouped with up to 4 activation rows (automatic dispatch takes
    k_dot for M <= 8 below 1024 tiles, and on more tiles where the launch
    takes the activation tile: M = 3 on 1120 tiles); one problem of M = 4 on
    2048 tiles with 16 k steps per wave takes k_skinny, and with it the
    whole plan runs on k_skinny_grouped."""
    assert _plan_case(oracle, DOT_PLAN_M4, F16, capi.KERNEL_DOT, seed=550, expect="dot") == 1
    assert _plan_case(oracle, DOT_PLAN_M4, F16, capi.KERNEL_AUTO, seed=551, expect="dot") == 1
    specs = DOT_PLAN_M4 + [(3, 17920, 1536, False, None)]
    assert _plan_case(oracle, specs, F16, capi.KERNEL_AUTO, seed=552, expect="dot") == 1
    specs = DOT_PLAN_M4 + [(4, 32768, 2048, False, None)]
    assert _plan_case(oracle, specs, F16, capi.KERNEL_AUTO, seed=553, expect="skinny") == 1


@pytest.mark.parametrize("outd", [F16, F32])
def test_dot_plan_up_to_eight_rows(gpu, oracle, outd):
    """k_dot_grouped with 5-8 activation rows in one launch (the MFMA path
    with 16 x 16 operand tiles, 8 of their rows used), mixed with plans of
    fewer rows, K tails and a long-row problem."""
    assert _plan_case(oracle, DOT_PLAN_M8, outd, capi.KERNEL_AUTO, seed=560, expect="dot") == 1


@pytest.mark.parametrize("outd", [F16, F32])
def test_dot_plan_up_to_sixteen_rows(gpu, oracle, outd):
    """k_dot_grouped forced on problems of up to 16 activation rows (16-row
    MFMA operands), one of them with activations read through the caches
    (K = 20480 does not fit the block's LDS at M = 16); without that one,
    the automatic dispatch takes k_dot for every problem too."""
    assert _plan_case(oracle, DOT_PLAN_M16, outd, capi.KERNEL_DOT, seed=570, expect="dot") == 1
    assert _plan_case(oracle, DOT_PLAN_M16[:5], outd, capi.KERNEL_AUTO, seed=571, expect="dot") == 1


@pytest.mark.parametrize("outd", [F16, F32])
def test_dot_plan_activation_tile(gpu, oracle, outd):
    """A grouped launch on the activation tile: gate and up at M = 16 and a
    ragged 12-row problem (17.4 + 1.6 MB of activations re-read across the
    tiles, 2-3 k steps per wave), and the same with 3-8 rows."""
    specs = [(16, 4864, 896, True, None), (16, 4864, 896, False, "sep"), (12, 300, 1040, False, "inplace")]
    assert sum(dot_x_reread_bytes(M, N, K) for M, N, K, _, _ in specs) >= 5 << 20
    assert _plan_case(oracle, specs, outd, capi.KERNEL_DOT, seed=640, expect="dot") == 1
    specs = [(8, 4864, 896, True, None), (3, 4864, 896, False, "sep"), (5, 4099, 1040, False, "inplace")]
    assert sum(dot_x_reread_bytes(M, N, K) for M, N, K, _, _ in specs) >= 5 << 20
    assert _plan_case(oracle, specs, outd, capi.KERNEL_DOT, seed=641, expect="dot") == 1


def test_dot_plan_without_lds_activations(gpu, oracle):
    """One problem's activations do not fit the block's LDS: the whole plan
    reads activations through the caches."""
    specs = DOT_PLAN[:4] + [(1, 64, 20480, True, "inplace")]
    assert _plan_case(oracle, specs, F16, capi.KERNEL_AUTO, seed=600, expect="dot") == 1


def test_plan_with_short_rows_is_not_streamed(gpu, oracle):
    """K = 256 (4 k steps) cannot fill the streaming pipeline.  Automatic
    dispatch runs such a plan as one k_dot_grouped launch (k_skinny_grouped
    when that family is forced); with the streaming family forced, the short
    problem falls back to the generic kernel and the plan runs one launch per
    problem."""
    specs = [(5, 896, 256, True, None), (1, 4864, 896, False, None)]
    assert _plan_case(oracle, specs, F16, capi.KERNEL_AUTO, seed=400, expect="dot") == 1
    assert _plan_case(oracle, specs, F16, capi.KERNEL_SKINNY, seed=400, expect="skinny") == 1
    assert _plan_case(oracle, specs, F16, capi.KERNEL_STREAM, seed=400, expect="auto") == 2


def test_plan_with_prefill_problem_runs_per_call(gpu, oracle):
    q, s, b = weights(256, 512, 5, oracle)
    rng = np.random.default_rng(5)
    xs = [rng.normal(0, 1, (M, 512)).astype(np.float16) for M in (1, 40)]
    d_q, d_s = capi.DevBuf.from_array(q), capi.DevBuf.from_array(s)
    d_x = [capi.DevBuf.from_array(x) for x in xs]
    d_y = [capi.DevBuf(x.shape[0] * 256 * 2) for x in xs]
    probs = [capi.Q8Problem(out=d_y[i].ptr, inp=d_x[i].ptr, residual=None, weight=d_q.ptr, scales=d_s.ptr,
                            bias=None, M=xs[i].shape[0], N=256, K=512) for i in range(2)]
    arr = (capi.Q8Problem * 2)(*probs)
    plan = ctypes.c_uint64()
    capi.call("vvh_plan_create", arr, 2, F16, F16, ctypes.byref(plan))
    n = ctypes.c_int()
    capi.call("vvh_plan_launches", plan.value, ctypes.byref(n))
    assert n.value == 2
    capi.call("vvh_plan_run", plan.value, None)
    capi.sync()
    for i, x in enumerate(xs):
        y = d_y[i].to_array(np.float16, (x.shape[0], 256)).astype(np.float32)
        ref = oracle.linear_q8(x.astype(np.float32), q, s)
        assert np.abs(y - ref).max() / np.abs(ref).max() <= TOL_F16
    capi.call("vvh_plan_destroy", plan.value)


def test_pool_on_device(gpu):
    before = capi.PoolStats()
    capi.call("vvh_pool_get_stats", ctypes.byref(before))
    p = ctypes.c_void_p()
    capi.call("vvh_pool_alloc", ctypes.byref(p), 1 << 20)
    first = p.value
    capi.call("vvh_pool_free", first)
    capi.call("vvh_pool_alloc", ctypes.byref(p), (1 << 20) - 100)
    assert p.value == first
    after = capi.PoolStats()
    capi.call("vvh_pool_get_stats", ctypes.byref(after))
    assert after.cache_hits == before.cache_hits + 1
    capi.call("vvh_pool_free", p.value)
    capi.call("vvh_pool_release_cached")
    z = ctypes.c_void_p(1)
    capi.call("vvh_pool_alloc", ctypes.byref(z), 0)
    assert z.value is None


def test_convert_and_fill(gpu):
    x = np.random.default_rng(0).normal(0, 10, 10007).astype(np.float32)
    d_x, d_h, d_f = capi.DevBuf.from_array(x), capi.DevBuf(10007 * 2), capi.DevBuf(10007 * 4)
    capi.call("vvh_convert", d_h.ptr, F16, d_x.ptr, F32, 10007, None)
    capi.call("vvh_convert", d_f.ptr, F32, d_h.ptr, F16, 10007, None)
    capi.sync()
    np.testing.assert_array_equal(d_h.to_array(np.float16, 10007), x.astype(np.float16))
    np.testing.assert_array_equal(d_f.to_array(np.float32, 10007), x.astype(np.float16).astype(np.float32))
    n = 1 << 20
    d = capi.DevBuf(n * 4)
    capi.call("vvh_fill_normal", d.ptr, F32, n, 1234, 0.5, 0.02, None)
    capi.sync()
    a = d.to_array(np.float32, n)
    assert abs(a.mean() - 0.5) < 1e-3 and abs(a.std() - 0.02) < 1e-3
    capi.call("vvh_fill_normal", d.ptr, F32, n, 1234, 0.5, 0.02, None)
    capi.sync()
    np.testing.assert_array_equal(d.to_array(np.float32, n), a)


# ---------------------------------------------------------------------------
# weights beyond 2^31 codes (64-bit row offsets)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("M,kernel", [(1, capi.KERNEL_DOT), (8, capi.KERNEL_SKINNY), (32, capi.KERNEL_GEMM)],
                         ids=["dot", "skinny", "gemm"])
def test_weight_beyond_2g_codes(gpu, oracle, M, kernel):
    """N = 2,400,000 rows of K = 896 codes (2.15 GB): weights filled and
    quantized on the device; rows at both ends (offsets past 2^31) are checked
    against the oracle on the same codes, copied back."""
    N, K = 2_400_000, 896
    print(f"[case] beyond 2^31 codes M={M} kernel={capi.KERNEL_NAMES[kernel]}", flush=True)
    d_wf = capi.DevBuf(64 * 1024 * K * 4)         # fp32 staging, 64K rows at a time
    d_q, d_s = capi.DevBuf(N * K), capi.DevBuf(N * 4)
    for r0 in range(0, N, 64 * 1024):
        rows = min(64 * 1024, N - r0)
        capi.call("vvh_fill_normal", d_wf.ptr, F32, rows * K, 4242 + r0, 0.0, 0.02, None)
        capi.call("vvh_quantize_per_channel", d_wf.ptr, rows, K, d_q.ptr + r0 * K, d_s.ptr + r0 * 4, None)
    del d_wf
    x = np.random.default_rng(5).normal(0, 1, (M, K)).astype(np.float16)
    d_x, d_y = capi.DevBuf.from_array(x), capi.DevBuf(M * N * 2)
    capi.set_kernel(kernel)
    try:
        capi.linear_q8_dev(d_y, d_x, d_q, d_s, None, None, M, N, K, F16, F16)
        capi.sync()
    finally:
        capi.set_kernel(capi.KERNEL_AUTO)
    check = list(range(0, 40)) + list(range(N - 2_000, N))
    assert (N - 2_000) * K > 2 ** 31
    q = np.empty((len(check), K), np.int8)
    s = np.empty(len(check), np.float32)
    for i, n in enumerate(check):
        capi.call("vvh_memcpy_d2h", q[i].ctypes.data, d_q.ptr + n * K, K)
        capi.call("vvh_memcpy_d2h", s[i:i + 1].ctypes.data, d_s.ptr + n * 4, 4)
    y = d_y.to_array(np.float16, (M, N)).astype(np.float32)[:, check]
    ref = oracle.linear_q8(x.astype(np.float32), q, s)
    err = float(np.abs(y - ref).max() / np.abs(ref).max())
    assert err <= TOL_F16, err


# ---------------------------------------------------------------------------
# weight ingestion: host BF16 / F32 rows quantized straight into the mirror
# ---------------------------------------------------------------------------
def _bf16_rows(N, K, seed, std=0.02):
    w = np.random.default_rng(seed).normal(0, std, (N, K)).astype(np.float32)
    return (w.view(np.uint32) >> 16).astype(np.uint16)  # truncated to BF16 bit patterns


@pytest.mark.parametrize("N,K", [(1, 1), (3, 1000), (896, 896), (4864, 896), (20000, 1000), (2, 9_000_000)],
                         ids=["1x1", "3x1000", "896x896", "4864x896", "20000x1000_two_chunks", "2x9M_row_chunks"])
def test_weight_ingest_bf16_bit_exact(gpu, oracle, N, K):
    print(f"[case] ingest bf16 N={N} K={K}", flush=True)
    bits = _bf16_rows(N, K, N + K)
    if N >= 3:  # special rows: zero, NaN/Inf, exact ties
        bits[0] = 0
        bits[1, : min(K, 4)] = [0x7FC0, 0x7F80, 0xFF80, 0x3F80][: min(K, 4)]
        bits[2, : min(K, 3)] = np.array([1.0, 0.5, -0.5], np.float32)[: min(K, 3)].view(np.uint32) >> 16
    scales = np.empty(N, np.float32)
    h = ctypes.c_uint64()
    capi.call("vvh_weight_ingest", bits.ctypes.data, capi.BF16, None, N, K, scales.ctypes.data, ctypes.byref(h))
    q_ref, s_ref = oracle.ingest_bf16(bits)
    dq, ds, db = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    n_, k_ = ctypes.c_size_t(), ctypes.c_size_t()
    capi.call("vvh_weight_device_ptrs", h.value, ctypes.byref(dq), ctypes.byref(ds), ctypes.byref(db),
              ctypes.byref(n_), ctypes.byref(k_))
    assert (n_.value, k_.value, db.value) == (N, K, None)
    q = np.empty((N, K), np.int8)
    s = np.empty(N, np.float32)
    capi.call("vvh_memcpy_d2h", q.ctypes.data, dq.value, N * K)
    capi.call("vvh_memcpy_d2h", s.ctypes.data, ds.value, N * 4)
    np.testing.assert_array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(scales.view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(q, q_ref)
    capi.call("vvh_weight_release", h.value)


def test_weight_ingest_f32_and_linear(gpu, oracle):
    """F32 rows ingest to the same codes as the host quantizer; the mirror
    serves vvh_linear_q8; re-ingesting the same tuple returns the same handle,
    and vvh_weight_register with the rows' address as the weight (what
    Backend::linear_q8 passes) finds the ingested mirror."""
    N, K = 896, 4864
    w = np.random.default_rng(3).normal(0, 0.02, (N, K)).astype(np.float32)
    b = np.random.default_rng(4).normal(0, 0.01, N).astype(np.float32)
    scales = np.empty(N, np.float32)
    h = ctypes.c_uint64()
    capi.call("vvh_weight_ingest", w.ctypes.data, capi.F32, b.ctypes.data, N, K, scales.ctypes.data, ctypes.byref(h))
    q_ref, s_ref = oracle.quantize_per_channel(w)
    np.testing.assert_array_equal(scales, s_ref)
    h2, h3 = ctypes.c_uint64(), ctypes.c_uint64()
    capi.call("vvh_weight_ingest", w.ctypes.data, capi.F32, b.ctypes.data, N, K, scales.ctypes.data, ctypes.byref(h2))
    capi.call("vvh_weight_register", w.ctypes.data, scales.ctypes.data, b.ctypes.data, N, K, ctypes.byref(h3))
    assert h.value == h2.value == h3.value
    for M in (1, 64):
        x = np.random.default_rng(M).normal(0, 1, (M, K)).astype(np.float16)
        d_x, d_y = capi.DevBuf.from_array(x), capi.DevBuf(M * N * 4)
        capi.call("vvh_linear_q8", d_y.ptr, d_x.ptr, h.value, None, M, N, K, F16, F32, None)
        capi.sync()
        ref = oracle.linear_q8(x.astype(np.float32), q_ref, s_ref, b)
        y = d_y.to_array(np.float32, (M, N))
        assert np.abs(y - ref).max() / np.abs(ref).max() <= TOL_F16
    capi.call("vvh_weight_release", h.value)


def test_headline_plan_every_projection(gpu, oracle):
    """The workload bench.py times for its headline line: 24
    layers x {q, k, v, o, gate, up, down} of device-made seeded weights, M=1,
    fp16 in and out, o and down adding their residual in place, as one
    grouped plan.  One run of the plan; every one of the 168 outputs is
    checked against the oracle on the same codes, scales, biases,
    activations and residuals (copied back from the device)."""
    import bench

    projs = bench.layer_projs(896, 128, 4864)
    tmp = capi.DevBuf(4864 * 896 * 4)
    (arena, lins), = bench.build_decode_set(1, 24, projs, tmp)
    plan = bench.make_plan(lins)
    assert capi.plan_kernel(plan) == "dot"
    before = []
    for l in lins:
        y0 = np.empty((1, l.N), np.float16)
        capi.call("vvh_memcpy_d2h", y0.ctypes.data, l.y, y0.nbytes)
        before.append(y0)
    print("[case] headline plan: 168 projections, one grouped launch", flush=True)
    capi.call("vvh_plan_run", plan, None)
    capi.sync()
    worst = 0.0
    for i, l in enumerate(lins):
        q = np.empty((l.N, l.K), np.int8)
        s = np.empty(l.N, np.float32)
        x = np.empty((1, l.K), np.float16)
        y = np.empty((1, l.N), np.float16)
        for arr, ptr in ((q, l.w), (s, l.s), (x, l.x), (y, l.y)):
            capi.call("vvh_memcpy_d2h", arr.ctypes.data, ptr, arr.nbytes)
        b = None
        if l.b:
            b = np.empty(l.N, np.float32)
            capi.call("vvh_memcpy_d2h", b.ctypes.data, l.b, b.nbytes)
        r = before[i].astype(np.float32) if l.has_res else None
        ref = oracle.linear_q8(x.astype(np.float32), q, s, b, r)
        err = float(np.abs(y.astype(np.float32) - ref).max() / np.abs(ref).max())
        worst = max(worst, err)
        assert err <= TOL_F16, f"projection {i} ({projs[i % 7][0]}, layer {i // 7}): {err:.3e}"
    print(f"[case] headline plan worst normalized error {worst:.2e}", flush=True)
    capi.call("vvh_plan_destroy", plan)


# ---------------------------------------------------------------------------
# fp32 activations on the MFMA GEMM (split into scaled fp16 high/low parts)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("outd", [F32, F16])
@pytest.mark.parametrize("M,N,K,res", [(16, 4864, 896, None), (32, 896, 896, "sep"), (128, 4864, 896, None),
                                       (512, 4864, 896, None), (512, 896, 4864, "inplace"),
                                       (130, 250, 4864, "sep"), (300, 776, 256, "inplace")])
def test_fp32_gemm(gpu, oracle, M, N, K, res, outd):
    """The reference's default (fp32) mode on the prefill GEMM: fp32 in,
    fp32 or fp16 out, against the oracle at the fp32 bar (1e-4 and, for fp32
    outputs, the fp32 accumulation bound).  Includes split-K (K = 4864 with
    few tiles), edge tiles (N = 250, 776; M = 130, 300) and M = 16, the
    smallest M the automatic choice sends to the GEMM."""
    kern = capi.KERNEL_AUTO
    if K % 64 == 0:
        assert capi.kernel_choice(M, N, K, F32, outd) == "gemm"
    run_case(oracle, M, N, K, F32, outd, bias=bool(N % 2 == 0), res=res, kernel=kern, seed=3 * M + N + K)


def test_fp32_gemm_scaled_rows(gpu, oracle):
    """Rows whose range needs the per-row power-of-two scaling: values far
    beyond fp16's range (1e5 .. 3e6), a row of tiny values (1e-30), an
    all-zero row, and a row mixing huge and tiny values; every output within
    the fp32 accumulation bound of the oracle."""
    M, N, K = 64, 384, 896
    rng = np.random.default_rng(8)
    q, s, b = weights(N, K, 8, oracle)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    x[1] *= np.float32(1e5)
    x[2] *= np.float32(3e6)
    x[3] *= np.float32(1e-30)
    x[4] = 0.0
    x[5, ::2] *= np.float32(1e4)
    x[5, 1::2] *= np.float32(1e-4)
    d = [capi.DevBuf.from_array(a) for a in (q, s, b, x)]
    y = capi.DevBuf(M * N * 4)
    print("[case] fp32 gemm scaled rows", flush=True)
    assert capi.kernel_choice(M, N, K, F32, F32) == "gemm"
    capi.linear_q8_dev(y, d[3], d[0], d[1], d[2], None, M, N, K, F32, F32)
    capi.sync()
    got = y.to_array(np.float32, (M, N))
    ref = oracle.linear_q8(x, q, s, b)
    assert np.isfinite(got).all()
    np.testing.assert_array_equal(got[4], b)  # zero row: the bias exactly
    check_f32_bound(got, ref, x, q, s, b, None, K)
