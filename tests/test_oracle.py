"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against (a) the reference's own test
assertions (src/quantize/quantize_test.cc, src/backend/backend_naive_test.cc),
(b) the golden vectors written from the reference compiled in place
(tests/golden/gen_golden.py), (c) the reference library itself when it is
built here (oracle/_ref), and (d) closed forms the mathematics fixes, chosen so
that a dropped term, a wrong index, a transposed operand or a wrong rounding
rule fails one of them.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# --------------------------------------------------------------------------
# quantize_per_channel
# --------------------------------------------------------------------------
def test_quantize_matches_golden(oracle):
    d = np.load(os.path.join(GOLDEN, "quantize_ref.npz"))
    names = sorted({k[2:-2] for k in d.files if k.endswith("_w")})
    assert len(names) == 8
    for n in names:
        q, s = oracle.quantize_per_channel(d[f"q_{n}_w"])
        np.testing.assert_array_equal(q, d[f"q_{n}_codes"], err_msg=n)
        np.testing.assert_array_equal(bits(s), bits(d[f"q_{n}_scales"]), err_msg=n)


def test_quantize_reference_assertions(oracle):
    # RoundtripAccuracy, quantize_test.cc:13-42
    w = np.array([[0.5, -0.3, 0.1, 0.9], [1.0, 0.0, -1.0, 0.5], [0.0, 0.2, 0.4, -0.8]], np.float32)
    q, s = oracle.quantize_per_channel(w)
    assert q.shape == (3, 4) and s.shape == (3,)
    deq = q.astype(np.float32) * s[:, None]
    assert np.all(np.abs(deq - w) <= s[:, None] + 1e-6)
    # ZeroRow, :44-55
    q, s = oracle.quantize_per_channel(np.zeros((1, 4), np.float32))
    assert s[0] == 0.0 and not q.any()
    # Saturation, :57-79
    q, s = oracle.quantize_per_channel(np.array([[127.0, -128.0, 0.0, 50.0]], np.float32))
    assert s[0] == np.float32(128.0) / np.float32(127.0)
    assert q[0, 1] == -127
    assert np.all(q >= -128) and np.all(q <= 127)
    # LargeMatrix, :81-100
    w = ((np.arange(64 * 128) % 255).astype(np.float32) / np.float32(127) - np.float32(1)).reshape(64, 128)
    q, s = oracle.quantize_per_channel(w)
    assert q.shape == (64, 128) and np.all(s > 0)


def test_quantize_closed_forms(oracle):
    # scale exactly 1.0 (absmax 127): codes are roundf(w), ties away from zero.
    # rint would give 62, -0, 2, -2, 0, -2, 126 on these.
    q, s = oracle.quantize_per_channel(np.array([[127, 62.5, -0.5, 2.5, -2.5, 0.5, -1.5, 126.5]], np.float32))
    assert s[0] == 1.0
    assert q[0].tolist() == [127, 63, -1, 3, -3, 1, -2, 127]
    # a row that is an exact multiple of its scale quantizes losslessly
    codes = np.array([[-127, -64, -1, 0, 1, 17, 100, 127]], np.float32)
    q, s = oracle.quantize_per_channel(codes * np.float32(0.5))
    assert s[0] == np.float32(63.5) / np.float32(127)
    assert q[0].tolist() == codes[0].astype(int).tolist()
    # rows are independent and sign-symmetric
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (9, 70)).astype(np.float32)
    q, s = oracle.quantize_per_channel(w)
    qn, sn = oracle.quantize_per_channel(-w)
    np.testing.assert_array_equal(qn, -q)
    np.testing.assert_array_equal(bits(sn), bits(s))
    q3, s3 = oracle.quantize_per_channel(w[3:4])
    np.testing.assert_array_equal(q3[0], q[3])
    # every code is within half a step of w/scale (no clamping at absmax/scale = 127)
    r = w / s[:, None]
    assert np.all(np.abs(q - r) <= 0.5 + 1e-4)
    assert np.all(np.abs(q).max(axis=1) == 127)


def test_quantize_nan_inf(oracle):
    # NaN is skipped by the absmax and codes to +127 (std::min(127, NaN) == 127)
    q, s = oracle.quantize_per_channel(np.array([[np.nan, 1.0, -2.0, 0.25]], np.float32))
    assert s[0] == np.float32(2.0) / np.float32(127.0)
    assert q[0].tolist() == [127, 64, -127, 16]
    q, s = oracle.quantize_per_channel(np.full((1, 5), np.nan, np.float32))
    assert s[0] == 0.0 and not q.any()
    # Inf: scale Inf, reciprocal 0; Inf*0 = NaN -> 127, finite -> 0
    q, s = oracle.quantize_per_channel(np.array([[np.inf, 1.0, -0.5, 3.0]], np.float32))
    assert np.isinf(s[0]) and q[0].tolist() == [127, 0, 0, 0]


# --------------------------------------------------------------------------
# linear_q8 / linear_q8_add
# --------------------------------------------------------------------------
def test_linear_reference_tests(oracle):
    # LinearQ8WithBias, backend_naive_test.cc:407-425
    y = oracle.linear_q8(np.array([[3.0, 5.0]], np.float32), np.array([[127, 0], [0, 127]], np.int8),
                         np.array([1 / 127, 1 / 127], np.float32), np.array([10.0, 20.0], np.float32))
    assert abs(y[0, 0] - 13.0) <= 1e-4 and abs(y[0, 1] - 25.0) <= 1e-4
    # LinearQ8MatchesFp32, :355-405 (codes from the test's own division-based quantization)
    w = np.array([[0.5, -0.3, 0.1, 0.9], [1.0, 0.0, -1.0, 0.5], [0.0, 0.2, 0.4, -0.8]], np.float32)
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    s = (np.abs(w).max(axis=1) / np.float32(127)).astype(np.float32)
    q = np.clip(np.round(w / s[:, None]), -128, 127).astype(np.int8)  # numpy ties-to-even is fine here
    y = oracle.linear_q8(x, q, s)
    ref = (x @ w.T)[0]
    assert np.all(np.abs(y[0] - ref) <= s * 4 * 0.5 + 1e-5)


def test_linear_matches_golden(oracle):
    d = np.load(os.path.join(GOLDEN, "linear_ref.npz"))
    cases = sorted({k[2:k.rindex("_")] for k in d.files if k.endswith("_out")})
    assert len(cases) >= 10
    for c in cases:
        p = f"l_{c}_"
        g = lambda k: d[p + k] if p + k in d.files else None
        meta = g("meta")
        inplace = bool(meta[3]) if meta is not None else False
        y = oracle.linear_q8(g("x"), g("q"), g("scales"), g("bias"), g("residual"), inplace=inplace)
        np.testing.assert_array_equal(bits(y), bits(g("out")), err_msg=c)


def test_linear_integer_closed_form(oracle):
    """Small-integer inputs, scale 1: every partial sum is an exact integer, so
    the output must equal the int64 matrix product exactly (catches a wrong
    index, a transposed operand, a dropped tail element or row)."""
    rng = np.random.default_rng(1)
    for (M, N, K) in [(1, 5, 4), (3, 7, 100), (2, 33, 64), (4, 9, 131), (1, 1, 1)]:
        x = rng.integers(-8, 9, (M, K)).astype(np.float32)
        q = rng.integers(-128, 128, (N, K)).astype(np.int8)
        y = oracle.linear_q8(x, q, np.ones(N, np.float32))
        exact = x.astype(np.int64) @ q.astype(np.int64).T
        np.testing.assert_array_equal(y, exact.astype(np.float32))
        b = rng.integers(-50, 50, N).astype(np.float32)
        r = rng.integers(-50, 50, (M, N)).astype(np.float32)
        y = oracle.linear_q8(x, q, np.ones(N, np.float32), b, r)
        np.testing.assert_array_equal(y, (exact + b + r).astype(np.float32))


def test_linear_fp64_bound_and_invariants(oracle):
    rng = np.random.default_rng(2)
    for (M, N, K) in [(1, 64, 896), (3, 40, 333), (2, 16, 4864)]:
        w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
        q, s = oracle.quantize_per_channel(w)
        x = rng.normal(0, 1, (M, K)).astype(np.float32)
        b = rng.normal(0, 0.01, N).astype(np.float32)
        y = oracle.linear_q8(x, q, s, b)
        exact = oracle.linear_q8_f64(x, q, s, b)
        # fp32 summation bound: K * eps * sum|x q| * scale, plus the epilogue roundings
        mag = (np.abs(x).astype(np.float64) @ np.abs(q.astype(np.float64)).T) * s
        bound = K * 2.0 ** -24 * mag + 2.0 ** -23 * (np.abs(exact) + np.abs(b))
        assert np.all(np.abs(y - exact) <= bound)
        # scale is applied after the dot product: doubling it doubles the output exactly
        y1 = oracle.linear_q8(x, q, s)
        y2 = oracle.linear_q8(x, q, s * np.float32(2))
        np.testing.assert_array_equal(y2, y1 * np.float32(2))
        # zero codes give the bias exactly
        np.testing.assert_array_equal(oracle.linear_q8(x, np.zeros_like(q), s, b), np.broadcast_to(b, (M, N)))


def test_linear_add_semantics(oracle):
    rng = np.random.default_rng(3)
    M, N, K = 3, 48, 160
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-3, 2e-3, N).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    b = rng.normal(0, 0.01, N).astype(np.float32)
    r = rng.normal(0, 1, (M, N)).astype(np.float32)
    # linear_q8_add == linear_q8 then an fp32 add (backend_naive.cc:322-335)
    y = oracle.linear_q8(x, q, s, b, r)
    np.testing.assert_array_equal(bits(y), bits(oracle.linear_q8(x, q, s, b) + r))
    # in place (out == residual) gives the same bits
    np.testing.assert_array_equal(bits(oracle.linear_q8(x, q, s, b, r, inplace=True)), bits(y))


def test_oracle_equals_reference_library(oracle):
    """Bit-exact against the reference's own code when oracle/_ref is built."""
    if not oracle.available("reference"):
        pytest.skip("oracle/_ref not built (reference tree absent); golden vectors cover this")
    rng = np.random.default_rng(4)
    for (M, N, K) in [(1, 896, 896), (2, 100, 4864), (5, 33, 77), (1, 7, 31), (3, 64, 96)]:
        w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
        q1, s1 = oracle.quantize_per_channel(w)
        q2, s2 = oracle.quantize_per_channel(w, kind="reference")
        np.testing.assert_array_equal(q1, q2)
        np.testing.assert_array_equal(bits(s1), bits(s2))
        x = rng.normal(0, 1, (M, K)).astype(np.float32)
        b = rng.normal(0, 0.01, N).astype(np.float32)
        r = rng.normal(0, 1, (M, N)).astype(np.float32)
        for args in [(None, None, False), (b, None, False), (b, r, False), (None, r, True)]:
            y1 = oracle.linear_q8(x, q1, s1, *args[:2], inplace=args[2])
            y2 = oracle.linear_q8(x, q1, s1, *args[:2], kind="reference", inplace=args[2])
            np.testing.assert_array_equal(bits(y1), bits(y2))


def test_planted_mistakes_are_caught(oracle):
    """The checks above would catch plausible oracle mistakes: emulate them on
    the CPU and confirm the golden vectors reject each."""
    d = np.load(os.path.join(GOLDEN, "linear_ref.npz"))
    p = "l_body_and_tail_k100_"
    x, q, s, b, y = d[p + "x"], d[p + "q"], d[p + "scales"], d[p + "bias"], d[p + "out"]
    good = oracle.linear_q8(x, q, s, b)
    assert np.array_equal(bits(good), bits(y))
    dropped_tail = oracle.linear_q8(x[:, :96], q[:, :96], s, b)          # tail not summed
    no_bias = oracle.linear_q8(x, q, s)                                   # bias dropped
    transposed_scale = oracle.linear_q8(x, q, s[::-1].copy(), b)         # wrong scale index
    for bad in (dropped_tail, no_bias, transposed_scale):
        assert not np.array_equal(bits(bad), bits(y))
    dq = np.load(os.path.join(GOLDEN, "quantize_ref.npz"))
    w = dq["q_ties_w"]
    rint_codes = np.clip(np.rint(w / dq["q_ties_scales"][:, None]), -128, 127).astype(np.int8)
    assert not np.array_equal(rint_codes, dq["q_ties_codes"])


def test_bf16_widening_closed_form(oracle):
    """orc_bf16_to_f32 (safetensors.cc:135-141) against the BF16 decoding
    (-1)^s * 2^(e-127) * (1 + m/128), subnormals 2^-126 * m/128, +-0, +-Inf and
    NaN, for every one of the 65536 bit patterns."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.bf16_to_f32(bits)
    s = (bits >> 15).astype(np.int64)
    e = ((bits >> 7) & 0xFF).astype(np.int64)
    m = (bits & 0x7F).astype(np.float64)
    sign = np.where(s == 1, -1.0, 1.0)
    with np.errstate(over="ignore"):
        normal = sign * np.ldexp(1.0 + m / 128.0, e - 127)
    sub = sign * np.ldexp(m / 128.0, -126)
    want = np.where(e == 0, sub, normal)
    want = np.where((e == 255) & (m == 0), sign * np.inf, want)
    nan = (e == 255) & (m != 0)
    assert np.isnan(got[nan]).all()
    ok = ~nan
    np.testing.assert_array_equal(got[ok], want[ok].astype(np.float32))
    np.testing.assert_array_equal(np.signbit(got[ok]), s[ok] == 1)  # -0 stays -0


def test_ingest_bf16_known_answers(oracle):
    """Host path of a BF16 weight (widen, then quantize): hand-computed rows.
    [1, -1, 0.5, 0]: scale = 1/127, 0.5 * 127 = 63.5 ties away from zero -> 64.
    [0, -0]: zero row -> scale 0, codes 0.  [2, 0.5, -0.25]: scale 2/127,
    codes 127, 31.75 -> 32, -15.875 -> -16."""
    def bf(x):  # exact BF16 patterns of values that have one
        return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)
    q, s = oracle.ingest_bf16(bf([[1.0, -1.0, 0.5, 0.0]]))
    assert s[0] == np.float32(1.0) / np.float32(127.0)
    assert q.tolist() == [[127, -127, 64, 0]]
    q, s = oracle.ingest_bf16(bf([[0.0, -0.0, 0.0]]))
    assert s[0] == 0.0 and q.tolist() == [[0, 0, 0]]
    q, s = oracle.ingest_bf16(bf([[2.0, 0.5, -0.25]]))
    assert s[0] == np.float32(2.0) / np.float32(127.0)
    assert q.tolist() == [[127, 32, -16]]


# ---------------------------------------------------------------------------
# the other BackendCPU operators (src/backend/backend_naive.cc)
# ---------------------------------------------------------------------------
def _need_ref(oracle):
    if not oracle.available("reference"):
        pytest.skip("oracle/_ref (the reference compiled in place) is not built here")


def test_ops_bit_exact_vs_reference(oracle):
    """Every restated operator agrees bit for bit with the reference's own
    BackendCPU compiled from its sources (same compiler, flags and libm)."""
    _need_ref(oracle)
    rng = np.random.default_rng(11)
    x = rng.normal(0, 2, 1000).astype(np.float32)
    y = rng.normal(0, 2, 1000).astype(np.float32)
    for op in ("add", "mul", "silu", "silu_mul"):
        a = oracle.eltwise(op, x, y)
        b = oracle.eltwise(op, x, y, kind="reference")
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=op)
    rows = rng.normal(0, 1, (3, 896)).astype(np.float32)
    w = rng.normal(1, 0.1, 896).astype(np.float32)
    np.testing.assert_array_equal(oracle.rms_norm(rows, w, 1e-6), oracle.rms_norm(rows, w, 1e-6, kind="reference"))
    np.testing.assert_array_equal(oracle.softmax(rows), oracle.softmax(rows, kind="reference"))
    q = rng.normal(0, 1, (3, 14, 64)).astype(np.float32)
    k = rng.normal(0, 1, (3, 2, 64)).astype(np.float32)
    for pos in (0, 7, 4000):
        a, b = oracle.rope(q, k, pos, 1e6), oracle.rope(q, k, pos, 1e6, kind="reference")
        np.testing.assert_array_equal(a[0], b[0])
        np.testing.assert_array_equal(a[1], b[1])
    X = rng.normal(0, 1, (3, 96)).astype(np.float32)
    W = rng.normal(0, 0.1, (40, 96)).astype(np.float32)
    bias = rng.normal(0, 0.1, 40).astype(np.float32)
    res = rng.normal(0, 1, (3, 40)).astype(np.float32)
    np.testing.assert_array_equal(oracle.linear(X, W, bias), oracle.linear(X, W, bias, kind="reference"))
    np.testing.assert_array_equal(oracle.linear(X, W, None, res), oracle.linear(X, W, None, res, kind="reference"))
    np.testing.assert_array_equal(oracle.matmul(X, W.T.copy()), oracle.matmul(X, W.T.copy(), kind="reference"))
    kc = rng.normal(0, 1, (50, 2, 64)).astype(np.float32)
    vc = rng.normal(0, 1, (50, 2, 64)).astype(np.float32)
    for q_idx, ln in ((0, 1), (1, 17), (2, 50)):
        np.testing.assert_array_equal(oracle.causal_attention(q, kc, vc, q_idx, ln, 0.125),
                                      oracle.causal_attention(q, kc, vc, q_idx, ln, 0.125, kind="reference"))


def test_ops_closed_forms(oracle):
    """What the mathematics fixes, independent of the restatement."""
    # RMSNorm of c*1 with unit weight and eps 0 is sign(c) exactly (c a power of 2)
    for c in (4.0, -0.25):
        np.testing.assert_array_equal(oracle.rms_norm(np.full((1, 64), c), np.ones(64), 0.0), np.sign(c))
    # softmax of a constant row of 2^k elements is 2^-k exactly
    np.testing.assert_array_equal(oracle.softmax(np.full((1, 256), 3.0)), np.float32(1 / 256))
    # RoPE at position 0 is the identity; at head_dim 2 the pair rotates by `pos` radians
    rng = np.random.default_rng(2)
    q = rng.normal(0, 1, (1, 3, 8)).astype(np.float32)
    k = rng.normal(0, 1, (1, 1, 8)).astype(np.float32)
    q0, k0 = oracle.rope(q, k, 0, 10000.0)
    np.testing.assert_array_equal(q0, q)
    np.testing.assert_array_equal(k0, k)
    q2 = np.array([[[1.0, 0.0]]], np.float32)
    r, _ = oracle.rope(q2, np.zeros((1, 1, 2), np.float32), 5, 10000.0)
    np.testing.assert_allclose(r[0, 0], [np.cos(5.0), np.sin(5.0)], atol=1e-6)
    # RoPE preserves the norm of every (i, i + D/2) pair
    qq, _ = oracle.rope(q, k, 123, 10000.0)
    n0 = q[..., :4] ** 2 + q[..., 4:] ** 2
    n1 = qq[..., :4] ** 2 + qq[..., 4:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)
    # attention over one position returns that position's value row (GQA: heads 0-6 -> kv 0)
    qa = rng.normal(0, 1, (1, 14, 64)).astype(np.float32)
    kv = rng.normal(0, 1, (1, 2, 64)).astype(np.float32)
    va = rng.normal(0, 1, (1, 2, 64)).astype(np.float32)
    out = oracle.causal_attention(qa, kv, va, 0, 1, 0.125).reshape(14, 64)
    np.testing.assert_array_equal(out[:7], np.broadcast_to(va[0, 0], (7, 64)))
    np.testing.assert_array_equal(out[7:], np.broadcast_to(va[0, 1], (7, 64)))
    # equal keys give uniform weights: the output is the mean of the values
    ke = np.broadcast_to(kv[:1], (8, 2, 64)).copy()
    ve = rng.normal(0, 1, (8, 2, 64)).astype(np.float32)
    out = oracle.causal_attention(qa, ke, ve, 0, 8, 0.125).reshape(14, 64)
    np.testing.assert_allclose(out[0], ve[:, 0].mean(axis=0), atol=1e-6)
    # integer-valued linear / matmul are exact (an index or transpose mistake fails)
    X = rng.integers(-8, 8, (3, 20)).astype(np.float32)
    W = rng.integers(-8, 8, (5, 20)).astype(np.float32)
    b = rng.integers(-8, 8, 5).astype(np.float32)
    want = X.astype(np.int64) @ W.astype(np.int64).T + b.astype(np.int64)
    np.testing.assert_array_equal(oracle.linear(X, W, b), want)
    np.testing.assert_array_equal(oracle.matmul(X, W.T.copy()), X.astype(np.int64) @ W.astype(np.int64).T)
    # silu(0) = 0, silu_mul(0, y) = 0, silu of a large x is x
    np.testing.assert_array_equal(oracle.eltwise("silu", np.zeros(4)), 0.0)
    np.testing.assert_array_equal(oracle.eltwise("silu_mul", np.zeros(4), np.ones(4)), 0.0)
    np.testing.assert_array_equal(oracle.eltwise("silu", np.array([40.0])), 40.0)
