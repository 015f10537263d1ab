"""Writes the golden vectors of the linear_q8 path from the reference itself.

Run in a container where the reference tree is present:
    make -C oracle ref && python tests/golden/gen_golden.py

It loads oracle/_ref/libvvllm_ref.so -- the reference's own
src/quantize/quantize.cc and src/backend/backend_naive.cc compiled in place
(oracle/Makefile) -- and records inputs and outputs of:
  * quantize_per_channel on the matrices of the reference's quantize tests
    (src/quantize/quantize_test.cc:13-100) plus tie / NaN / Inf rows;
  * BackendCPU::linear_q8 on the inputs of the reference's linear_q8 tests
    (src/backend/backend_naive_test.cc:355-425);
  * BackendCPU::linear_q8 / linear_q8_add on seeded shapes chosen to run the
    AVX2 body, the scalar tail, M > 1, bias / no bias, a residual, and the
    in-place (out == residual) form.
The files hold data only (numpy .npz, loadable with allow_pickle=False).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402

QUANT_CASES = {
    # quantize_test.cc:15-21 (RoundtripAccuracy)
    "roundtrip": np.array([[0.5, -0.3, 0.1, 0.9], [1.0, 0.0, -1.0, 0.5], [0.0, 0.2, 0.4, -0.8]], np.float32),
    # quantize_test.cc:47 (ZeroRow)
    "zero_row": np.zeros((1, 4), np.float32),
    # quantize_test.cc:60 (Saturation)
    "saturation": np.array([[127.0, -128.0, 0.0, 50.0]], np.float32),
    # quantize_test.cc:84-88 (LargeMatrix)
    "large": ((np.arange(64 * 128) % 255).astype(np.float32) / np.float32(127.0) - np.float32(1.0)).reshape(64, 128),
    # ties at scale 1.0 (roundf vs rint), NaN, all-NaN and Inf rows
    "ties": np.array([[127.0, 62.5, -0.5, 2.5, -2.5, 0.5, -1.5, 126.5]], np.float32),
    "nan": np.array([[np.nan, 1.0, -2.0, 0.25]], np.float32),
    "all_nan": np.array([[np.nan, np.nan, np.nan, np.nan]], np.float32),
    "inf": np.array([[np.inf, 1.0, -0.5, 3.0]], np.float32),
}

# (name, M, N, K, bias, residual, inplace, seed)
LINEAR_CASES = [
    ("tail_only_k4", 1, 3, 4, False, False, False, 1),
    ("avx_body_k32", 1, 8, 32, True, False, False, 2),
    ("body_and_tail_k100", 3, 17, 100, True, False, False, 3),
    ("m4_k256", 4, 40, 256, False, False, False, 4),
    ("k896_n64", 1, 64, 896, True, False, False, 5),
    ("add_k192", 2, 33, 192, True, True, False, 6),
    ("add_inplace_k320", 3, 24, 320, False, True, True, 7),
    ("add_inplace_bias_k96", 5, 16, 96, True, True, True, 8),
]


def main():
    if not O.available("reference"):
        sys.exit("oracle/_ref/libvvllm_ref.so is missing: run `make -C oracle ref` where the reference tree is")
    out = {}
    for name, w in QUANT_CASES.items():
        q, s = O.quantize_per_channel(w, kind="reference")
        out[f"q_{name}_w"], out[f"q_{name}_codes"], out[f"q_{name}_scales"] = w, q, s
    np.savez(os.path.join(HERE, "quantize_ref.npz"), **out)

    out = {}
    # backend_naive_test.cc:407-425 (LinearQ8WithBias)
    wq = np.array([[127, 0], [0, 127]], np.int8)
    sc = np.array([1.0 / 127.0] * 2, np.float32)
    bi = np.array([10.0, 20.0], np.float32)
    x = np.array([[3.0, 5.0]], np.float32)
    out.update(l_withbias_x=x, l_withbias_q=wq, l_withbias_scales=sc, l_withbias_bias=bi,
               l_withbias_out=O.linear_q8(x, wq, sc, bi, kind="reference"))
    # backend_naive_test.cc:355-405 (LinearQ8MatchesFp32): codes from the
    # reference quantizer of the same matrix, input 1..4
    q, s = O.quantize_per_channel(QUANT_CASES["roundtrip"], kind="reference")
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    out.update(l_matches_x=x, l_matches_q=q, l_matches_scales=s,
               l_matches_out=O.linear_q8(x, q, s, kind="reference"))
    for name, M, N, K, has_b, has_r, inplace, seed in LINEAR_CASES:
        rng = np.random.default_rng(seed)
        w = rng.normal(0.0, 0.02, (N, K)).astype(np.float32)
        q, s = O.quantize_per_channel(w, kind="reference")
        x = rng.normal(0.0, 1.0, (M, K)).astype(np.float32)
        b = rng.normal(0.0, 0.01, N).astype(np.float32) if has_b else None
        r = rng.normal(0.0, 1.0, (M, N)).astype(np.float32) if has_r else None
        y = O.linear_q8(x, q, s, b, r, kind="reference", inplace=inplace)
        p = f"l_{name}_"
        out[p + "x"], out[p + "q"], out[p + "scales"], out[p + "out"] = x, q, s, y
        if b is not None:
            out[p + "bias"] = b
        if r is not None:
            out[p + "residual"] = r
        out[p + "meta"] = np.array([M, N, K, int(inplace)], np.int64)
    np.savez(os.path.join(HERE, "linear_ref.npz"), **out)
    print("wrote", os.path.join(HERE, "quantize_ref.npz"), os.path.join(HERE, "linear_ref.npz"))


if __name__ == "__main__":
    main()
