"""GPU parity of the device sampler vvh_sample (the reference's cuda_sample,
src/backend/cuda_kernels.cu:1228-1349, behind SamplerCUDA::sample,
src/sampler/sampler_cuda.cc:13-18) against the CPU oracle's restatement
(oracle/oracle.c orc_sample, pinned in tests/test_oracle_sample.py).

* Temperature 0 gives the first index of the maximum, exactly.
* Temperature > 0 gives the oracle's index wherever the two largest noisy
  values are not within 1e-5 of each other (device and host log() may differ
  in the last bit, which can only matter at a near-tie).
* One-hot logits always give their index; temperature -> 0 gives the argmax.
* Over many steps the sampled frequencies follow softmax(logit / T)
  (chi-square), on the device as on the host.
"""
import numpy as np
import pytest
from scipy import stats

from vvllm_amd import capi

pytestmark = pytest.mark.gpu

F16, F32 = capi.F16, capi.F32


def sample(dx, dtype, n, T, seed, step, di, slot=0):
    capi.call("vvh_sample", dx.ptr, dtype, n, T, 0.9, seed, step, di.ptr + 4 * slot, None)


def test_sample_matches_oracle(gpu, oracle):
    rng = np.random.default_rng(11)
    di = capi.DevBuf(4)
    checked = 0
    # one block, a one-element second block, many blocks, > 1024 blocks' worth
    for n in (1, 7, 2048, 2049, 151936, 3_000_001):
        for trial in range(3 if n < 1_000_000 else 1):
            x = (rng.standard_normal(n) * 3).astype(np.float32)
            for T, seed, step in ((0.7, 1234, trial), (1.0, 2**63 + 17, 5 + trial), (0.05, 7, 1000 + trial)):
                dx = capi.DevBuf.from_array(x)
                sample(dx, F32, n, T, seed, step, di)
                capi.sync()
                got = int(di.to_array(np.int32, (1,))[0])
                want, best, second = oracle.sample(x, T, seed, step)
                if best - second <= 1e-5 * max(1.0, abs(best)):
                    continue
                assert got == want, (n, T, seed, step)
                checked += 1
    assert checked >= 40


def test_sample_fp16_logits(gpu, oracle):
    rng = np.random.default_rng(12)
    di = capi.DevBuf(4)
    for n in (33, 5000, 151936):
        x16 = (rng.standard_normal(n) * 4).astype(np.float16)
        dx = capi.DevBuf.from_array(x16)
        for step in range(4):
            sample(dx, F16, n, 0.8, 99, step, di)
            capi.sync()
            want, best, second = oracle.sample(x16.astype(np.float32), 0.8, 99, step)
            if best - second > 1e-5 * max(1.0, abs(best)):
                assert int(di.to_array(np.int32, (1,))[0]) == want
        sample(dx, F16, n, 0.0, 99, 0, di)
        capi.sync()
        assert int(di.to_array(np.int32, (1,))[0]) == int(np.argmax(x16))


def test_temperature_zero_and_limit(gpu):
    rng = np.random.default_rng(13)
    di = capi.DevBuf(4)
    for n in (1000, 151936):
        x = rng.standard_normal(n).astype(np.float32)
        x[[5, n - 3]] = 9.0  # tie: the first index, as std::max_element
        dx = capi.DevBuf.from_array(x)
        sample(dx, F32, n, 0.0, 1, 0, di)
        capi.sync()
        assert int(di.to_array(np.int32, (1,))[0]) == 5
        x[5] = 8.9  # a gap of 0.1 / 1e-6 in the scaled logits swamps any Gumbel noise
        dx = capi.DevBuf.from_array(x)
        for step in range(5):
            sample(dx, F32, n, 1e-6, 3, step, di)
            capi.sync()
            assert int(di.to_array(np.int32, (1,))[0]) == n - 3


def test_one_hot_and_degenerate(gpu):
    di = capi.DevBuf(4 * 64)
    for n, hot in ((9, 6), (4096, 4095), (151936, 70000)):
        x = np.full(n, -np.inf, np.float32)
        x[hot] = 0.0
        dx = capi.DevBuf.from_array(x)
        for s in range(64):
            sample(dx, F32, n, (0.01, 0.7, 3.0)[s % 3], 5, s, di, slot=s)
        capi.sync()
        assert np.all(di.to_array(np.int32, (64,)) == hot)
        # no candidate above -1e30: index 0, as the reference's starting value
        dx = capi.DevBuf.from_array(np.full(n, -np.inf, np.float32))
        sample(dx, F32, n, 1.0, 5, 0, di)
        capi.sync()
        assert int(di.to_array(np.int32, (1,))[0]) == 0


def test_sampled_distribution_chi_square(gpu):
    logits = np.array([1.0, 0.2, -0.5, 2.0, 0.0, 1.5, -1.0, 0.7], np.float32)
    T, steps = 0.8, 20000
    dx = capi.DevBuf.from_array(logits)
    di = capi.DevBuf(4 * steps)
    for s in range(steps):
        sample(dx, F32, logits.size, T, 4242, s, di, slot=s)
    capi.sync()
    idx = di.to_array(np.int32, (steps,))
    z = logits.astype(np.float64) / T
    p = np.exp(z - z.max())
    p /= p.sum()
    obs = np.bincount(idx, minlength=logits.size).astype(np.float64)
    assert stats.chisquare(obs, p * steps).pvalue > 1e-3
