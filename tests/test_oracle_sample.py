"""Pins the oracle's restatement of the device sampler before it judges the GPU.

The reference samples on the device with the Gumbel-max trick
(src/backend/cuda_kernels.cu:1228-1317, cuda_sample :1322-1349, called by
SamplerCUDA::sample, src/sampler/sampler_cuda.cc:13-18).  That file needs
nvcc and cannot be built here, so the restatement (oracle/oracle.c,
orc_sample*) is pinned by what the mathematics and published algorithms fix:

* the hash is the splitmix64 finaliser applied to seed ^ (step * golden
  gamma + idx * c): with seed 0 and idx 0, step s gives splitmix64's s-th
  published output for seed 0;
* the uniforms are uniform (Kolmogorov-Smirnov over indices);
* temperature 0 is std::max_element (sampler.cc:21-25);
* argmax(logit / T + Gumbel) is a draw of softmax(logit / T): a chi-square
  test over many steps accepts the oracle and rejects the same sampler with
  the sign of the Gumbel term flipped (a planted mistake).
"""
import math

import numpy as np
import pytest
from scipy import stats

# splitmix64 outputs 1..3 for seed 0 (Steele, Lea, Flood, "Fast splittable
# pseudorandom number generators", OOPSLA 2014; the generator behind Java's
# SplittableRandom)
SPLITMIX64_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_hash_is_splitmix64(oracle):
    for s, want in enumerate(SPLITMIX64_SEED0, start=1):
        assert oracle.sample_hash(0, s, 0) == want
    # the seed enters by xor before mixing: seed g with step 0 is step 1 with seed 0
    assert oracle.sample_hash(0x9E3779B97F4A7C15, 0, 0) == SPLITMIX64_SEED0[0]


def test_hash_index_term_mixes(oracle):
    # one flipped index bit changes about half of the 64 output bits
    rng = np.random.default_rng(5)
    flips = []
    for _ in range(400):
        i = int(rng.integers(0, 1 << 30))
        b = int(rng.integers(0, 30))
        h0 = oracle.sample_hash(12345, 7, i)
        h1 = oracle.sample_hash(12345, 7, i ^ (1 << b))
        flips.append(bin(h0 ^ h1).count("1"))
    assert 28 < np.mean(flips) < 36
    # negative steps take the two's-complement multiple, as the int -> unsigned
    # long long conversion in the reference
    assert oracle.sample_hash(0, -1, 0) != oracle.sample_hash(0, 1, 0)


def test_uniform_scaling_and_distribution(oracle):
    for seed, step, idx in [(0, 1, 0), (42, 3, 17), (2**63 + 5, 1000, 151935)]:
        h = oracle.sample_hash(seed, step, idx)
        want = np.float32(np.float32(h >> 11) * np.float32(2.0 ** -53)) + np.float32(1e-10)
        assert np.float32(oracle.sample_uniform(seed, step, idx)) == want
    u = np.array([oracle.sample_uniform(99, 4, i) for i in range(20000)])
    assert u.min() > 0.0 and u.max() <= 1.0
    assert stats.kstest(u, "uniform").pvalue > 1e-3
    u2 = np.array([oracle.sample_uniform(99, s, 3) for s in range(20000)])
    assert stats.kstest(u2, "uniform").pvalue > 1e-3


def test_temperature_zero_is_max_element(oracle):
    x = np.array([1.0, 3.0, -2.0, 3.0, 2.5], np.float32)
    assert oracle.sample(x, 0.0, 1, 0)[0] == 1  # first of the tied maxima
    rng = np.random.default_rng(0)
    for _ in range(20):
        x = rng.standard_normal(1000).astype(np.float32)
        assert oracle.sample(x, 0.0, 3, 9)[0] == int(np.argmax(x))


def test_dominant_and_one_hot_logits(oracle):
    x = np.zeros(7, np.float32)
    x[4] = 60.0  # every other index has probability below e^-58 at T = 1
    assert all(oracle.sample(x, 1.0, 11, s)[0] == 4 for s in range(500))
    oh = np.full(9, -np.inf, np.float32)
    oh[6] = 0.0
    for t in (1e-3, 0.7, 1.0, 5.0):
        assert all(oracle.sample(oh, t, 3, s)[0] == 6 for s in range(200))
    # no candidate above -1e30: the reference's start, index 0
    assert oracle.sample(np.full(5, -np.inf, np.float32), 1.0, 3, 0)[0] == 0


def gumbel_draws(oracle, logits, T, seed, steps, sign=-1.0):
    """Index per step of argmax(logit / T + g) with g = sign * log(-log(u)) over
    the oracle's uniforms (sign -1 is the Gumbel noise; +1 a planted mistake)."""
    n = len(logits)
    out = np.empty(steps, np.int64)
    for s in range(steps):
        u = np.array([oracle.sample_uniform(seed, s, i) for i in range(n)], np.float64)
        out[s] = int(np.argmax(np.asarray(logits, np.float64) / T + sign * np.log(-np.log(u))))
    return out


def softmax(x, T):
    z = np.asarray(x, np.float64) / T
    e = np.exp(z - z.max())
    return e / e.sum()


def chi2_p(idx, p):
    obs = np.bincount(idx, minlength=len(p)).astype(np.float64)
    return stats.chisquare(obs, p * obs.sum()).pvalue


def test_sampled_frequencies_follow_softmax(oracle):
    logits = np.array([1.0, 0.2, -0.5, 2.0, 0.0, 1.5], np.float32)
    T, steps = 0.8, 12000
    idx = np.array([oracle.sample(logits, T, 2024, s)[0] for s in range(steps)])
    assert chi2_p(idx, softmax(logits, T)) > 1e-3
    # the same test on the same uniforms rejects a flipped Gumbel sign and a
    # temperature applied as a multiplication
    bad = gumbel_draws(oracle, logits, T, 2024, 3000, sign=+1.0)
    assert chi2_p(bad, softmax(logits, T)) < 1e-6
    bad_t = np.array([int(np.argmax(logits * T - np.log(-np.log(
        [oracle.sample_uniform(2024, s, i) for i in range(len(logits))])))) for s in range(3000)])
    assert chi2_p(bad_t, softmax(logits, T)) < 1e-6


def test_oracle_matches_float64_gumbel(oracle):
    # the oracle's fp32 arithmetic picks the same index as the float64 formula
    # on the same uniforms wherever the best two noisy values are apart
    rng = np.random.default_rng(1)
    agree = 0
    for s in range(300):
        x = rng.standard_normal(257).astype(np.float32) * 2
        i, best, second = oracle.sample(x, 0.9, 77, s)
        if best - second < 1e-4 * max(1.0, abs(best)):
            continue
        u = np.array([oracle.sample_uniform(77, s, j) for j in range(x.size)], np.float64)
        assert i == int(np.argmax(x.astype(np.float64) / np.float64(np.float32(0.9)) - np.log(-np.log(u))))
        agree += 1
    assert agree > 250
