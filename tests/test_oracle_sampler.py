"""CPU checks of the sampler oracle: the C restatement of Sampler::sample
(crates/inferi/src/models/sampler.rs:32-131, f32 running sums) and the
exact-sum model the device sampler implements.

The reference has no sampler tests and no golden vectors for it, so the
restatement is pinned by answers worked by hand from the reference's text,
closed forms (uniform and one-hot distributions), brute force over dyadic
inputs on which f32 sums are exact (there both versions must agree on every
case), and a published splitmix64 vector for the device coin.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from tests.sampling import robust_mult, robust_topp


def test_softmax_closed_forms():
    # equal logits: exp(0) = 1 each, sum n exact, 1/n correctly rounded
    for n in (1, 3, 7, 1000):
        p = O.softmax(np.full(n, 2.5, np.float32))
        assert np.all(p == np.float32(1.0) / np.float32(n))
    # one dominant logit: the rest underflow to 0
    v = np.zeros(5, np.float32)
    v[3] = 200.0
    p = O.softmax(v)
    assert p[3] == 1.0 and np.all(np.delete(p, 3) == 0.0)
    # against an f64 softmax
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(4096) * 3).astype(np.float32)
    e = np.exp(x.astype(np.float64) - x.max())
    ref = e / e.sum()
    # the f32 left-to-right sum of 4096 terms drifts by ~1e-6 relative
    assert np.allclose(O.softmax(x), ref, rtol=2e-5, atol=1e-12)


def test_sample_mult_known_answers():
    q = np.full(4, 0.25, np.float32)
    assert [O.sample_mult(q, c) for c in (0.0, 0.1, 0.26, 0.6, 0.99)] == [0, 0, 1, 2, 3]
    # the coin lands exactly on a boundary: coin < cdf is strict
    assert O.sample_mult(q, 0.25) == 1 and O.sample_mult(q, 0.5) == 2
    # the running sum never exceeds the coin: the last index (sampler.rs:75)
    assert O.sample_mult(np.array([0.1, 0.1], np.float32), 0.5) == 1
    one = np.zeros(9, np.float32)
    one[6] = 1.0
    assert all(O.sample_mult(one, c) == 6 for c in (0.0, 0.5, 0.999))


def test_sample_topp_known_answers():
    # worked from sampler.rs:83-131: cutoff (1-0.7)/3 = 0.1 keeps all four;
    # sorted 0.5(1) 0.25(3) 0.15(2) 0.1(0); running 0.5, 0.75 > 0.7 -> last
    # position 1, cumulative 0.75; r = coin * 0.75
    p = np.array([0.1, 0.5, 0.15, 0.25], np.float32)
    assert O.sample_topp(p, 0.7, 0.5) == (1, 1, 0.75)  # r 0.375 < 0.5
    assert O.sample_topp(p, 0.7, 0.9)[0] == 3           # r 0.675 in [0.5, 0.75)
    # ties keep index order (stable sort): 0, 1, 2 kept (0.75 > 0.6)
    q = np.full(4, 0.25, np.float32)
    assert O.sample_topp(q, 0.6, 0.99) == (2, 2, 0.75)
    assert O.sample_topp(q, 0.6, 0.5)[0] == 1
    assert O.sample_topp(q, 0.6, 0.0)[0] == 0
    # the cutoff (1-0.5)/3 = 0.1667 drops 0.05s; 0.6 alone exceeds 0.5
    c = np.array([0.05, 0.3, 0.6, 0.05], np.float32)
    assert all(O.sample_topp(c, 0.5, k)[0] == 2 for k in (0.0, 0.5, 0.999))
    # no running sum exceeds topp (0.999 > 0.5 + 0.25 + 0.125): all kept
    d = np.array([0.125, 0.5, 0.25], np.float32)
    assert O.sample_topp(d, 0.999, 0.99) == (0, 2, 0.875)
    # nothing reaches the cutoff: the reference has nothing to sort
    assert O.sample_topp(np.full(4, 0.25, np.float32), 0.1, 0.5)[0] == -1


def test_exact_model_known_answers():
    p = np.array([0.1, 0.5, 0.15, 0.25], np.float32)
    assert O.sample_topp_exact(p, 0.7, 0.5, -1) == 1 and O.sample_topp_exact(p, 0.7, 0.9, -1) == 3
    q = np.full(4, 0.25, np.float32)
    assert [O.sample_mult_exact(q, c) for c in (0.0, 0.1, 0.25, 0.26, 0.5, 0.99)] == [0, 0, 1, 1, 2, 3]
    assert O.sample_topp_exact(q, 0.6, 0.99, -1) == 2
    assert O.sample_topp_exact(np.full(4, 0.25, np.float32), 0.1, 0.5, 7) == 7
    assert O.sample_mult_exact(np.array([0.1, 0.1], np.float32), 0.5) == 1


@pytest.mark.parametrize("n", [2, 5, 16, 64])
def test_exact_model_matches_restatement_on_dyadic_inputs(n):
    """Probabilities, coins and topp on the 2^-12 grid: every f32 sum and the
    product coin * cum are exact, so the reference's f32 algorithm and the
    exact-sum model must choose the same element in every case."""
    rng = np.random.default_rng(n)
    for case in range(300):
        w = rng.integers(0, 6, n).astype(np.int64)
        if case % 3 == 0:  # many ties
            w = rng.integers(1, 3, n).astype(np.int64)
        w[rng.integers(0, n)] += 1
        # scale the weights onto the 2^-12 grid, summing to at most 1
        scale = 4096 // int(w.sum())
        p = (w * scale).astype(np.float32) / np.float32(4096)
        topp = np.float32(rng.integers(1, 4096) / 4096)
        coin = np.float32(rng.integers(0, 4096) / 4096)
        assert O.sample_mult(p, coin) == O.sample_mult_exact(p, coin)
        ref = O.sample_topp(p, topp, coin)[0]
        got = O.sample_topp_exact(p, topp, coin, -1)
        assert ref == got, (case, p, topp, coin)


@pytest.mark.parametrize("n", [8, 64, 1024])
def test_uniform_closed_forms(n):
    """p = 1/n (n a power of two, exact): sample_mult picks floor(coin * n);
    top-p keeps floor(topp * n) + 1 elements in index order and picks
    floor(coin * (that count))."""
    p = np.full(n, 1.0 / n, np.float32)
    rng = np.random.default_rng(1)
    for _ in range(50):
        coin = np.float32(rng.random())
        assert O.sample_mult(p, coin) == O.sample_mult_exact(p, coin) == int(np.floor(np.float64(coin) * n))
        topp = np.float32(rng.uniform(0.01, 0.99))
        if abs(topp * n - round(topp * n)) < 1e-3:
            continue
        if topp * n < 1:  # 1/n < cutoff (1 - topp)/(n - 1): no candidate
            assert O.sample_topp(p, topp, coin)[0] == -1
            assert O.sample_topp_exact(p, topp, coin, -1) == -1
            continue
        kept = int(np.floor(np.float64(topp) * n)) + 1
        want = int(np.floor(np.float64(coin) * kept))
        if abs(np.float64(coin) * kept - round(np.float64(coin) * kept)) < 1e-4:
            continue
        assert O.sample_topp(p, topp, coin)[0] == want
        assert O.sample_topp_exact(p, topp, coin, -1) == want


@pytest.mark.parametrize("n,sigma", [(1000, 4.0), (32000, 6.0)])
def test_exact_model_matches_restatement_on_logits(n, sigma):
    """Softmax outputs of random logits: both versions agree wherever the
    coin and topp are further from a boundary than the f32 drift."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * sigma).astype(np.float32)
    checked = 0
    for t in (0.7, 1.0):
        for topp in (0.0, 0.5, 0.9, 0.95):
            for coin in rng.random(16).astype(np.float32):
                ref, p = O.sample(x, t, topp, coin)
                if topp == 0.0:
                    if robust_mult(p, coin):
                        assert ref == O.sample_mult_exact(p, coin)
                        checked += 1
                elif robust_topp(p, topp, coin):
                    assert ref == O.sample_topp_exact(p, topp, coin, -1)
                    checked += 1
    assert checked >= 64


def test_temperature_zero_is_argmax():
    x = np.array([0.5, 3.0, -1.0, 3.0], np.float32)
    idx, v = O.sample(x, 0.0, 0.95, 0.3)
    assert idx == 1 and np.array_equal(v, x)


def test_seeded_coin_splitmix64_vector():
    """splitmix64 seeded with 0 first returns 0xE220A8397B1DCDAF (Vigna's
    reference generator); the coin keeps its top 24 bits."""
    assert O.seeded_coin(0, 1) == np.float32(0xE220A8 / 16777216.0)
    coins = [O.seeded_coin(12345, p) for p in range(1000)]
    assert all(0.0 <= c < 1.0 for c in coins)
    assert abs(np.mean(coins) - 0.5) < 0.05
