"""GPU parity of the device sampler through the C ABI: ifr_sample
(Sampler::sample, crates/inferi/src/models/sampler.rs:32-131) and the
sampling decode step (ifr_llama2_set_sampler; sample_next_token,
crates/inferi-chat/src/sampler.rs:91-111).

Bars: the probabilities within 1e-5 relative of an f64 softmax of the same
f32 y = logits / T (the reference's own f32 sum drifts by about as much);
the chosen index identical to the exact-sum model of the reference's
algorithm on the device's probabilities (integer work: bit-exact), and
identical to the reference restatement itself whenever the coin and topp
lie further from a decision boundary than the two sides' measured
differences (twice the drift of the reference's f32 running sums plus the
relative difference of the probabilities).
"""

import numpy as np
import pytest

import inferi_amd as I
import oracle as O
from tests.sampling import rel_diff, robust_mult, robust_topp

pytestmark = pytest.mark.gpu

P_RTOL = 1e-5


def softmax64(x, t):
    y = (np.asarray(x, np.float32) / np.float32(t)).astype(np.float64)
    e = np.exp(y - y.max())
    return e / e.sum()


def first_argmax_y(x, t):
    y = np.asarray(x, np.float32) / np.float32(t)
    return int(np.argmax(y))


def run_sample(ctx, x, t, topp, coins, in_place=False):
    """ifr_sample once per coin; returns (indices, probabilities of the
    last call)."""
    n = x.size
    dl = ctx.upload(np.ascontiguousarray(x, np.float32))
    dp = dl if in_place else ctx.alloc(n * 4)
    dc = ctx.upload(np.asarray(coins, np.float32))
    di = ctx.zeros(4 * len(coins))
    for k in range(len(coins)):
        if in_place and k:
            dl.upload(np.ascontiguousarray(x, np.float32))
        ctx.sample(dl, dp, n, t, topp, dc.at(4 * k), di.at(4 * k))
    idx = di.download(np.uint32, len(coins)).astype(np.int64)
    p = dp.download(np.float32, n)
    for b in {dl, dp, dc, di}:
        b.free()
    return idx, p


def check_case(ctx, x, t, topp, coins, in_place=False):
    n = x.size
    print(f"sample n={n} T={t} topp={topp} coins={len(coins)} in_place={in_place}", flush=True)
    idx, p = run_sample(ctx, x, t, topp, coins, in_place)
    p64 = softmax64(x, t)
    err = np.abs(p.astype(np.float64) - p64) / np.maximum(p64, 1e-30)
    big = p64 > 1e-30
    assert err[big].max() <= P_RTOL, f"probabilities: max rel err {err[big].max():.2e}"
    mult = topp <= 0.0 or topp >= 1.0
    robust = 0
    for k, c in enumerate(coins):
        exact = O.sample_mult_exact(p, c) if mult else O.sample_topp_exact(p, topp, c, first_argmax_y(x, t))
        assert idx[k] == exact, f"coin {c}: device {idx[k]} exact model {exact}"
        ref, pref = O.sample(x, t, topp, c)
        rel = rel_diff(pref, p)
        ok = robust_mult(pref, c, rel) if mult else robust_topp(pref, topp, c, rel)
        if ref >= 0 and ok:
            assert idx[k] == ref, f"coin {c}: device {idx[k]} reference {ref}"
            robust += 1
    return robust


COINS = [0.0, 0.05, 0.3, 0.5, 0.77, 0.9, 0.999, float(np.nextafter(np.float32(1), np.float32(0)))]


@pytest.mark.parametrize("n", [32000, 128256])
@pytest.mark.parametrize("t", [0.7, 1.0])
@pytest.mark.parametrize("topp", [0.95, 0.5, 0.0, 1.0])
def test_sample_vocab_sizes(ctx, oracle_lib, n, t, topp):
    rng = np.random.default_rng(n + int(t * 10) + int(topp * 100))
    x = (rng.standard_normal(n) * 4).astype(np.float32)
    check_case(ctx, x, t, topp, COINS)


@pytest.mark.parametrize("n", [1, 2, 3, 255, 257, 1001, 4099])
def test_sample_small_and_ragged(ctx, oracle_lib, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 2).astype(np.float32)
    for topp in (0.9, 0.0):
        check_case(ctx, x, 0.8, topp, COINS)


def test_sample_flat_distribution_ties(ctx, oracle_lib):
    """Equal logits: every probability ties, so top-p keeps index order
    (the reference's stable sort) and the selection runs the tie pass."""
    for n in (1000, 262144):
        x = np.full(n, 0.25, np.float32)
        for topp in (0.95, 0.5, 0.0):
            check_case(ctx, x, 0.7, topp, COINS)
    # two tie classes
    x = np.zeros(50000, np.float32)
    x[::3] = 1.0
    check_case(ctx, x, 1.0, 0.9, COINS)


def test_sample_peaked_and_sharp(ctx, oracle_lib):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(32000) * 1.5).astype(np.float32)
    x[1234] = 40.0  # nearly one-hot
    check_case(ctx, x, 0.7, 0.95, COINS)
    x[99] = 40.0  # two equal winners
    check_case(ctx, x, 0.7, 0.95, COINS)
    check_case(ctx, x, 0.7, 0.0, COINS)


def test_sample_topp_edges(ctx, oracle_lib):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(32000) * 3).astype(np.float32)
    for topp in (1e-6, 0.999999, 0.9999999):
        check_case(ctx, x, 1.0, topp, COINS)
    # no candidate reaches the cutoff: the most probable token
    flat = np.full(1001, 1.0, np.float32)
    idx, _ = run_sample(ctx, flat, 1.0, 0.0005, [0.5])
    assert idx[0] == 0


def test_sample_negative_temperature_and_in_place(ctx, oracle_lib):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(5000) * 3).astype(np.float32)
    check_case(ctx, x, -1.3, 0.9, COINS)
    check_case(ctx, x, 0.7, 0.95, COINS, in_place=True)


def test_sample_agrees_with_reference_often(ctx, oracle_lib):
    """Realistically peaked logits: the device index equals the reference
    restatement's on every robust coin, and most coins are robust."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32000) * 6).astype(np.float32)
    coins = rng.random(64).astype(np.float32)
    assert check_case(ctx, x, 0.7, 0.95, coins) >= 48


def test_sample_temperature_zero_is_argmax(ctx, oracle_lib):
    x = np.array([0.5, 3.0, -1.0, 3.0] * 100, np.float32)
    idx, _ = run_sample(ctx, x, 0.0, 0.95, [0.5])
    assert idx[0] == 1


def test_sample_rejects_bad_arguments(ctx):
    d = ctx.alloc(4 * 300000)
    c = ctx.upload(np.array([0.5], np.float32))
    o = ctx.alloc(4)
    with pytest.raises(I.HipError):
        ctx.sample(d, d, 16, float("nan"), 0.9, c, o)
    with pytest.raises(I.HipError):
        ctx.sample(d, d, 16, 0.7, float("nan"), c, o)
    with pytest.raises(I.HipError):
        ctx.sample(d, d, 262145, 0.7, 0.9, c, o)
    with pytest.raises(I.HipError):
        ctx.sample(d.at(4), d.at(4), 16, 0.7, 0.9, c, o)
    with pytest.raises(I.HipError):
        ctx.sample(d, d, 16, 0.7, 0.9, None, o)
    with pytest.raises(I.HipError):
        ctx.sample(d, d, 0, 0.7, 0.9, c, o)
    for b in (d, c, o):
        b.free()


# ------------------------------------------------------- decode step --

def tiny_model(ctx, vocab=512):
    cfg = I.Llama2Config(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, vocab=vocab, max_pos=24,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=3, mat_dtype=I.Q4_K, head_dtype=I.Q6_K, embd_dtype=I.Q4_K)
    return cfg, w


def test_decode_step_samples(ctx, oracle_lib):
    """Each sampled step: probabilities = softmax(logits / T) of the step's
    own logits, and the stored token = the exact model's choice with the
    coin of (seed, p + 1); forced positions are not sampled."""
    cfg, w = tiny_model(ctx)
    s = I.Llama2State(ctx, cfg)
    try:
        t, topp, seed = 0.7, 0.95, 77
        s.set_sampler(t, topp, seed)
        prompt = [5, 9, 11]
        s.reset(prompt, 0)
        for p in range(10):
            print(f"sampled step pos={p}", flush=True)
            I.Llama2.launch(ctx, s, w)
            logits, probs = s.read("logits"), s.read("probs")
            nxt = int(s.tokens(p + 1, 1)[0])
            if p + 1 < len(prompt):
                assert nxt == prompt[p + 1]
                assert not probs.any(), "a forced position was sampled"
                continue
            p64 = softmax64(logits, t)
            big = p64 > 1e-30
            assert (np.abs(probs - p64) / np.maximum(p64, 1e-30))[big].max() <= P_RTOL
            coin = O.seeded_coin(seed, p + 1)
            assert nxt == O.sample_topp_exact(probs, topp, coin, first_argmax_y(logits, t)), p
    finally:
        s.close()
        w.close()


def test_decode_sampler_graph_and_switch(ctx, oracle_lib):
    """The captured step follows the sampler: graph and step-by-step runs
    give the same tokens for the same seed, a new seed changes them, and
    temperature 0 returns to greedy decoding (recaptured each time)."""
    cfg, w = tiny_model(ctx)
    s = I.Llama2State(ctx, cfg)
    try:
        def run(graph, n=16):
            s.reset([5], 0)
            if graph:
                I.Llama2.generate(ctx, s, w, n, use_graph=True)
            else:
                for _ in range(n):
                    I.Llama2.launch(ctx, s, w)
            return s.tokens(0, n + 1)

        greedy = run(True)
        s.set_sampler(1.0, 0.0, 1)
        a_graph, a_eager = run(True), run(False)
        assert np.array_equal(a_graph, a_eager)
        s.set_sampler(1.0, 0.0, 2)
        b = run(True)
        assert not np.array_equal(a_graph, b)
        s.set_sampler(0.0, 0.0, 0)
        assert np.array_equal(run(True), greedy)
        assert np.array_equal(run(False), greedy)
    finally:
        s.close()
        w.close()


def test_set_sampler_rejects(ctx):
    cfg, w = tiny_model(ctx, vocab=262145)
    s = I.Llama2State(ctx, cfg)
    try:
        with pytest.raises(I.HipError):
            s.set_sampler(0.7, 0.95, 0)
        s.set_sampler(0.0, 0.95, 0)  # argmax has no vocabulary limit
        with pytest.raises(I.HipError):
            s.set_sampler(float("inf"), 0.9, 0)
    finally:
        s.close()
        w.close()
